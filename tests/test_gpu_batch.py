"""GPU: the batched path (MFMA GEMMs over rows) against the one-token path.

Every batched result must equal, bit for bit, what feeding the same tokens one
at a time produces: cache entries, logits, sampled tokens, replay verdicts.
The one-token path is itself checked against the oracle elsewhere; here the
oracle also checks greedy tokens of a batched prefill directly.
"""
import numpy as np
import pytest

import oracle_py as O
from defer_amd import gpu as G
from defer_amd import host as H
from defer_amd import synthetic

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same_cache(a, b, layers):
    assert len(a) == len(b)
    for l in range(layers):
        for x, y in zip(a.read(l), b.read(l)):
            assert np.array_equal(bits(x), bits(y)), f"layer {l}"


@pytest.fixture(scope="module")
def tiny():
    cfg = synthetic.CONFIGS["tiny"]
    w = synthetic.make_weights(cfg, 5)
    return cfg, G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)


@pytest.fixture(scope="module")
def m135():
    cfg = synthetic.CONFIGS["smollm2-135m"]
    w = synthetic.make_weights(cfg, 0)
    return cfg, G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)


def test_forward_batch_rows_equal_single_forwards(tiny):
    cfg, gm, om = tiny
    say("tiny: 5 caches at different lengths, one batched forward vs one-by-one")
    gm.set_batching(0)
    V = cfg["vocab_size"]
    prompts = [synthetic.make_prompt(V, n, seed=n) for n in (1, 3, 7, 12, 20)]
    A, B = [], []
    for p in prompts:
        a, b = gm.new_cache(64), gm.new_cache(64)
        gm.prompt(a, p)
        gm.prompt(b, p)
        A.append(a)
        B.append(b)
    toks = [7, 100, 3, 255, 42]
    lg = gm.forward_batch(A, toks, logits=True)
    for i, (b, t) in enumerate(zip(B, toks)):
        ref = gm.forward(t, b)
        assert np.array_equal(bits(lg[i]), bits(ref)), f"row {i}"
        assert np.array_equal(bits(A[i].last_logits()), bits(ref))
        same_cache(A[i], b, cfg["num_layers"])
    # a following step continues from each cache's batched logits
    for a, b in zip(A, B):
        assert gm.step(a, 0.0) == gm.step(b, 0.0)


def test_forward_batch_same_cache_consecutive_positions(tiny):
    cfg, gm, om = tiny
    say("tiny: one cache listed 9 times (a prefill) vs 9 forwards")
    gm.set_batching(0)
    a, b = gm.new_cache(64), gm.new_cache(64)
    gm.prompt(a, [1, 2])
    gm.prompt(b, [1, 2])
    toks = [5, 6, 7, 8, 9, 10, 11, 12, 13]
    lg = gm.forward_batch([a] * 9, toks, logits=True)
    for i, t in enumerate(toks):
        ref = gm.forward(t, b)
        assert np.array_equal(bits(lg[i]), bits(ref)), f"row {i}"
    same_cache(a, b, cfg["num_layers"])


def test_batched_prompt_and_replay_match_token_by_token(tiny):
    cfg, gm, om = tiny
    say("tiny: prompt 30 + 60 at T=0.8; batched vs token-by-token prompt and replay")
    V = cfg["vocab_size"]
    prompt = [int(x) for x in synthetic.make_prompt(V, 30, seed=4)]
    words = H.chacha8_words(H.seed_from_u64(11), 0, 60)
    gm.set_batching(0)
    live = gm.new_cache(128)
    gm.prompt(live, prompt)
    toks = gm.generate(live, 60, 0.8, words)
    hist = prompt + toks
    res = {}
    for mb in (0, 1):
        gm.set_batching(mb)
        c = gm.new_cache(128)
        gm.prompt(c, prompt)
        res[("prompt", mb)] = (c.last_logits(), c)
        r = gm.new_cache(128)
        fd, sd = gm.replay(r, hist, len(prompt), 0.8, words)
        assert fd == -1
        res[("replay", mb)] = (r.last_logits(), r)
        bad = list(hist)
        bad[45] = (bad[45] + 1) % V
        x = gm.new_cache(128)
        res[("div", mb)] = (gm.replay(x, bad, len(prompt), 0.8, words), len(x), x.last_logits())
    gm.set_batching(16)
    for kind in ("prompt", "replay"):
        la, ca = res[(kind, 0)]
        lb, cb = res[(kind, 1)]
        assert np.array_equal(bits(la), bits(lb)), kind
        same_cache(ca, cb, cfg["num_layers"])
    assert np.array_equal(bits(res[("replay", 1)][0]), bits(live.last_logits()))
    (fd0, sd0), n0, l0 = res[("div", 0)]
    (fd1, sd1), n1, l1 = res[("div", 1)]
    assert fd0 == fd1 == 45 and sd0 == sd1 == hist[45] and n0 == n1 == 45
    assert np.array_equal(bits(l0), bits(l1))


def test_step_batch_equals_individual_steps(tiny):
    cfg, gm, om = tiny
    say("tiny: 6 sessions x 10 lockstep steps at T=0.6 vs per-session steps")
    gm.set_batching(0)
    V = cfg["vocab_size"]
    A, B = [], []
    for k in range(6):
        p = synthetic.make_prompt(V, 4 + 3 * k, seed=30 + k)
        a, b = gm.new_cache(64), gm.new_cache(64)
        gm.prompt(a, p)
        gm.prompt(b, p)
        A.append(a)
        B.append(b)
    for step in range(10):
        words = [int(x) for x in H.chacha8_words(H.seed_from_u64(step), 0, 6)]
        got = gm.step_batch(A, 0.6, words)
        want = [gm.step(b, 0.6, w) for b, w in zip(B, words)]
        assert got == want, step
    for a, b in zip(A, B):
        assert np.array_equal(bits(a.last_logits()), bits(b.last_logits()))


def test_135m_batched_prefill_matches_and_oracle_tokens(m135):
    cfg, gm, om = m135
    say("135m: prompt 300 batched vs token by token (bitwise), then 4 greedy vs oracle")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 300, seed=21)
    gm.set_batching(0)
    a = gm.new_cache(512)
    gm.prompt(a, prompt)
    gm.set_batching(16)
    b = gm.new_cache(512)
    gm.prompt(b, prompt)
    assert np.array_equal(bits(a.last_logits()), bits(b.last_logits()))
    for l in (0, 14, 29):
        for x, y in zip(a.read(l), b.read(l)):
            assert np.array_equal(bits(x), bits(y))
    toks = gm.generate(b, 4, 0.0)
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 4)
    d = float(np.max(np.abs(b.last_logits() - olog)))
    say(f"135m batched prefill: max|dlogit| vs oracle after 4 greedy = {d:.3e}")
    assert toks == otoks
    assert d <= 1e-3


def test_135m_batched_replay_matches_sequential(m135):
    cfg, gm, om = m135
    say("135m: 64 prompt + 200 at T=0.7; replay batched vs token by token")
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 64, seed=9)]
    words = H.chacha8_words(H.seed_from_u64(7), 0, 200)
    gm.set_batching(0)
    live = gm.new_cache(512)
    gm.prompt(live, prompt)
    toks = gm.generate(live, 200, 0.7, words)
    hist = prompt + toks
    gm.set_batching(16)
    r = gm.new_cache(512)
    fd, _ = gm.replay(r, hist, 64, 0.7, words)
    assert fd == -1
    assert len(r) == len(hist)
    assert np.array_equal(bits(r.last_logits()), bits(live.last_logits()))
    for l in (0, 29):
        for x, y in zip(r.read(l), live.read(l)):
            assert np.array_equal(bits(x), bits(y))


def test_135m_batched_prefill_from_unaligned_position(m135):
    """A batched prompt continuing a cache at position 37: the first attention
    tile holds positions 37..47 only."""
    cfg, gm, om = m135
    say("135m: 37 tokens one by one, then 100 batched vs 137 one by one")
    p = synthetic.make_prompt(cfg["vocab_size"], 137, seed=33)
    gm.set_batching(0)
    a = gm.new_cache(256)
    gm.prompt(a, p)
    b = gm.new_cache(256)
    gm.prompt(b, p[:37])
    gm.set_batching(16)
    gm.prompt(b, p[37:])
    assert len(b) == 137
    assert np.array_equal(bits(a.last_logits()), bits(b.last_logits()))
    for l in (0, 17, 29):
        for x, y in zip(a.read(l), b.read(l)):
            assert np.array_equal(bits(x), bits(y))


def test_1b_shape_lockstep_sessions_bit_identical_and_oracle():
    """The many-session configuration's shape (Llama-3.2-1B: h 2048, 32/8
    heads, ff 8192, vocab 128256, tied), cut to 2 layers: 8 sessions stepped
    together equal their own batch-1 steps bit for bit, and session 0's
    greedy tokens equal the oracle's."""
    cfg = dict(synthetic.CONFIGS["llama-3.2-1b"])
    cfg["num_layers"] = 2
    say("1b shape x 2 layers: weights")
    w = synthetic.make_weights(cfg, 0)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    V = cfg["vocab_size"]
    lens = [12, 5, 17, 30, 9, 16, 22, 40]
    A, B = [], []
    for k, n in enumerate(lens):
        p = synthetic.make_prompt(V, n, seed=100 + k)
        a, b = gm.new_cache(128), gm.new_cache(128)
        gm.set_batching(16)
        gm.prompt(a, p)
        gm.set_batching(0)
        gm.prompt(b, p)
        assert np.array_equal(bits(a.last_logits()), bits(b.last_logits())), k
        A.append(a)
        B.append(b)
    say("1b shape: 4 lockstep greedy steps of 8 sessions vs per-session steps")
    steps = []
    for step in range(4):
        got = gm.step_batch(A, 0.0)
        want = [gm.step(b, 0.0) for b in B]
        assert got == want, step
        steps.append(got)
    for a, b in zip(A, B):
        assert np.array_equal(bits(a.last_logits()), bits(b.last_logits()))
    say("1b shape: session 0 vs the oracle (12 + 4 forwards on the CPU)")
    om = O.OracleModel(cfg, w)
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0,
                                 synthetic.make_prompt(V, 12, seed=100), 4)
    assert [s[0] for s in steps] == otoks
    d = float(np.max(np.abs(A[0].last_logits() - olog)))
    say(f"1b shape: max|dlogit| vs oracle = {d:.3e}")
    assert d <= 1e-3
