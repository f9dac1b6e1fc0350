"""GPU: the reference's edge cases on the device path.

* sampler (sampler.rs:24-109, its tests at 116-162): ties go to the lowest
  index, NaN is skipped, all -inf (or all NaN) gives 0, a degenerate T > 0
  distribution falls back to argmax, overflowing logits -- run through the
  device sampler on exact logit vectors (defer_gpu_cache_set_logits);
* the sums a sample leaves never leak into a later sample at another
  temperature (one tag per sampling event);
* range errors (model.rs:417-422) leave the cache untouched through forward,
  forward_batch and replay; a prompt feeds the tokens before the first bad
  one (engine.rs:62-71);
* GeLU and q/k/v biases against the oracle;
* attribution invariants (tests/attribution.rs:35-46, 97-129): a traced
  forward perturbs nothing, an empty mask is the plain forward, and clone +
  truncate + masked forwards (attribution.rs:254-258) equal a full masked
  recompute, bit for bit.
"""
import numpy as np
import pytest

import oracle_py as O
from defer_amd import gpu as G
from defer_amd import host as H
from defer_amd import synthetic

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
NEG = -np.inf


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def tiny():
    cfg = synthetic.CONFIGS["tiny"]
    w = synthetic.make_weights(cfg, 21)
    return cfg, w, G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)


def padded(vals, V, fill=NEG):
    a = np.full(V, fill, dtype=np.float32)
    a[: len(vals)] = np.asarray(vals, dtype=np.float32)
    return a


# ------------------------------------------------------------------ sampler

def test_sampler_edge_cases_on_device(tiny):
    cfg, w, gm, om = tiny
    V = cfg["vocab_size"]
    c = gm.new_cache(64)
    gm.forward(3, c, logits=False)
    nan = np.float32("nan")
    cases = [
        # sampler.rs:116-121
        (padded([1.0, 3.0, 3.0, 2.0], V), 0.0, 1),
        (padded([nan, 0.0, 0.0], V), 0.0, 1),
        (np.full(V, NEG, np.float32), 0.0, 0),
        (np.full(V, nan, np.float32), 0.0, 0),
        # ties across vocabulary chunks, NaN inside the winning chunk
        (padded([0.0] * 70 + [5.0] + [0.0] * 129 + [5.0], V, 0.0), 0.0, 70),
        (padded([0.0] * 64 + [nan, 7.0, nan, 7.0], V, 0.0), 0.0, 65),
        # degenerate T > 0 (sampler.rs:60-69): all -inf, all NaN, +inf overflow
        (np.full(V, NEG, np.float32), 0.7, 0),
        (np.full(V, nan, np.float32), 0.7, 0),
        (padded([1.0, 2.0, 3.0, 4.0, 5.0, np.inf, 6.0], V), 0.7, 5),
        (padded([np.inf, 1.0, np.inf], V), 1.3, 0),
    ]
    for k, (lg, T, want) in enumerate(cases):
        for word in (0, 0x9E3779B9, 0xFFFFFFFF):
            c.set_logits(lg)
            got = gm.sample(c, T, word)
            ref = O.sample_token(lg, T, word)
            assert got == ref == want, (k, T, word, got, ref, want)
    say("sampler: fixed edge cases equal the reference's answers")
    # sampler.rs:133-145's cases at T = 0.7 against the oracle, many draws
    rng = np.random.Generator(np.random.PCG64(8))
    for vals in ([0.0, 1.0, 2.0], [NEG, NEG], [nan, 5.0], [1e30, -1e30, 1e30]):
        lg = padded(vals, V)
        for word in rng.integers(0, 2**32, size=40, dtype=np.uint64):
            c.set_logits(lg)
            assert gm.sample(c, 0.7, int(word)) == O.sample_token(lg, 0.7, int(word)), vals


def test_sampler_random_logits_against_oracle(tiny):
    """Random logits at several temperatures, including logits with ties,
    -inf and NaN entries: the device token equals the reference's on every
    draw, in every execution mode (persistent kernel, graph, eager)."""
    cfg, w, gm, om = tiny
    V = cfg["vocab_size"]
    rng = np.random.Generator(np.random.PCG64(17))
    for mode in (G.EXEC_PERSISTENT, G.EXEC_GRAPH, G.EXEC_EAGER):
        gm.set_exec(mode)
        c = gm.new_cache(64)
        gm.forward(5, c, logits=False)
        for T in (0.3, 0.7, 1.0, 2.5):
            for k in range(60):
                lg = (rng.standard_normal(V) * 3).astype(np.float32)
                if k % 4 == 1:
                    lg = np.round(lg)  # many exact ties
                if k % 4 == 2:
                    lg[rng.integers(0, V, 20)] = -np.inf
                if k % 4 == 3:
                    lg[rng.integers(0, V, 20)] = np.nan
                word = int(rng.integers(0, 2**32, dtype=np.uint64))
                c.set_logits(lg)
                got, ref = gm.sample(c, T, word), O.sample_token(lg, T, word)
                assert got == ref, (mode, T, k, word, got, ref)
        c.close()
    gm.set_exec(G.EXEC_PERSISTENT)
    say("sampler: 3 x 240 random draws identical to sample_token")


@pytest.mark.parametrize("mode", [G.EXEC_PERSISTENT, G.EXEC_GRAPH, G.EXEC_EAGER])
def test_sample_then_step_at_another_temperature(tiny, mode):
    """sample(T=0.7) leaves chunk sums in the cache's mailbox; a following
    step at T=1.5 must not read them: it equals the same step on a clone
    that never sampled."""
    cfg, w, gm, om = tiny
    gm.set_exec(mode)
    try:
        words = H.chacha8_words(H.seed_from_u64(31), 0, 40)
        c = gm.new_cache(128)
        gm.prompt(c, [7, 1, 8, 2, 8])
        for k in range(20):
            twin = c.clone()
            gm.sample(c, 0.7, int(words[2 * k]))
            a = gm.step(c, 1.5, int(words[2 * k + 1]))
            b = gm.step(twin, 1.5, int(words[2 * k + 1]))
            assert a == b, k
            assert np.array_equal(bits(c.last_logits()), bits(twin.last_logits())), k
            twin.close()
    finally:
        gm.set_exec(G.EXEC_PERSISTENT)


# ------------------------------------------------------------ range errors

def _snapshot(c, layers):
    return len(c), [tuple(bits(x).copy() for x in c.read(l)) for l in range(layers)]


def _same(a, b):
    assert a[0] == b[0]
    for x, y in zip(a[1], b[1]):
        for u, v in zip(x, y):
            assert np.array_equal(u, v)


def test_range_errors_leave_caches_untouched(tiny):
    cfg, w, gm, om = tiny
    V, L = cfg["vocab_size"], cfg["num_layers"]
    c = gm.new_cache(12)
    gm.prompt(c, [1, 2, 3, 4])
    before, lg = _snapshot(c, L), bits(c.last_logits()).copy()
    with pytest.raises(G.DeferGpuError) as e:
        gm.forward(V, c)
    assert e.value.code == G.E_TOKEN
    _same(before, _snapshot(c, L))
    assert np.array_equal(lg, bits(c.last_logits()))
    others = [gm.new_cache(12) for _ in range(3)]
    for o in others:
        gm.prompt(o, [5, 6])
    snaps = [_snapshot(o, L) for o in others]
    with pytest.raises(G.DeferGpuError) as e:
        gm.forward_batch(others + [c], [1, 2, 3, V + 7])
    assert e.value.code == G.E_TOKEN
    for o, s in zip(others, snaps):
        _same(s, _snapshot(o, L))
    _same(before, _snapshot(c, L))
    # context: 12 positions, 4 used; a batch of 9 rows for c overflows
    with pytest.raises(G.DeferGpuError) as e:
        gm.forward_batch([c] * 9, [1] * 9)
    assert e.value.code == G.E_CONTEXT
    _same(before, _snapshot(c, L))
    for n in range(8):
        gm.forward(9, c, logits=False)
    with pytest.raises(G.DeferGpuError) as e:
        gm.forward(9, c)
    assert e.value.code == G.E_CONTEXT
    assert len(c) == 12
    r = gm.new_cache(12)
    with pytest.raises(G.DeferGpuError) as e:
        gm.replay(r, [1, 2, V, 4], 2, 0.0)
    assert e.value.code == G.E_TOKEN
    assert len(r) == 0
    with pytest.raises(G.DeferGpuError) as e:
        gm.replay(r, list(range(13)), 13, 0.0)
    assert e.value.code == G.E_CONTEXT
    assert len(r) == 0


@pytest.mark.parametrize("batching", [0, 4])
def test_prompt_feeds_the_tokens_before_an_error(tiny, batching):
    """Session::prompt feeds token by token (engine.rs:62-71): what came
    before the failing token stays in the cache (and the session history),
    prompt_len does not move, and the cache equals feeding the prefix."""
    cfg, w, gm, om = tiny
    V, L = cfg["vocab_size"], cfg["num_layers"]
    gm.set_batching(batching)
    try:
        good = [int(x) for x in synthetic.make_prompt(V, 9, seed=2)]
        c = gm.new_cache(32)
        with pytest.raises(G.DeferGpuError) as e:
            gm.prompt(c, good[:6] + [V] + good[6:])
        assert e.value.code == G.E_TOKEN and len(c) == 6
        ref = gm.new_cache(32)
        gm.prompt(ref, good[:6])
        _same(_snapshot(ref, L), _snapshot(c, L))
        assert np.array_equal(bits(ref.last_logits()), bits(c.last_logits()))
        small = gm.new_cache(7)
        with pytest.raises(G.DeferGpuError) as e:
            gm.prompt(small, good)
        assert e.value.code == G.E_CONTEXT and len(small) == 7
        s = H.Session(gm, H.seed_from_u64(1), 0.0, capacity=32)
        with pytest.raises(H.DeferHostError):
            s.prompt(good[:4] + [V + 1])
        assert s.history == good[:4] and s.prompt_len == 0
        with pytest.raises(H.DeferHostError):
            s.prompt(good)  # generation is taken to have started (history != prompt_len)
        s.close()
    finally:
        gm.set_batching(16)


# ------------------------------------------------------- activation, biases

def test_gelu_and_qkv_bias_against_oracle():
    cfg = dict(synthetic.CONFIGS["tiny"])
    cfg["activation"] = 1
    cfg["has_bias"] = 1
    w = synthetic.make_weights(cfg, 6)
    gm, om = G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 30, seed=12)]
    gc, oc = gm.new_cache(128), om.new_cache()
    worst = 0.0
    for t in prompt:
        worst = max(worst, float(np.max(np.abs(gm.forward(t, gc) - om.forward(t, oc)))))
    say(f"tiny, GeLU + biases: max|dlogit| over 30 positions = {worst:.3e}")
    assert worst <= LOGIT_TOL
    toks = gm.generate(gc, 20, 0.0)
    otoks, _, _ = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 20)
    assert toks == otoks
    b = gm.new_cache(128)
    gm.prompt(b, prompt)  # batched
    assert gm.generate(b, 20, 0.0) == toks
    assert np.array_equal(bits(b.last_logits()), bits(gc.last_logits()))
    words = H.chacha8_words(H.seed_from_u64(4), 0, 20)
    x = gm.new_cache(128)
    gm.prompt(x, prompt)
    st, _, _ = om.generate(om.new_cache(), O.seed_from_u64(4), 0.9, prompt, 20)
    assert gm.generate(x, 20, 0.9, words) == st


# ------------------------------------------------------------- attribution

def test_tracing_does_not_perturb_generation(tiny):
    """tests/attribution.rs:35-46 on the device: 30 steps at T=0.8 with and
    without the attention trace give the same tokens, caches, logits and
    rng position, bit for bit."""
    cfg, w, gm, om = tiny
    L = cfg["num_layers"]
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 11, seed=5)]
    words = H.chacha8_words(H.seed_from_u64(5), 0, 30)
    a, b = gm.new_cache(64), gm.new_cache(64)
    gm.prompt(a, prompt)
    for t in prompt:
        gm.forward(t, b, logits=False, trace=True)
    ta = gm.generate(a, 30, 0.8, words)
    tb, used = [], 0
    for k in range(30):
        tok = gm.sample(b, 0.8, int(words[k]))
        used += 1
        gm.forward(tok, b, logits=False, trace=True)
        tb.append(tok)
    assert ta == tb and used == 30
    _same(_snapshot(a, L), _snapshot(b, L))
    assert np.array_equal(bits(a.last_logits()), bits(b.last_logits()))


def test_ablation_prefix_reuse_equals_full_masked_recompute(tiny):
    """tests/attribution.rs:97-129 with attribution.rs:254-258's prefix
    reuse: clone the full cache, truncate to p + 1, forward the rest with p
    masked -- bit-identical to recomputing everything with the mask, and
    deterministic; an empty mask is the plain forward; the masked logits
    agree with the oracle's."""
    cfg, w, gm, om = tiny
    ctx = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 14, seed=9)]
    full = gm.new_cache(64)
    plain = []
    for t in ctx:
        plain.append(gm.forward(t, full))
    e = gm.new_cache(64)
    for t, p in zip(ctx, plain):
        assert np.array_equal(bits(gm.forward(t, e, masked=[])), bits(p))
    changed = False
    for p in (0, len(ctx) // 2, len(ctx) - 2):
        runs = []
        for _ in range(2):
            c = full.clone()
            c.truncate(p + 1)
            lg = None
            for t in ctx[p + 1:]:
                lg = gm.forward(t, c, masked=[p])
            runs.append(lg)
            c.close()
        fresh = gm.new_cache(64)
        oc = om.new_cache()
        for t in ctx:
            lf = gm.forward(t, fresh, masked=[p])
            lo = om.forward(t, oc, masked=[p])
        assert np.array_equal(bits(runs[0]), bits(runs[1])), p
        assert np.array_equal(bits(runs[0]), bits(lf)), p
        assert float(np.max(np.abs(lf - lo))) <= LOGIT_TOL
        changed |= not np.array_equal(bits(lf), bits(plain[-1]))
        fresh.close()
    assert changed, "ablation should change something"
