"""GPU parity of the forward pass and sampler against the CPU oracle.

Every call goes through libdefer_gpu.so's C ABI. Floating-point bar:
max |logit_gpu - logit_oracle| <= 1e-3 (observed maxima are printed);
integer bar: greedy tokens identical. Among GPU runs (persistent, graph,
eager, repeat runs, replays) every bit must match.
"""
import numpy as np
import pytest

import oracle_py as O
from defer_amd import gpu as G
from defer_amd import synthetic

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def say(msg):
    print(msg, flush=True)


def _models(name, seed):
    cfg = synthetic.CONFIGS[name]
    w = synthetic.make_weights(cfg, seed)
    return cfg, w, G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)


@pytest.fixture(scope="module")
def tiny():
    return _models("tiny", 1234)


@pytest.fixture(scope="module")
def small135():
    return _models("smollm2-135m", 0)


def words_for(seed_u64, n):
    s = O.seed_from_u64(seed_u64)
    return [O.chacha8_word(s, i) for i in range(n)]


def test_tiny_logits_match_oracle(tiny):
    cfg, w, gm, om = tiny
    say("tiny: 40-token prompt, per-token logits vs oracle")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 40, seed=7)
    gc, oc = gm.new_cache(), om.new_cache()
    worst = 0.0
    for t in prompt:
        lg = gm.forward(int(t), gc)
        lo = om.forward(int(t), oc)
        worst = max(worst, float(np.max(np.abs(lg - lo))))
    say(f"tiny max|dlogit| = {worst:.3e}")
    assert worst <= LOGIT_TOL
    assert len(gc) == len(oc) == 40
    for layer in range(cfg["num_layers"]):
        kg, vg = gc.read(layer)
        ko, vo = oc.read(layer)
        assert np.max(np.abs(kg - ko)) <= 1e-4
        assert np.max(np.abs(vg - vo)) <= 1e-4


def test_tiny_greedy_tokens_identical(tiny):
    cfg, w, gm, om = tiny
    say("tiny: prompt 20 + 48 greedy, tokens vs oracle")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 20, seed=3)
    gc = gm.new_cache()
    gm.prompt(gc, prompt)
    toks = gm.generate(gc, 48, 0.0)
    otoks, words, _ = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 48)
    assert words == 0
    assert toks == otoks


def test_tiny_sampled_tokens_match_oracle(tiny):
    cfg, w, gm, om = tiny
    say("tiny: prompt 12 + 40 at T=0.7 seed 42, tokens vs oracle")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 12, seed=5)
    seed = O.seed_from_u64(42)
    words = words_for(42, 40)
    gc = gm.new_cache()
    gm.prompt(gc, prompt)
    toks = gm.generate(gc, 40, 0.7, words)
    otoks, nwords, _ = om.generate(om.new_cache(), seed, 0.7, prompt, 40)
    assert nwords == 40
    assert toks == otoks


@pytest.mark.parametrize("temperature", [0.0, 0.7])
def test_tiny_exec_modes_bit_identical(tiny, temperature):
    cfg, w, gm, om = tiny
    prompt = synthetic.make_prompt(cfg["vocab_size"], 16, seed=11)
    words = words_for(9, 12)
    results = {}
    for mode in (G.EXEC_PERSISTENT, G.EXEC_GRAPH, G.EXEC_EAGER):
        say(f"tiny: exec mode {mode}, T={temperature}")
        gm.set_exec(mode)
        gc = gm.new_cache()
        gm.prompt(gc, prompt)
        toks = gm.generate(gc, 12, temperature, words)
        k, v = gc.read(1)
        results[mode] = (toks, gc.last_logits(), k, v)
    gm.set_exec(G.EXEC_PERSISTENT)
    base = results[G.EXEC_PERSISTENT]
    for mode, r in results.items():
        assert r[0] == base[0], mode
        for a, b in zip(r[1:], base[1:]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), mode


def test_tiny_replay_bit_identical_and_divergence(tiny):
    cfg, w, gm, om = tiny
    say("tiny: generate 30 at T=0.7, replay on a fresh cache, then a tampered replay")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 10, seed=2)
    words = words_for(42424242, 30)
    live = gm.new_cache()
    gm.prompt(live, prompt)
    toks = gm.generate(live, 30, 0.7, words)
    history = list(map(int, prompt)) + toks
    rep = gm.new_cache()
    fd, _ = gm.replay(rep, history, len(prompt), 0.7, words)
    assert fd == -1
    assert len(rep) == len(live)
    for layer in range(cfg["num_layers"]):
        for a, b in zip(rep.read(layer), live.read(layer)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(rep.last_logits().view(np.uint32), live.last_logits().view(np.uint32))
    bad = list(history)
    bad[-1] = (bad[-1] + 1) % cfg["vocab_size"]
    fd, sampled = gm.replay(gm.new_cache(), bad, len(prompt), 0.7, words)
    assert fd == len(history) - 1
    assert sampled == history[-1]


def test_tiny_repeat_runs_bit_identical(tiny):
    cfg, w, gm, om = tiny
    say("tiny: 5 repeat runs of prompt 8 + 24 at T=0.7")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 8, seed=1)
    words = words_for(42424242, 24)
    ref = None
    for run in range(5):
        gc = gm.new_cache()
        gm.prompt(gc, prompt)
        toks = gm.generate(gc, 24, 0.7, words)
        state = (toks, gc.last_logits().tobytes(),
                 b"".join(x.tobytes() for l in range(cfg["num_layers"]) for x in gc.read(l)))
        if ref is None:
            ref = state
        assert state == ref, f"run {run} deviated"


def test_135m_greedy_parity(small135):
    cfg, w, gm, om = small135
    say("smollm2-135m shape: prompt 32 + 16 greedy vs oracle")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 32, seed=0)
    gc = gm.new_cache()
    gm.prompt(gc, prompt)
    toks = gm.generate(gc, 16, 0.0)
    glog = gc.last_logits()
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 16)
    d = float(np.max(np.abs(glog - olog)))
    top2 = np.sort(olog)[-2:]
    say(f"135m max|dlogit| after 48 positions = {d:.3e}; top-2 gap {top2[1] - top2[0]:.3e}")
    assert toks == otoks
    assert d <= LOGIT_TOL


def test_attention_trace_matches_oracle():
    """forward_ext's trace (model.rs:486-488): per layer and head, the
    attention probabilities over positions 0..pos, masked ones zero."""
    cfg = synthetic.CONFIGS["tiny"]
    w = synthetic.make_weights(cfg, 12)
    gm, om = G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)
    gc, oc = gm.new_cache(64), om.new_cache()
    for t in [5, 9, 200, 31, 7, 77, 3]:
        gm.forward(t, gc, logits=False)
        om.forward(t, oc)
    for masked in ((), (1, 4)):
        lg, tr = gm.forward(11, gc, masked=masked, trace=True)
        lo, to = om.forward(11, oc, masked=masked, trace=True)
        assert tr.shape == (cfg["num_layers"], cfg["num_heads"], 8)
        assert float(np.max(np.abs(tr - to))) <= 1e-5
        assert np.allclose(tr.sum(axis=2), 1.0, atol=1e-5)
        for p in masked:
            assert np.all(tr[:, :, p] == 0.0)
        assert float(np.max(np.abs(lg - lo))) <= LOGIT_TOL
        gc.truncate(7)
        oc.truncate(7)


def _wo(cfg, w, layer):
    """W_o of a layer from the canonical tensor list [h, q]."""
    names = [n for n, _, _ in synthetic.tensor_specs(cfg)]
    return w[names.index(f"model.layers.{layer}.self_attn.o_proj.weight")]


@pytest.mark.parametrize("name", ["tiny", "smollm2-135m"])
def test_value_norms_match_oracle_bitwise(name):
    """ValueNorms::sync on the device (attribution.rs:116-148) equals the
    oracle's sequential loop bit for bit on the same cached V rows, and the
    ValueNorms mirror extends and truncates as the reference does."""
    cfg = synthetic.CONFIGS[name]
    w = synthetic.make_weights(cfg, 4)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    c = gm.new_cache(256)
    n = 20 if name == "tiny" else 12
    say(f"{name}: prompt of {n}, value norms of every position")
    gm.prompt(c, synthetic.make_prompt(cfg["vocab_size"], n, seed=6))
    got = c.value_norms(0, n)
    L, nh, nkv, hd, h = (cfg["num_layers"], cfg["num_heads"], cfg["num_kv_heads"],
                         cfg["head_dim"], cfg["hidden_size"])
    assert got.shape == (L, n, nh)
    for l in range(L):
        _, vals = c.read(l)
        ref = O.value_norms(_wo(cfg, w, l), vals, h, nh, nkv, hd, 0, n)
        assert np.array_equal(got[l].view(np.uint32), ref.view(np.uint32)), f"layer {l}"
    vn = G.ValueNorms(gm)
    vn.sync(c)
    assert len(vn) == n
    c.truncate(n - 5)
    vn.sync(c)
    assert len(vn) == n - 5
    gm.prompt(c, [1, 2, 3])
    vn.sync(c)
    assert len(vn) == n - 2
    again = c.value_norms(0, n - 2)
    for l in range(L):
        assert np.array_equal(vn.per_layer[l].view(np.uint32), again[l].view(np.uint32))
    assert vn.get(0, 0, 0) == float(again[0, 0, 0])
    with pytest.raises(G.DeferGpuError):
        c.value_norms(0, n + 5)
