"""GPU: the host Session over the device path, the WAL round trip, longer
contexts (several attention chunks, separate combine), and the staged
persistent kernel against the per-phase kernels on the 135M shape.

Bars as in test_gpu_forward.py: tokens identical to the oracle, logits within
1e-3, and bit-identical results among GPU runs.
"""
import numpy as np
import pytest

import oracle_py as O
from defer_amd import gpu as G
from defer_amd import host as H
from defer_amd import synthetic

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def tiny():
    cfg = synthetic.CONFIGS["tiny"]
    w = synthetic.make_weights(cfg, 77)
    return cfg, w, G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)


@pytest.fixture(scope="module")
def m135():
    cfg = synthetic.CONFIGS["smollm2-135m"]
    w = synthetic.make_weights(cfg, 0)
    return cfg, w, G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)


def test_session_sampling_matches_oracle(tiny):
    cfg, w, gm, om = tiny
    say("tiny: host session, prompt 9 + 50 at T=0.8 seed 5, vs oracle")
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 9, seed=1)]
    s = H.Session(gm, H.seed_from_u64(5), 0.8)
    s.prompt(prompt)
    toks = s.generate(50)
    otoks, words, _ = om.generate(om.new_cache(), O.seed_from_u64(5), 0.8, prompt, 50)
    assert toks == otoks
    assert s.rng_word_pos == words == 50
    assert s.history == prompt + toks and s.prompt_len == 9


def _fingerprint_of_rows(cache) -> bytes:
    """model.rs:233-242 over the cache's host copy: len as u64 LE, then per
    layer every key, then every value, as f32 LE bits (hashlib's SHA-256)."""
    import hashlib

    h = hashlib.sha256(len(cache).to_bytes(8, "little"))
    layers, kvd = cache.shape()
    for l in range(layers):
        k, v = cache.read(l)
        assert k.shape == v.shape == (len(cache), kvd)
        h.update(k.astype("<f4").tobytes())
        h.update(v.astype("<f4").tobytes())
    return h.digest()


def test_cache_fingerprint_and_repeat_runs(tiny):
    """KvCache::fingerprint on a device cache equals an independent SHA-256
    of its rows, an empty cache hashes 8 zero bytes, and repeated sessions
    give the same tokens, the same fingerprint, bit-equal last logits and
    the same rng word position (verification.rs:46-59: 100 runs)."""
    import hashlib

    cfg, w, gm, om = tiny
    say("tiny: cache fingerprint vs hashlib, empty cache, 100 repeat runs of prompt 7 + 24 at T=0.9")
    empty = gm.new_cache(16)
    assert H.cache_fingerprint(empty) == hashlib.sha256(bytes(8)).digest()
    assert empty.shape() == (cfg["num_layers"], cfg["num_kv_heads"] * cfg["head_dim"])
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 7, seed=3)]
    runs = []
    for k in range(100):
        if k:
            s.close()
        s = H.Session(gm, H.seed_from_u64(21), 0.9)
        s.prompt(prompt)
        toks = s.generate(24)
        fp = H.cache_fingerprint(s.cache)
        if k < 3:
            assert fp == _fingerprint_of_rows(s.cache)
        runs.append((toks, fp, bits_of(s.cache.last_logits()).tobytes(), s.rng_word_pos))
    assert all(r == runs[0] for r in runs)
    assert runs[0][3] == 24
    c = s.cache
    c.truncate(10)
    assert H.cache_fingerprint(c) == _fingerprint_of_rows(c) != runs[0][1]


def bits_of(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("T", [0.0, 0.7, 1.5])
def test_checkout_cache_is_bit_identical(tiny, T):
    """verification.rs:84-107 at T in {0, 0.7, 1.5}: a checkout of a live
    session's checkpoint (history, rng position) gives the live cache, the
    cache of the whole history fed as one prompt, bit-equal last logits and
    the same rng word position."""
    cfg, w, gm, om = tiny
    seed = H.seed_from_u64(4242)
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 9, seed=8)]
    live = H.Session(gm, seed, T)
    live.prompt(prompt)
    live.generate(30)
    rep = H.Session.checkout(gm, seed, T, live.history, len(prompt), live.rng_word_pos)
    fresh = H.Session(gm, seed, T)
    fresh.prompt(live.history)
    assert rep.rng_word_pos == live.rng_word_pos == (30 if T else 0)
    for other in (rep, fresh):
        for layer in range(cfg["num_layers"]):
            for x, y in zip(other.cache.read(layer), live.cache.read(layer)):
                assert np.array_equal(bits_of(x), bits_of(y))
        assert np.array_equal(bits_of(other.cache.last_logits()), bits_of(live.cache.last_logits()))
    assert H.cache_fingerprint(rep.cache) == H.cache_fingerprint(live.cache)
    for x in (live, rep, fresh):
        x.close()


def test_session_steps_equal_generate(tiny):
    cfg, w, gm, om = tiny
    say("tiny: 20 single steps vs one generate of 20")
    prompt = [3, 1, 4, 1, 5]
    a = H.Session(gm, H.seed_from_u64(9), 0.6)
    a.prompt(prompt)
    steps = [a.step() for _ in range(20)]
    b = H.Session(gm, H.seed_from_u64(9), 0.6)
    b.prompt(prompt)
    assert b.generate(20) == steps
    assert a.rng_word_pos == b.rng_word_pos == 20
    with pytest.raises(H.DeferHostError, match="after generation started"):
        a.prompt([1])


def test_wal_checkout_rebuilds_cache_and_detects_divergence(tiny, tmp_path):
    cfg, w, gm, om = tiny
    say("tiny: generate 40 at T=0.7 into a WAL, checkout, tamper, checkout")
    seed = H.seed_from_u64(123)
    prompt = [10, 20, 30, 40, 50, 60]
    live = H.Session(gm, seed, 0.7)
    live.prompt(prompt)
    toks = live.generate(40)
    p = str(tmp_path / "s.wal")
    wal = H.Wal.create(p, bytes(32), seed, 0.7, len(prompt), 0, prompt)
    for i, t in enumerate(toks):
        wal.append(t, i + 1)
    wal.close()
    log = H.Wal.read(p)
    rep = H.Session.checkout(gm, log["base_seed"], log["temperature"], log["history"],
                             log["prompt_len"], log["rng_word_pos"])
    assert rep.history == live.history and rep.rng_word_pos == live.rng_word_pos
    for layer in range(cfg["num_layers"]):
        for x, y in zip(rep.cache.read(layer), live.cache.read(layer)):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    assert np.array_equal(rep.cache.last_logits().view(np.uint32),
                          live.cache.last_logits().view(np.uint32))
    bad = list(log["history"])
    bad[20] = (bad[20] + 1) % cfg["vocab_size"]
    with pytest.raises(H.Divergence, match=f"at position 20, checkpoint recorded {bad[20]}"):
        H.Session.checkout(gm, seed, 0.7, bad, len(prompt), 40)
    with pytest.raises(H.DeferHostError, match="inconsistent"):
        H.Session.checkout(gm, seed, 0.7, log["history"], len(prompt), 39)


def test_masked_forward_matches_oracle(tiny):
    cfg, w, gm, om = tiny
    say("tiny: forward with masked positions vs oracle")
    gc, oc = gm.new_cache(), om.new_cache()
    for t in range(1, 9):
        gm.forward(t, gc, logits=False)
        om.forward(t, oc)
    lg = gm.forward(11, gc, masked=[0, 3, 5])
    lo = om.forward(11, oc, masked=[0, 3, 5])
    assert float(np.max(np.abs(lg - lo))) <= LOGIT_TOL


def test_135m_long_prompt_split_attention_and_combine(m135):
    """300 positions: several attention chunks and the separate combine phase."""
    cfg, w, gm, om = m135
    say("135m: prompt 300 + 6 greedy vs oracle (oracle side takes ~15 s)")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 300, seed=21)
    gc = gm.new_cache()
    gm.prompt(gc, prompt)
    toks = gm.generate(gc, 6, 0.0)
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 6)
    d = float(np.max(np.abs(gc.last_logits() - olog)))
    say(f"135m at 306 positions: max|dlogit| = {d:.3e}")
    assert toks == otoks
    assert d <= LOGIT_TOL


def test_135m_persistent_and_phase_kernels_bit_identical(m135):
    cfg, w, gm, om = m135
    say("135m: prompt 40 + 24 at T=0.7, persistent (staged) vs eager kernels")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 40, seed=8)
    words = H.chacha8_words(H.seed_from_u64(3), 0, 24)
    res = {}
    for mode in (G.EXEC_PERSISTENT, G.EXEC_EAGER):
        gm.set_exec(mode)
        c = gm.new_cache()
        gm.prompt(c, prompt)
        toks = gm.generate(c, 24, 0.7, words)
        res[mode] = (toks, c.last_logits(), c.read(7))
    gm.set_exec(G.EXEC_PERSISTENT)
    a, b = res[G.EXEC_PERSISTENT], res[G.EXEC_EAGER]
    assert a[0] == b[0]
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    for x, y in zip(a[2], b[2]):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_360m_rows_loaded_directly_greedy_parity():
    """The 360M shape does not fit the LDS staging: compute waves load their
    rows from HBM (same arithmetic order)."""
    cfg = synthetic.CONFIGS["smollm2-360m"]
    w = synthetic.make_weights(cfg, 0)
    gm, om = G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)
    say("360m: prompt 24 + 8 greedy vs oracle")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 24, seed=2)
    c = gm.new_cache(64)
    gm.prompt(c, prompt)
    toks = gm.generate(c, 8, 0.0)
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 8)
    d = float(np.max(np.abs(c.last_logits() - olog)))
    say(f"360m max|dlogit| = {d:.3e}")
    assert toks == otoks
    assert d <= LOGIT_TOL
    c.close()
    gm.close()


def test_tiny_past_2048_positions_chunk_256_vs_oracle():
    """Past 2048 positions the attention chunk is 256 positions: decode and
    batched prefill there, against the oracle and each other."""
    cfg = dict(synthetic.CONFIGS["tiny"])
    cfg["max_seq_len"] = 4096
    w = synthetic.make_weights(cfg, 3)
    gm, om = G.GpuModel(G.Config.from_dict(cfg), w), O.OracleModel(cfg, w)
    say("tiny: prompt 2300 (batched) + 8 greedy vs oracle; and vs token by token")
    prompt = synthetic.make_prompt(cfg["vocab_size"], 2300, seed=5)
    a = gm.new_cache(2400)
    gm.prompt(a, prompt)
    toks = gm.generate(a, 8, 0.0)
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 8)
    d = float(np.max(np.abs(a.last_logits() - olog)))
    say(f"tiny at 2308 positions: max|dlogit| = {d:.3e}")
    assert toks == otoks
    assert d <= LOGIT_TOL
    gm.set_batching(0)
    b = gm.new_cache(2400)
    gm.prompt(b, prompt)
    gm.set_batching(16)
    assert gm.generate(b, 8, 0.0) == toks
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))


def test_8b_shape_head_dim_128_untied_vs_oracle():
    """The 8B shape (h 4096, 32/8 heads, head_dim 128, ff 14336, vocab 128256,
    untied lm_head) cut to 2 layers: greedy tokens and logits vs the oracle,
    batched prefill bit-identical to token by token."""
    cfg = dict(synthetic.CONFIGS["llama-3-8b"])
    cfg["num_layers"] = 2
    say("8b shape x 2 layers: weights (about 6 GB)")
    w = synthetic.make_weights(cfg, 0)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    prompt = synthetic.make_prompt(cfg["vocab_size"], 20, seed=8)
    a = gm.new_cache(64)
    gm.prompt(a, prompt)
    toks = gm.generate(a, 3, 0.0)
    gm.set_batching(0)
    b = gm.new_cache(64)
    gm.prompt(b, prompt)
    gm.set_batching(16)
    assert gm.generate(b, 3, 0.0) == toks
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))
    say("8b shape: oracle (20 + 3 forwards on the CPU)")
    om = O.OracleModel(cfg, w)
    otoks, _, olog = om.generate(om.new_cache(), bytes(32), 0.0, prompt, 3)
    d = float(np.max(np.abs(a.last_logits() - olog)))
    say(f"8b shape: max|dlogit| vs oracle = {d:.3e}")
    assert toks == otoks
    assert d <= LOGIT_TOL
    del om
    a.close()
    b.close()
    gm.close()


def test_checkpoint_file_checkout_rebuilds_session(tiny, tmp_path):
    """Session::checkpoint -> file -> Session::checkout (engine.rs:223-274):
    same history, rng position, cache and logits; a wrong model signature and
    a tampered record are refused with the reference's messages."""
    cfg, w, gm, om = tiny
    say("tiny: generate 30 at T=0.9, checkpoint to a file, checkout from it")
    sig = H.sha256(b"".join(x.tobytes() for x in w))
    live = H.Session(gm, H.seed_from_u64(77), 0.9)
    live.prompt([9, 8, 7, 6])
    live.generate(30)
    p = str(tmp_path / "s.ckpt")
    live.checkpoint(sig, p)
    rep = H.Session.checkout_file(gm, sig, p)
    assert rep.history == live.history and rep.prompt_len == 4
    assert rep.rng_word_pos == live.rng_word_pos == 30
    assert np.array_equal(rep.cache.last_logits().view(np.uint32),
                          live.cache.last_logits().view(np.uint32))
    for x, y in zip(rep.cache.read(1), live.cache.read(1)):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    assert rep.step() == live.step()
    with pytest.raises(H.DeferHostError, match="model signature mismatch"):
        H.Session.checkout_file(gm, bytes(32), p)
    ck = H.Checkpoint.load(p)
    bad = list(ck["history"])
    bad[15] = (bad[15] + 1) % cfg["vocab_size"]
    H.Checkpoint.save(p, sig, ck["base_seed"], ck["temperature"], ck["prompt_len"],
                      ck["rng_word_pos"], bad)
    with pytest.raises(H.Divergence, match=f"at position 15, checkpoint recorded {bad[15]}"):
        H.Session.checkout_file(gm, sig, p)


def test_model_load_from_safetensors(tmp_path):
    """Model::load (model.rs:285-347): the file's tensors by name, the config
    from its defer.config metadata (or config.json), the signature = SHA-256
    of the file; logits bit-identical to the model built from the arrays."""
    import hashlib
    import json
    import safetensors.numpy as stn
    cfg = synthetic.CONFIGS["tiny"]
    w = synthetic.make_weights(cfg, 31)
    names = [n for n, _, _ in synthetic.tensor_specs(cfg)]
    hf = {"vocab_size": cfg["vocab_size"], "hidden_size": cfg["hidden_size"],
          "intermediate_size": cfg["intermediate_size"], "num_hidden_layers": cfg["num_layers"],
          "num_attention_heads": cfg["num_heads"], "num_key_value_heads": cfg["num_kv_heads"],
          "head_dim": cfg["head_dim"], "rms_norm_eps": cfg["rms_norm_eps"],
          "rope_theta": cfg["rope_theta"], "max_position_embeddings": cfg["max_seq_len"],
          "tie_word_embeddings": bool(cfg["tie_word_embeddings"]), "hidden_act": "silu"}
    p = str(tmp_path / "model.safetensors")
    stn.save_file(dict(zip(names, w)), p, metadata={"defer.config": json.dumps(hf)})
    say("tiny: load from a safetensors file vs the arrays")
    gm, lcfg, sig = H.load_model(p)
    assert sig == hashlib.sha256(open(p, "rb").read()).digest()
    ref = G.GpuModel(G.Config.from_dict(cfg), w)
    a, b = gm.new_cache(64), ref.new_cache(64)
    for t in (4, 40, 200):
        la, lb = gm.forward(t, a), ref.forward(t, b)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    # F16 tensors with the config in config.json beside the file
    d = tmp_path / "half"
    d.mkdir()
    p2 = str(d / "model.safetensors")
    stn.save_file({n: x.astype(np.float16) for n, x in zip(names, w)}, p2)
    (d / "config.json").write_text(json.dumps(hf))
    gm2, lcfg2, _ = H.load_model(p2)
    assert lcfg2 == lcfg
    ref2 = G.GpuModel(G.Config.from_dict(cfg), [x.astype(np.float16).astype(np.float32) for x in w])
    c2, d2 = gm2.new_cache(64), ref2.new_cache(64)
    la, lb = gm2.forward(9, c2), ref2.forward(9, d2)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_full_cache_step_at_temperature_reports_context(tiny):
    """A session whose cache is full, stepped at T > 0: the context error
    with the reference's message (model.rs:420-422), the history unchanged,
    and the rng position one word further on, because Session::step samples
    (one word) before feed fails (engine.rs:113-117). generate past the end
    commits the tokens that fit, then reports the same error."""
    cfg, w, gm, om = tiny
    prompt = synthetic.make_prompt(cfg["vocab_size"], 8, seed=2)
    s = H.Session(gm, H.seed_from_u64(5), 0.9, capacity=12)
    s.prompt(prompt)
    toks = s.generate(4)
    assert len(toks) == 4 and s.rng_word_pos == 4
    hist = s.history
    with pytest.raises(H.DeferHostError, match="context length"):
        s.step()
    assert s.history == hist and s.rng_word_pos == 5
    s2 = H.Session(gm, H.seed_from_u64(5), 0.9, capacity=12)
    s2.prompt(prompt)
    with pytest.raises(H.DeferHostError, match="context length"):
        s2.generate(10)
    assert s2.history == hist and s2.rng_word_pos == 5
    s.close()
    s2.close()
