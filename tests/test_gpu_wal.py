"""GPU: write-ahead logging while the device generates.

The reference appends and flushes one WAL record per token as Session::generate
commits it (main.rs:292-296 -> wal.rs:241-250). Here the persistent kernel
hands each committed token to the host through pinned memory and the host
appends the record while later tokens are still being generated
(defer_gpu_generate_cb, defer_host_session_generate_logged). Tests:
  * records land while the run is still going, one 29-byte record per token;
  * tests/verification.rs:138-180 on the device path: a WAL written during
    generation, a torn tail, the log's checkpoint equal to the live session's,
    checkout bit-identical, then resume-append and continue;
  * an on_token error stops the call at that token, as the reference's `?`.
"""
import os
import time

import numpy as np
import pytest

from defer_amd import gpu as G
from defer_amd import host as H
from defer_amd import synthetic

pytestmark = pytest.mark.gpu

RECORD = 29  # wal.rs:42


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def tiny():
    cfg = synthetic.CONFIGS["tiny"]
    w = synthetic.make_weights(cfg, 99)
    sig = H.sha256(b"".join(x.tobytes() for x in w))
    return cfg, G.GpuModel(G.Config.from_dict(cfg), w), sig


def test_records_land_while_the_device_generates(tmp_path):
    """256 tokens of the 135M shape: each record is on disk (flushed) when its
    on_token returns, and the first arrives long before the run ends."""
    cfg = synthetic.CONFIGS["smollm2-135m"]
    w = synthetic.make_weights(cfg, 0)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    gm.set_batching(0)
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 32, seed=42)]
    c = gm.new_cache(512)
    gm.prompt(c, prompt)
    path = str(tmp_path / "stream.wal")
    wal = H.Wal.create(path, bytes(32), bytes(32), 0.0, len(prompt), 0, prompt)
    base = os.path.getsize(path)
    seen, sizes, times = [], [], []
    t0 = time.perf_counter()

    def on_token(i, t):
        wal.append(t, 0)
        sizes.append(os.path.getsize(path))
        times.append(time.perf_counter() - t0)
        seen.append((i, t))
        return 0

    toks = gm.generate_cb(c, 256, 0.0, on_token=on_token)
    total = time.perf_counter() - t0
    wal.close()
    say(f"135m: 256 tokens in {total * 1e3:.1f} ms; first record after {times[0] * 1e3:.2f} ms, "
        f"half of them after {times[127] * 1e3:.1f} ms")
    assert [i for i, _ in seen] == list(range(256))
    assert [t for _, t in seen] == toks
    assert sizes == [base + RECORD * (i + 1) for i in range(256)]
    assert times[0] < 0.1 * total and times[127] < 0.75 * total
    ref = gm.new_cache(512)
    gm.prompt(ref, prompt)
    assert gm.generate(ref, 256, 0.0) == toks
    assert np.array_equal(bits(ref.last_logits()), bits(c.last_logits()))
    log = H.Wal.read(path)
    assert log["history"] == prompt + toks and not log["torn_tail"]
    c.close()
    ref.close()
    gm.close()


def test_wal_reconstructs_session_on_the_device(tiny, tmp_path):
    """tests/verification.rs:138-180 through the device path."""
    cfg, gm, sig = tiny
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 17, seed=8)]
    seed = H.seed_from_u64(42)
    path = str(tmp_path / "gen.wal")
    s = H.Session(gm, seed, 0.7, capacity=256)
    s.prompt(prompt)
    w = H.Wal.create(path, sig, seed, 0.7, len(prompt), 0, prompt)
    toks = s.generate(30, wal=w)
    w.close()
    assert len(toks) == 30
    with open(path, "ab") as f:  # a crash mid-record
        f.write(bytes([0x01, 0xAA, 0xBB]))
    log = H.Wal.read(path)
    assert log["torn_tail"]
    assert len(log["history"]) == len(prompt) + 30
    ck = str(tmp_path / "live.ckpt")
    s.checkpoint(sig, ck)
    live = H.Checkpoint.load(ck)
    for key in ("base_seed", "temperature", "prompt_len", "rng_word_pos", "history"):
        assert log[key] == live[key], key
    restored = H.Session.checkout(gm, log["base_seed"], log["temperature"], log["history"],
                                  log["prompt_len"], log["rng_word_pos"], capacity=256)
    for layer in range(cfg["num_layers"]):
        for x, y in zip(restored.cache.read(layer), s.cache.read(layer)):
            assert np.array_equal(bits(x), bits(y))
    assert np.array_equal(bits(restored.cache.last_logits()), bits(s.cache.last_logits()))
    w2 = H.Wal.resume(path)
    more = restored.generate(5, wal=w2)
    w2.close()
    log2 = H.Wal.read(path)
    assert not log2["torn_tail"]
    ck2 = str(tmp_path / "cont.ckpt")
    restored.checkpoint(sig, ck2)
    cont = H.Checkpoint.load(ck2)
    for key in ("base_seed", "temperature", "prompt_len", "rng_word_pos", "history"):
        assert log2[key] == cont[key], key
    assert log2["history"] == prompt + toks + more
    # the same continuation on the uninterrupted session
    assert s.generate(5) == more
    restored.close()
    s.close()


def test_on_token_error_stops_the_call(tiny):
    cfg, gm, sig = tiny
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    words = H.chacha8_words(H.seed_from_u64(5), 0, 40)
    a = gm.new_cache(128)
    gm.prompt(a, prompt)
    b = a.clone()
    full = gm.generate(b, 40, 0.9, words)

    def on_token(i, t):
        return 17 if i == 5 else 0

    with pytest.raises(G.DeferGpuError) as e:
        gm.generate_cb(a, 40, 0.9, words, on_token=on_token)
    assert e.value.code == G.E_CALLBACK
    assert gm.last_n == 6
    assert len(a) == len(prompt) + 6
    # the cache holds exactly the six tokens: feeding the seventh gives the
    # uninterrupted run's next logits
    c = gm.new_cache(128)
    gm.prompt(c, prompt + full[:7])
    gm.forward(full[6], a, logits=False)
    assert np.array_equal(bits(a.last_logits()), bits(c.last_logits()))
    for x in (a, b, c):
        x.close()


def test_durable_log_cost(tiny, tmp_path):
    """Reported, not asserted: tokens/s of a logged generate, flushed vs
    synced per record (wal.rs:245-247 --durable)."""
    cfg, gm, sig = tiny
    prompt = [int(x) for x in synthetic.make_prompt(cfg["vocab_size"], 8, seed=1)]
    rates = {}
    for durable in (False, True):
        s = H.Session(gm, H.seed_from_u64(1), 0.0, capacity=512)
        s.prompt(prompt)
        w = H.Wal.create(str(tmp_path / f"d{int(durable)}.wal"), sig, bytes(32), 0.0, len(prompt), 0,
                         prompt, durable=durable)
        t0 = time.perf_counter()
        s.generate(200, wal=w)
        rates[durable] = 200 / (time.perf_counter() - t0)
        w.close()
        s.close()
    say(f"tiny: logged generate {rates[False]:.0f} tok/s flushed, {rates[True]:.0f} tok/s synced")
    assert rates[False] > 0 and rates[True] > 0
