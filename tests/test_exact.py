"""The exact sampler (defer_amd/csrc/exact.h, phases.h `sample_exact`): the
device's T > 0 token equals sample_token's (sampler.rs:43-109) on the same
logits, bit for bit, not within a tolerance.

CPU: expf_ref (the host build of the device's expf) against the libm expf
the reference's f32::exp calls, over a strided sweep of all 2^32 inputs (the
full sweep with DEFER_EXHAUSTIVE=1); the oracle's sampling helpers against
closed forms.
GPU (tests/probe/libexact_probe.so): the device expf_ref on every input the
sampler can meet in a large sample; the wave prefix sum; the walker on term
sequences built to hit its hard cases (ties, subnormals, region changes,
uniform and sparse terms) against the oracle's sequential loops; and the
whole sampler through the C ABI on 49,152- and 128,256-wide logits against
oracle sample_token, every draw identical.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle_py as O  # noqa: E402

PROBE = os.path.join(ROOT, "tests", "probe", "libexact_probe.so")


def probe():
    if not os.path.exists(PROBE):
        pytest.skip("tests/probe/libexact_probe.so not built (python -m defer_amd.build probe)")
    L = ctypes.CDLL(PROBE)
    vp, u32, u64, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t
    L.probe_expf_sweep.argtypes = [u32, u64, u32, ctypes.POINTER(u64), ctypes.POINTER(u32)]
    L.probe_expf_device.argtypes = [vp, vp, sz]
    L.probe_scan_device.argtypes = [vp, vp, u32]
    L.probe_walk.argtypes = [vp, u32, vp, u32, vp]
    return L


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------- CPU

def test_expf_ref_equals_libm_expf_strided():
    L = probe()
    full = os.environ.get("DEFER_EXHAUSTIVE") == "1"
    stride = 1 if full else 61
    nd, fd = ctypes.c_uint64(), ctypes.c_uint32()
    L.probe_expf_sweep(0, (1 << 32) // stride + (1 if full else 0), stride, ctypes.byref(nd), ctypes.byref(fd))
    assert nd.value == 0, f"{nd.value} inputs differ, first {fd.value:#010x}"
    # every input of the sampler's own range near 0 and near the underflow edge
    for first in (0x80000000, 0xC2A00000):
        L.probe_expf_sweep(first, 1 << 22, 1, ctypes.byref(nd), ctypes.byref(fd))
        assert nd.value == 0, f"{nd.value} inputs differ, first {fd.value:#010x}"


def test_oracle_sample_terms_closed_forms():
    # uniform terms: total = n exactly for n <= 2^24, r picks floor(r * n)
    n = 1000
    p = np.ones(n, np.float32)
    for word in (0, 0x80000000, 0xFFFFFFFF, 0x12345678):
        tok, tot = O.sample_terms(p, word)
        assert tot == np.float32(n)
        r = (word >> 8) / 2.0 ** 24
        # q = 1/1000 rounded; the cumulative float sum of it decides, which
        # lands within one index of floor(r * n)
        assert abs(tok - int(r * n)) <= 1
    # one positive term: always it
    p = np.zeros(300, np.float32)
    p[123] = np.float32(0.25)
    assert O.sample_terms(p, 0xFFFFFFFF)[0] == 123
    # margin of a uniform draw at the first token's edge
    lg = np.zeros(4, np.float32)
    tok, m = O.sample_margin(lg, 1.0, 0)
    assert tok == 0 and m == 0.0


def test_oracle_sample_terms_against_numpy_sequential_accumulate():
    """The oracle's two sequential f32 sums (total, then the CDF of p * inv)
    against numpy's float32 add.accumulate, which adds strictly in index
    order: the total's bits and the index (first r < cdf, else the last
    positive q) agree on term sequences with ties, subnormal terms, zeros and
    a few large terms. A tree or pairwise order fails this on most draws."""
    rng = np.random.default_rng(5)
    cases = [
        rng.random(49152, dtype=np.float32),
        np.exp(rng.normal(0.0, 2.0, 20000)).astype(np.float32),
        (rng.integers(1, 8, 5000) * np.float32(0.125)).astype(np.float32),  # exact ties likely
        np.where(rng.random(3000) < 0.9, 0.0, rng.random(3000)).astype(np.float32),
        (rng.random(2000) * np.float32(1e-40)).astype(np.float32),  # subnormal terms
    ]
    for p in cases:
        total = np.add.accumulate(p, dtype=np.float32)[-1]
        inv = np.float32(1.0) / total
        q = (p * inv).astype(np.float32)
        cdf = np.add.accumulate(q, dtype=np.float32)
        for word in rng.integers(0, 2 ** 32, 40, dtype=np.uint64):
            r = np.float32((int(word) >> 8) * 2.0 ** -24)
            above = np.nonzero(r < cdf)[0]
            if above.size:
                want = int(above[0])
            else:
                pos = np.nonzero(q > 0)[0]
                want = int(pos[-1]) if pos.size else 0
            tok, tot = O.sample_terms(p, int(word))
            assert tot.view(np.uint32) == total.view(np.uint32)
            assert tok == want


def test_oracle_expf_is_libm():
    x = np.array([0.0, -1.0, -0.5, -87.5, -103.9, -104.0, 1.0], np.float32)
    y = O.expf(x)
    assert y[0] == 1.0 and y[5] == 0.0
    assert abs(float(y[1]) - np.exp(-1.0)) < 1e-7


# ------------------------------------------------------------------- GPU

@pytest.mark.gpu
def test_device_expf_equals_libm_expf():
    """The device expf_ref against libm's on 2^24 random non-positive
    inputs, every input in [-2^-10, 0] and around the subnormal and
    underflow edges, and the special values."""
    L = probe()
    rng = np.random.default_rng(5)
    parts = [
        rng.integers(0x80000000, 0xC2D00000, 1 << 24, dtype=np.uint64).astype(np.uint32),
        np.arange(0x80000000, 0x80000000 + (1 << 22), dtype=np.uint64).astype(np.uint32),
        np.arange(0xBA800000 - (1 << 20), 0xBA800000 + (1 << 20), dtype=np.uint64).astype(np.uint32),
        np.arange(0xC2AE0000, 0xC2D00000, dtype=np.uint64).astype(np.uint32),
        np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x3F800000,
                  0x42B17218, 0x42B17217, 0xC2CFF1B4, 0xC2CFF1B5], np.uint32),
    ]
    bits = np.concatenate(parts)
    x = bits.view(np.float32)
    y = np.empty_like(x)
    assert L.probe_expf_device(ptr(x), ptr(y), x.size) == 0
    want = O.expf(x)
    same = (y.view(np.uint32) == want.view(np.uint32)) | (np.isnan(y) & np.isnan(want))
    bad = np.nonzero(~same)[0]
    print(f"device expf: {x.size} inputs, {len(bad)} differ", flush=True)
    assert len(bad) == 0, [(hex(int(bits[i])), float(y[i]), float(want[i])) for i in bad[:5]]


@pytest.mark.gpu
def test_device_wave_scan():
    L = probe()
    rng = np.random.default_rng(1)
    x = rng.integers(0, 1 << 24, 64 * 100, dtype=np.uint32)
    y = np.empty_like(x)
    assert L.probe_scan_device(ptr(x), ptr(y), x.size) == 0
    want = np.cumsum(x.reshape(-1, 64).astype(np.uint64), axis=1).astype(np.uint32).ravel()
    assert np.array_equal(y, want)


def term_cases():
    """(name, terms): sequences built to hit the walker's hard cases."""
    rng = np.random.default_rng(12)
    out = []
    for n in (1, 5, 63, 64, 65, 1000, 4097, 49152, 128256):
        sd = 0.5 + 2.5 * rng.random()
        out.append((f"softmax{n}", np.exp(rng.normal(0, sd, n) - 4 * sd).astype(np.float32)))
        out.append((f"coarse{n}", (rng.integers(0, 8, n) * 0.125).astype(np.float32)))
        out.append((f"pow2_{n}", np.ldexp(rng.integers(0, 3, n).astype(np.float32), -rng.integers(0, 30, n))))
        out.append((f"sparse{n}", np.where(rng.random(n) < 0.1,
                                           np.exp(-rng.random(n) * 110), 0).astype(np.float32)))
        out.append((f"uniform{n}", np.full(n, np.float32(1.0) / np.float32(n), np.float32)))
        p = np.exp(-rng.random(n) * 20).astype(np.float32)
        p[n // 2] = 1.0
        out.append((f"peak{n}", p))
    return out


@pytest.mark.gpu
def test_walker_against_sequential_loops():
    """Total and index of the device walker equal the oracle's sequential
    loops (sampler.rs:58-108) for every case and draw."""
    L = probe()
    rng = np.random.default_rng(3)
    n_bad = 0
    for name, p in term_cases():
        p = np.ascontiguousarray(p, np.float32)
        if not np.any(p > 0):
            p[0] = 1.0
        words = np.concatenate([[0, 0xFFFFFFFF, 0x80000000], rng.integers(0, 1 << 32, 13, dtype=np.uint64)]
                               ).astype(np.uint32)
        out = np.zeros(2 * words.size, np.uint32)
        assert L.probe_walk(ptr(p), p.size, ptr(words), words.size, ptr(out)) == 0, name
        for i, w in enumerate(words):
            tok, tot = O.sample_terms(p, int(w))
            got_tot = np.uint32(out[2 * i]).view(np.float32)
            if np.float32(tot).view(np.uint32) != out[2 * i] or tok != out[2 * i + 1]:
                n_bad += 1
                print(f"{name} word {int(w):#x}: device ({float(got_tot)!r}, {int(out[2 * i + 1])}) "
                      f"oracle ({float(tot)!r}, {tok})", flush=True)
    assert n_bad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("V,T,quant", [(49152, 0.7, 0.0), (49152, 1.5, 0.0), (128256, 0.8, 0.0), (300, 0.3, 0.0),
                                        (49152, 0.02, 0.0), (49152, 50.0, 0.0), (49152, 1.0, 0.25)])
def test_sampler_equals_sample_token_on_wide_logits(V, T, quant):
    """Logits shaped like the benchmark models' (N(0, 0.5)), set on a cache,
    sampled by the device with 200 words: every token equals oracle
    sample_token's. The model is the tiny one with its head resized to V.
    T = 0.02 leaves a few terms and many subnormal or zero ones; T = 50 makes
    the terms nearly equal (a total near V, long runs in each spacing);
    logits rounded to multiples of `quant` repeat a few values of p, so
    equal terms and ties in the running sums are common."""
    from defer_amd import gpu as G
    from defer_amd import synthetic

    cfg = dict(synthetic.CONFIGS["tiny"])
    cfg["vocab_size"] = V
    w = synthetic.make_weights(cfg, 2)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    c = gm.new_cache(16)
    gm.forward(1, c)  # set_logits replaces the logits of a forward
    rng = np.random.default_rng(V)
    n_bad = 0
    for trial in range(4):
        lg = rng.normal(0, 0.5, V).astype(np.float32)
        if quant:
            lg = (np.round(lg / quant) * quant).astype(np.float32)
        c.set_logits(lg)
        for word in rng.integers(0, 1 << 32, 50, dtype=np.uint64):
            tok = gm.sample(c, T, int(word))
            want = O.sample_token(lg, T, int(word))
            n_bad += tok != want
    print(f"V={V} T={T} quant={quant}: 200 draws, {n_bad} differ from sample_token", flush=True)
    assert n_bad == 0
    c.close()
    gm.close()
