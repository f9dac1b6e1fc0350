"""GPU: the allocation-free generate (defer_gpu_generate_static) against
defer_gpu_generate, through the C ABI: tokens, logits and caches bit for
bit, on two calls in a row (the second with fewer tokens), greedy and at
T > 0, with a stop list; sizes past the static limits are rejected before
anything runs; and a call on a fresh cache longer than any run buffer the
cache has makes no allocation (the library's allocation count and the
device's free memory unchanged), where defer_gpu_generate would have to
allocate."""
import numpy as np
import pytest

from defer_amd import gpu as G
from defer_amd import host as H
from defer_amd import synthetic

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same_state(a, b, layers):
    assert len(a) == len(b)
    assert np.array_equal(bits(a.last_logits()), bits(b.last_logits()))
    for l in range(layers):
        for x, y in zip(a.read(l), b.read(l)):
            assert np.array_equal(bits(x), bits(y)), l


@pytest.mark.parametrize("name", ["tiny", "smollm2-135m"])
def test_generate_static_equals_generate(name):
    cfg = synthetic.CONFIGS[name]
    w = synthetic.make_weights(cfg, 13)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    L, V = cfg["num_layers"], cfg["vocab_size"]
    prompt = synthetic.make_prompt(V, 20, seed=6)
    words = H.chacha8_words(H.seed_from_u64(12), 0, 64)
    a = gm.new_cache(256)
    gm.prompt(a, prompt)
    b = a.clone()
    say(f"{name}: call 1, 48 tokens at T=0.8, static vs allocating")
    ta = gm.generate_static(a, 48, 0.8, words[:48])
    tb = gm.generate(b, 48, 0.8, words[:48])
    assert ta == tb and len(ta) == 48
    same_state(a, b, L)
    say(f"{name}: call 2, 6 greedy tokens")
    ta = gm.generate_static(a, 6, 0.0)
    tb = gm.generate(b, 6, 0.0)
    assert ta == tb and len(ta) == 6
    same_state(a, b, L)
    say(f"{name}: call 3, stop list")
    probe = a.clone()
    nxt = gm.generate(probe, 3, 0.0)
    probe.close()
    ta = gm.generate_static(a, 10, 0.0, stop=[nxt[1], V - 1])
    tb = gm.generate(b, 10, 0.0, stop=[nxt[1], V - 1])
    assert ta == tb and len(ta) <= 2 and ta[-1] in (nxt[1], V - 1)
    same_state(a, b, L)
    for mode in (G.EXEC_GRAPH, G.EXEC_EAGER):
        gm.set_exec(mode)
        ta = gm.generate_static(a, 4, 0.8, words[48:52])
        tb = gm.generate(b, 4, 0.8, words[48:52])
        assert ta == tb
        same_state(a, b, L)
    gm.set_exec(G.EXEC_PERSISTENT)
    n0 = len(a)
    with pytest.raises(G.DeferGpuError) as e:
        gm.generate_static(a, 1 << 17, 0.0)
    assert e.value.code == G.E_INVALID and len(a) == n0
    with pytest.raises(G.DeferGpuError) as e:
        gm.generate_static(a, 2, 0.0, stop=list(range(300)))
    assert e.value.code == G.E_INVALID and len(a) == n0
    a.close()
    b.close()
    gm.close()


def test_generate_static_allocates_nothing():
    """A fresh cache (capacity 1536) after a 4-token prompt has run buffers
    for a few tokens only; 1100 tokens through defer_gpu_generate_static
    leave the library's allocation count and hipMemGetInfo's free bytes as
    they were, while the same call through defer_gpu_generate allocates."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]

    def free_bytes():
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value

    cfg = dict(synthetic.CONFIGS["tiny"])
    cfg["max_seq_len"] = 4096
    w = synthetic.make_weights(cfg, 14)
    gm = G.GpuModel(G.Config.from_dict(cfg), w)
    warm = gm.new_cache(64)
    gm.prompt(warm, [1, 2, 3])
    gm.generate_static(warm, 8, 0.0)  # the kernels' first launch done before counting
    words = H.chacha8_words(H.seed_from_u64(5), 0, 1100)
    a = gm.new_cache(1536)
    gm.prompt(a, [4, 5, 6, 7])
    b = a.clone()
    n0, f0 = G.allocation_count(), free_bytes()
    say("tiny: 1100 tokens at T=0.9 through generate_static on a fresh cache")
    ta = gm.generate_static(a, 1100, 0.9, words)
    n1, f1 = G.allocation_count(), free_bytes()
    say(f"allocations {n0} -> {n1}, device free bytes {f0} -> {f1}")
    assert n1 == n0 and f1 == f0
    tb = gm.generate(b, 1100, 0.9, words)
    assert G.allocation_count() > n1  # the allocating entry point grew its run buffers
    assert ta == tb
    same_state(a, b, cfg["num_layers"])
    for c in (warm, a, b):
        c.close()
    gm.close()
