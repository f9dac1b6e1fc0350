"""ctypes binding of the C ABI in include/defer_gpu.h (libdefer_gpu.so).

Mirrors the reference's hot-path types: ``GpuModel`` stands for ``Model``
(model.rs:271-280) and ``GpuCache`` for ``KvCache`` (model.rs:182-243), with
the KV cache kept in HBM. The library is required: importing this module on a
machine without the built ``libdefer_gpu.so`` raises, and there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdefer_gpu.so")

EXEC_PERSISTENT = 0
EXEC_GRAPH = 1
EXEC_EAGER = 2

OK = 0
E_INVALID = 1
E_TOKEN = 2
E_CONTEXT = 3
E_HIP = 4
E_NO_LOGITS = 5
E_TIMEOUT = 6
E_CALLBACK = 7


class DeferGpuError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"defer_gpu error {code}: {msg}")
        self.code = code


class Config(ctypes.Structure):
    """defer_gpu_config: Model::Config (model.rs:23-39)."""

    _fields_ = [
        ("vocab_size", ctypes.c_uint32),
        ("hidden_size", ctypes.c_uint32),
        ("intermediate_size", ctypes.c_uint32),
        ("num_layers", ctypes.c_uint32),
        ("num_heads", ctypes.c_uint32),
        ("num_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("max_seq_len", ctypes.c_uint32),
        ("tie_word_embeddings", ctypes.c_uint32),
        ("activation", ctypes.c_uint32),
        ("has_bias", ctypes.c_uint32),
    ]

    @classmethod
    def from_dict(cls, d: dict) -> "Config":
        c = cls()
        for name, _ in cls._fields_:
            setattr(c, name, d[name])
        return c

    def to_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


# defer_gpu_token_fn: int (*)(void* user, uint32_t index, uint32_t token)
TOKEN_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32)

_lib = None


def lib() -> ctypes.CDLL:
    """Load libdefer_gpu.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')"
        )
    L = ctypes.CDLL(LIB_PATH)
    u32, f32, sz, vp = ctypes.c_uint32, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p
    P = ctypes.POINTER
    L.defer_gpu_model_create.argtypes = [P(Config), P(vp), sz, u32, P(vp)]
    L.defer_gpu_model_create.restype = ctypes.c_int
    L.defer_gpu_model_destroy.argtypes = [vp]
    L.defer_gpu_model_destroy.restype = None
    L.defer_gpu_model_tensor_count.argtypes = [P(Config)]
    L.defer_gpu_model_tensor_count.restype = sz
    L.defer_gpu_model_set_exec.argtypes = [vp, u32]
    L.defer_gpu_model_set_exec.restype = ctypes.c_int
    L.defer_gpu_cache_create.argtypes = [vp, u32, P(vp)]
    L.defer_gpu_cache_create.restype = ctypes.c_int
    L.defer_gpu_cache_destroy.argtypes = [vp]
    L.defer_gpu_cache_destroy.restype = None
    L.defer_gpu_cache_len.argtypes = [vp]
    L.defer_gpu_cache_len.restype = u32
    L.defer_gpu_cache_truncate.argtypes = [vp, u32]
    L.defer_gpu_cache_truncate.restype = ctypes.c_int
    L.defer_gpu_cache_clone.argtypes = [vp, P(vp)]
    L.defer_gpu_cache_clone.restype = ctypes.c_int
    L.defer_gpu_cache_read.argtypes = [vp, u32, vp, vp]
    L.defer_gpu_cache_read.restype = ctypes.c_int
    L.defer_gpu_cache_shape.argtypes = [vp, P(u32), P(u32)]
    L.defer_gpu_cache_shape.restype = ctypes.c_int
    L.defer_gpu_value_norms.argtypes = [vp, u32, u32, vp]
    L.defer_gpu_value_norms.restype = ctypes.c_int
    L.defer_gpu_forward.argtypes = [vp, vp, u32, vp, sz, vp, vp]
    L.defer_gpu_forward.restype = ctypes.c_int
    L.defer_gpu_last_logits.argtypes = [vp, vp]
    L.defer_gpu_last_logits.restype = ctypes.c_int
    L.defer_gpu_sample.argtypes = [vp, vp, f32, u32, P(u32)]
    L.defer_gpu_sample.restype = ctypes.c_int
    L.defer_gpu_step.argtypes = [vp, vp, f32, u32, P(u32)]
    L.defer_gpu_step.restype = ctypes.c_int
    L.defer_gpu_generate.argtypes = [vp, vp, u32, f32, vp, vp, sz, vp, P(u32)]
    L.defer_gpu_generate.restype = ctypes.c_int
    L.defer_gpu_generate_cb.argtypes = [vp, vp, u32, f32, vp, vp, sz, vp, P(u32), TOKEN_FN, vp]
    L.defer_gpu_generate_cb.restype = ctypes.c_int
    L.defer_gpu_generate_static.argtypes = [vp, vp, u32, f32, vp, vp, sz, vp, P(u32)]
    L.defer_gpu_generate_static.restype = ctypes.c_int
    L.defer_gpu_prompt.argtypes = [vp, vp, vp, sz]
    L.defer_gpu_prompt.restype = ctypes.c_int
    L.defer_gpu_replay.argtypes = [vp, vp, vp, sz, sz, f32, vp, P(ctypes.c_int64), P(u32)]
    L.defer_gpu_replay.restype = ctypes.c_int
    L.defer_gpu_last_error.argtypes = []
    L.defer_gpu_last_error.restype = ctypes.c_char_p
    L.defer_gpu_allocation_count.argtypes = []
    L.defer_gpu_allocation_count.restype = ctypes.c_uint64
    L.defer_gpu_shutdown.argtypes = []
    L.defer_gpu_shutdown.restype = ctypes.c_int
    L.defer_gpu_last_device_ms.argtypes = [vp]
    L.defer_gpu_last_device_ms.restype = ctypes.c_double
    L.defer_gpu_model_set_batching.argtypes = [vp, u32]
    L.defer_gpu_model_set_batching.restype = ctypes.c_int
    L.defer_gpu_forward_batch.argtypes = [vp, P(vp), vp, u32, vp]
    L.defer_gpu_forward_batch.restype = ctypes.c_int
    L.defer_gpu_step_batch.argtypes = [vp, P(vp), u32, f32, vp, vp]
    L.defer_gpu_step_batch.restype = ctypes.c_int
    L.defer_gpu_cache_set_logits.argtypes = [vp, vp]
    L.defer_gpu_cache_set_logits.restype = ctypes.c_int
    L.defer_gpu_model_set_grid.argtypes = [vp, u32, u32]
    L.defer_gpu_model_set_grid.restype = ctypes.c_int
    L.defer_gpu_cache_capacity.argtypes = [vp]
    L.defer_gpu_cache_capacity.restype = u32
    L.defer_gpu_model_set_profiling.argtypes = [vp, u32]
    L.defer_gpu_model_set_profiling.restype = ctypes.c_int
    L.defer_gpu_batch_stats.argtypes = [vp, P(ctypes.c_double), u32]
    L.defer_gpu_batch_stats.restype = ctypes.c_int
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != OK:
        msg = lib().defer_gpu_last_error().decode(errors="replace")
        raise DeferGpuError(rc, msg)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def allocation_count() -> int:
    """Device and pinned host allocations the library has made so far."""
    return int(lib().defer_gpu_allocation_count())


def shutdown() -> None:
    """Synchronise and reset every device the library made a model on, once
    every model and cache is closed (raises DeferGpuError otherwise). The reset
    frees every allocation of the process on those devices: call it last."""
    _check(lib().defer_gpu_shutdown())


def tensor_count(cfg: Config) -> int:
    return int(lib().defer_gpu_model_tensor_count(ctypes.byref(cfg)))


class GpuModel:
    """Weights resident in HBM (Model::from_safetensors, model.rs:301-363)."""

    def __init__(self, cfg: Config, tensors: Sequence[np.ndarray]):
        self.cfg = cfg
        arrs = [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
        ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
        h = ctypes.c_void_p()
        _check(lib().defer_gpu_model_create(ctypes.byref(cfg), ptrs, len(arrs), 0, ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().defer_gpu_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vocab_size(self) -> int:
        return int(self.cfg.vocab_size)

    def set_exec(self, mode: int) -> None:
        _check(lib().defer_gpu_model_set_exec(self._h, mode))

    def new_cache(self, capacity: int = 0) -> "GpuCache":
        return GpuCache(self, capacity)

    def forward(self, token: int, cache: "GpuCache", masked: Sequence[int] = (),
                logits: bool = True, trace: bool = False):
        """Model::forward_ext (model.rs:394-520); logits copied out if asked.
        With trace=True returns (logits, probabilities [L, num_heads, pos + 1])."""
        out = np.empty(self.vocab_size, dtype=np.float32) if logits else None
        m = _u32(masked) if len(masked) else None
        tr = None
        if trace:
            tr = np.empty((self.cfg.num_layers, self.cfg.num_heads, len(cache) + 1), dtype=np.float32)
        _check(lib().defer_gpu_forward(self._h, cache._h, int(token), _ptr(m),
                                       0 if m is None else len(m), _ptr(out), _ptr(tr)))
        return (out, tr) if trace else out

    def prompt(self, cache: "GpuCache", tokens: Sequence[int]) -> None:
        t = _u32(tokens)
        _check(lib().defer_gpu_prompt(self._h, cache._h, _ptr(t), len(t)))

    def sample(self, cache: "GpuCache", temperature: float, word: int = 0) -> int:
        out = ctypes.c_uint32()
        _check(lib().defer_gpu_sample(self._h, cache._h, float(temperature), int(word) & 0xFFFFFFFF,
                                      ctypes.byref(out)))
        return int(out.value)

    def step(self, cache: "GpuCache", temperature: float, word: int = 0) -> int:
        out = ctypes.c_uint32()
        _check(lib().defer_gpu_step(self._h, cache._h, float(temperature), int(word) & 0xFFFFFFFF,
                                    ctypes.byref(out)))
        return int(out.value)

    def generate(self, cache: "GpuCache", max_tokens: int, temperature: float,
                 words: Optional[Sequence[int]] = None, stop: Sequence[int] = ()) -> list:
        w = _u32(words) if words is not None else None
        if temperature != 0.0 and (w is None or len(w) < max_tokens):
            raise ValueError("need one rng word per token when temperature > 0")
        s = _u32(stop) if len(stop) else None
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        n = ctypes.c_uint32()
        _check(lib().defer_gpu_generate(self._h, cache._h, int(max_tokens), float(temperature),
                                        _ptr(w), _ptr(s), 0 if s is None else len(s), _ptr(out),
                                        ctypes.byref(n)))
        return [int(x) for x in out[: n.value]]

    def generate_cb(self, cache: "GpuCache", max_tokens: int, temperature: float,
                    words: Optional[Sequence[int]] = None, stop: Sequence[int] = (),
                    on_token=None) -> list:
        """generate() with on_token(index, token) -> int called per committed
        token while the device still runs (defer_gpu_generate_cb)."""
        w = _u32(words) if words is not None else None
        if temperature != 0.0 and (w is None or len(w) < max_tokens):
            raise ValueError("need one rng word per token when temperature > 0")
        s = _u32(stop) if len(stop) else None
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        n = ctypes.c_uint32()
        fn = TOKEN_FN(lambda _u, i, t: int(on_token(int(i), int(t)) or 0)) if on_token else TOKEN_FN(0)
        rc = lib().defer_gpu_generate_cb(self._h, cache._h, int(max_tokens), float(temperature),
                                         _ptr(w), _ptr(s), 0 if s is None else len(s), _ptr(out),
                                         ctypes.byref(n), fn, None)
        self.last_n = int(n.value)
        _check(rc)
        return [int(x) for x in out[: n.value]]

    def generate_static(self, cache: "GpuCache", max_tokens: int, temperature: float,
                        words: Optional[Sequence[int]] = None, stop: Sequence[int] = ()) -> list:
        """generate() through the allocation-free entry point."""
        w = _u32(words) if words is not None else None
        if temperature != 0.0 and (w is None or len(w) < max_tokens):
            raise ValueError("need one rng word per token when temperature > 0")
        s = _u32(stop) if len(stop) else None
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        n = ctypes.c_uint32()
        _check(lib().defer_gpu_generate_static(self._h, cache._h, int(max_tokens),
                                               float(temperature), _ptr(w), _ptr(s),
                                               0 if s is None else len(s), _ptr(out),
                                               ctypes.byref(n)))
        return [int(x) for x in out[: n.value]]

    def replay(self, cache: "GpuCache", history: Sequence[int], prompt_len: int,
               temperature: float, words: Optional[Sequence[int]] = None):
        """Returns (first_divergence_index or -1, sampled token at it)."""
        h = _u32(history)
        w = _u32(words) if words is not None else None
        fd = ctypes.c_int64(-1)
        sd = ctypes.c_uint32(0)
        _check(lib().defer_gpu_replay(self._h, cache._h, _ptr(h), len(h), int(prompt_len),
                                      float(temperature), _ptr(w), ctypes.byref(fd),
                                      ctypes.byref(sd)))
        return int(fd.value), int(sd.value)

    def last_device_ms(self) -> float:
        return float(lib().defer_gpu_last_device_ms(self._h))

    def set_batching(self, min_rows: int) -> None:
        """Prompts and replays of at least min_rows tokens take the batched
        (MFMA GEMM) path; 0 feeds token by token. Same bits either way."""
        _check(lib().defer_gpu_model_set_batching(self._h, int(min_rows)))

    def forward_batch(self, caches: Sequence["GpuCache"], tokens: Sequence[int],
                      logits: bool = False) -> Optional[np.ndarray]:
        """Feeds tokens[b] to caches[b] as one batch (a cache listed k times
        gets k consecutive positions); [n, V] logits if asked."""
        t = _u32(tokens)
        hs = (ctypes.c_void_p * len(caches))(*[c._h for c in caches])
        out = np.empty((len(t), self.vocab_size), dtype=np.float32) if logits else None
        _check(lib().defer_gpu_forward_batch(self._h, hs, _ptr(t), len(t), _ptr(out)))
        return out

    def set_grid(self, workgroups: int = 0, gemm_cus: int = 0) -> None:
        """Launch geometry (0: the device's); before the first cache only."""
        _check(lib().defer_gpu_model_set_grid(self._h, int(workgroups), int(gemm_cus)))

    def set_profiling(self, on: bool) -> None:
        _check(lib().defer_gpu_model_set_profiling(self._h, 1 if on else 0))

    def batch_stats(self, reset: bool = True) -> dict:
        """Event-timed GEMM / attention totals of batched calls since the last reset."""
        st = (ctypes.c_double * 6)()
        _check(lib().defer_gpu_batch_stats(self._h, st, 1 if reset else 0))
        return {"gemm_ms": st[0], "gemm_flop": st[1], "gemm_launches": int(st[2]),
                "attn_ms": st[3], "attn_flop": st[4], "attn_launches": int(st[5])}

    def step_batch(self, caches: Sequence["GpuCache"], temperature: float,
                   words: Optional[Sequence[int]] = None) -> list:
        """Session::step on distinct caches in lockstep."""
        w = _u32(words) if words is not None else None
        if temperature != 0.0 and (w is None or len(w) < len(caches)):
            raise ValueError("need one rng word per cache when temperature > 0")
        hs = (ctypes.c_void_p * len(caches))(*[c._h for c in caches])
        out = np.zeros(max(len(caches), 1), dtype=np.uint32)
        _check(lib().defer_gpu_step_batch(self._h, hs, len(caches), float(temperature), _ptr(w),
                                          _ptr(out)))
        return [int(x) for x in out[: len(caches)]]


class GpuCache:
    """KvCache (model.rs:182-243), preallocated in HBM."""

    def __init__(self, model: GpuModel, capacity: int = 0, _handle=None):
        self.model = model
        if _handle is not None:
            self._h = _handle
            return
        h = ctypes.c_void_p()
        _check(lib().defer_gpu_cache_create(model._h, int(capacity), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().defer_gpu_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(lib().defer_gpu_cache_len(self._h))

    @property
    def capacity(self) -> int:
        return int(lib().defer_gpu_cache_capacity(self._h))

    def truncate(self, n: int) -> None:
        _check(lib().defer_gpu_cache_truncate(self._h, int(n)))

    def clone(self) -> "GpuCache":
        h = ctypes.c_void_p()
        _check(lib().defer_gpu_cache_clone(self._h, ctypes.byref(h)))
        return GpuCache(self.model, _handle=h)

    def shape(self) -> tuple:
        """(layers, kv_dim): the shape of each layer's keys / values rows."""
        nl, kv = ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().defer_gpu_cache_shape(self._h, ctypes.byref(nl), ctypes.byref(kv)))
        return int(nl.value), int(kv.value)

    def read(self, layer: int):
        """(keys, values) of one layer as [len, kv_dim] arrays."""
        c = self.model.cfg
        kvd = c.num_kv_heads * c.head_dim
        n = len(self)
        k = np.empty((n, kvd), dtype=np.float32)
        v = np.empty((n, kvd), dtype=np.float32)
        _check(lib().defer_gpu_cache_read(self._h, int(layer), _ptr(k), _ptr(v)))
        return k, v

    def value_norms(self, t0: int, t1: int) -> np.ndarray:
        """||W_o,h . v_{t,kv(h)}|| for positions [t0, t1): [layers, t1 - t0, heads]
        (the extension step of ValueNorms::sync, attribution.rs:116-148)."""
        c = self.model.cfg
        out = np.empty((c.num_layers, t1 - t0, c.num_heads), dtype=np.float32)
        _check(lib().defer_gpu_value_norms(self._h, int(t0), int(t1), _ptr(out)))
        return out

    def set_logits(self, logits) -> None:
        """Replace the last logits (the next sample / step samples these)."""
        a = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
        if a.shape != (self.model.vocab_size,):
            raise ValueError(f"need {self.model.vocab_size} logits")
        _check(lib().defer_gpu_cache_set_logits(self._h, _ptr(a)))

    def last_logits(self) -> np.ndarray:
        out = np.empty(self.model.vocab_size, dtype=np.float32)
        _check(lib().defer_gpu_last_logits(self._h, _ptr(out)))
        return out


class ValueNorms:
    """Cache of ||W_o,h . v_{t,kv(h)}|| per (layer, position, query head)
    (attribution.rs:91-153): values depend only on the cached V rows, so they
    are computed once per position -- on the device -- and reused."""

    def __init__(self, model: "GpuModel"):
        self.num_heads = model.cfg.num_heads
        self._len = 0
        self.per_layer = [np.zeros((0, self.num_heads), dtype=np.float32)
                          for _ in range(model.cfg.num_layers)]

    def __len__(self) -> int:
        return self._len

    def is_empty(self) -> bool:
        return self._len == 0

    def sync(self, cache: "GpuCache") -> None:
        """Bring the cache in line with `cache` (extend, or drop stale entries)."""
        n = len(cache)
        if n < self._len:
            self.per_layer = [v[:n] for v in self.per_layer]
            self._len = n
        if n > self._len:
            new = cache.value_norms(self._len, n)
            self.per_layer = [np.concatenate([v, new[l]]) for l, v in enumerate(self.per_layer)]
        self._len = n

    def get(self, layer: int, t: int, head: int) -> float:
        return float(self.per_layer[layer][t, head])
