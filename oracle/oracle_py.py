"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU
baseline), never as part of the product path.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

E_TOKEN = 1
E_CONTEXT = 2


class OracleConfig(ctypes.Structure):
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
    def from_dict(cls, d: dict) -> "OracleConfig":
        c = cls()
        for name, _ in cls._fields_:
            setattr(c, name, d[name])
        return c


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, u32, f32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float
    P = ctypes.POINTER
    L.oracle_matmul_sequential.argtypes = [vp, vp, vp, sz, sz, sz]
    L.oracle_linear.argtypes = [vp, vp, vp, vp, sz, sz]
    L.oracle_dot.argtypes = [vp, vp, sz]
    L.oracle_dot.restype = f32
    L.oracle_rmsnorm.argtypes = [vp, vp, vp, sz, f32]
    L.oracle_layernorm.argtypes = [vp, vp, vp, vp, sz, f32]
    L.oracle_silu.argtypes = [f32]
    L.oracle_silu.restype = f32
    L.oracle_gelu.argtypes = [f32]
    L.oracle_gelu.restype = f32
    L.oracle_add_inplace.argtypes = [vp, vp, sz]
    L.oracle_mul_inplace.argtypes = [vp, vp, sz]
    L.oracle_softmax_inplace.argtypes = [vp, sz]
    L.oracle_model_create.argtypes = [P(OracleConfig), P(vp), sz]
    L.oracle_model_create.restype = vp
    L.oracle_model_destroy.argtypes = [vp]
    L.oracle_model_tensor_count.argtypes = [P(OracleConfig)]
    L.oracle_model_tensor_count.restype = sz
    L.oracle_cache_create.argtypes = [vp]
    L.oracle_cache_create.restype = vp
    L.oracle_cache_destroy.argtypes = [vp]
    L.oracle_cache_len.argtypes = [vp]
    L.oracle_cache_len.restype = u32
    L.oracle_cache_truncate.argtypes = [vp, u32]
    L.oracle_cache_read.argtypes = [vp, u32, vp, vp]
    L.oracle_forward_ext.argtypes = [vp, vp, u32, vp, sz, vp, vp]
    L.oracle_forward_ext.restype = ctypes.c_int
    L.oracle_argmax.argtypes = [vp, sz]
    L.oracle_argmax.restype = u32
    L.oracle_softmax_with_temperature.argtypes = [vp, sz, f32, vp]
    L.oracle_unit_f32.argtypes = [u32]
    L.oracle_unit_f32.restype = f32
    L.oracle_sample_token.argtypes = [vp, sz, f32, u32]
    L.oracle_sample_token.restype = u32
    L.oracle_sample_margin.argtypes = [vp, sz, f32, u32, P(f32)]
    L.oracle_sample_margin.restype = u32
    L.oracle_sample_terms.argtypes = [vp, sz, u32, P(f32)]
    L.oracle_sample_terms.restype = u32
    L.oracle_expf_array.argtypes = [vp, vp, sz]
    L.oracle_expf_array.restype = None
    L.oracle_chacha_block.argtypes = [vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, vp]
    L.oracle_seed_from_u64.argtypes = [ctypes.c_uint64, vp]
    L.oracle_pcg32_step.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    L.oracle_pcg32_step.restype = ctypes.c_uint64
    L.oracle_pcg32_output.argtypes = [ctypes.c_uint64]
    L.oracle_pcg32_output.restype = ctypes.c_uint32
    L.oracle_chacha8_word.argtypes = [vp, ctypes.c_uint64]
    L.oracle_chacha8_word.restype = u32
    L.oracle_generate.argtypes = [vp, vp, vp, f32, vp, sz, sz, vp, vp]
    L.oracle_generate.restype = ctypes.c_int64
    L.oracle_checkout.argtypes = [vp, vp, vp, f32, vp, sz, sz, P(u32), vp]
    L.oracle_value_norms.argtypes = [vp, vp, u32, u32, u32, u32, u32, u32, vp]
    L.oracle_value_norms.restype = None
    L.oracle_checkout.restype = ctypes.c_int64
    _lib = L
    return L


def f32a(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _p(a: Optional[np.ndarray]):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


# ---- ops -------------------------------------------------------------------

def linear(x, w, bias=None, out_dim=None) -> np.ndarray:
    x = f32a(x)
    w = f32a(w)
    out_dim = out_dim if out_dim is not None else w.size // x.size
    out = np.empty(out_dim, dtype=np.float32)
    b = f32a(bias) if bias is not None else None
    lib().oracle_linear(_p(out), _p(x), _p(w), _p(b), x.size, out_dim)
    return out


def matmul_sequential(a, b, m, n, k) -> np.ndarray:
    a, b = f32a(a), f32a(b)
    out = np.empty(m * n, dtype=np.float32)
    lib().oracle_matmul_sequential(_p(out), _p(a), _p(b), m, n, k)
    return out


def dot(a, b) -> float:
    a, b = f32a(a), f32a(b)
    return float(lib().oracle_dot(_p(a), _p(b), a.size))


def rmsnorm(x, w, eps) -> np.ndarray:
    x, w = f32a(x), f32a(w)
    out = np.empty_like(x)
    lib().oracle_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def layernorm(x, w, b, eps) -> np.ndarray:
    x, w, b = f32a(x), f32a(w), f32a(b)
    out = np.empty_like(x)
    lib().oracle_layernorm(_p(out), _p(x), _p(w), _p(b), x.size, eps)
    return out


def silu(x: float) -> float:
    return float(lib().oracle_silu(x))


def gelu(x: float) -> float:
    return float(lib().oracle_gelu(x))


def softmax(x) -> np.ndarray:
    x = f32a(x).copy()
    lib().oracle_softmax_inplace(_p(x), x.size)
    return x


def add_inplace(a, b) -> np.ndarray:
    a, b = f32a(a).copy(), f32a(b)
    lib().oracle_add_inplace(_p(a), _p(b), a.size)
    return a


def mul_inplace(a, b) -> np.ndarray:
    a, b = f32a(a).copy(), f32a(b)
    lib().oracle_mul_inplace(_p(a), _p(b), a.size)
    return a


# ---- sampler -----------------------------------------------------------------

def argmax(logits) -> int:
    l = f32a(logits)
    return int(lib().oracle_argmax(_p(l), l.size))


def value_norms(wo, vals, hidden: int, nh: int, nkv: int, hd: int, t0: int, t1: int) -> np.ndarray:
    """ValueNorms::sync for one layer (attribution.rs:116-148): [t1 - t0, nh]."""
    w = f32a(wo)
    v = f32a(vals)
    out = np.zeros((t1 - t0, nh), dtype=np.float32)
    lib().oracle_value_norms(_p(w), _p(v), hidden, nh, nkv, hd, t0, t1, _p(out))
    return out


def softmax_with_temperature(logits, t) -> np.ndarray:
    l = f32a(logits)
    out = np.empty_like(l)
    lib().oracle_softmax_with_temperature(_p(l), l.size, t, _p(out))
    return out


def unit_f32(word: int) -> float:
    return float(lib().oracle_unit_f32(word & 0xFFFFFFFF))


def sample_token(logits, t: float, word: int) -> int:
    l = f32a(logits)
    return int(lib().oracle_sample_token(_p(l), l.size, t, word & 0xFFFFFFFF))


def sample_margin(logits, t: float, word: int):
    """(token, margin): sample_token at T > 0 and the distance of the draw
    from the chosen token's CDF edges, in the reference's float arithmetic."""
    l = f32a(logits)
    m = ctypes.c_float()
    tok = int(lib().oracle_sample_margin(_p(l), l.size, t, word & 0xFFFFFFFF, ctypes.byref(m)))
    return tok, float(m.value)


def sample_terms(p, word: int):
    """(index, total): sampler.rs:58-108 on un-normalised terms p."""
    a = f32a(p)
    tot = ctypes.c_float()
    tok = int(lib().oracle_sample_terms(_p(a), a.size, word & 0xFFFFFFFF, ctypes.byref(tot)))
    return tok, np.float32(tot.value)


def expf(x) -> np.ndarray:
    """The reference's f32::exp (libm expf) elementwise."""
    a = f32a(x)
    out = np.empty_like(a)
    lib().oracle_expf_array(_p(a), _p(out), a.size)
    return out


# ---- rng -----------------------------------------------------------------------

def chacha_block(key_words: Sequence[int], counter: int, stream: int, rounds: int) -> list:
    k = np.asarray(key_words, dtype=np.uint32)
    out = np.empty(16, dtype=np.uint32)
    lib().oracle_chacha_block(_p(k), counter, stream, rounds, _p(out))
    return [int(x) for x in out]


def seed_from_u64(seed: int) -> bytes:
    out = np.empty(32, dtype=np.uint8)
    lib().oracle_seed_from_u64(seed, _p(out))
    return out.tobytes()


def chacha8_word(seed: bytes, index: int) -> int:
    s = np.frombuffer(seed, dtype=np.uint8).copy()
    return int(lib().oracle_chacha8_word(_p(s), index))


# ---- model -----------------------------------------------------------------------

class OracleModel:
    """Model (model.rs:271-363) over borrowed host tensors."""

    def __init__(self, cfg: dict, tensors: Sequence[np.ndarray]):
        self.cfg = OracleConfig.from_dict(cfg)
        self._keep = [f32a(t) for t in tensors]
        ptrs = (ctypes.c_void_p * len(self._keep))(*[t.ctypes.data for t in self._keep])
        self._h = lib().oracle_model_create(ctypes.byref(self.cfg), ptrs, len(self._keep))
        if not self._h:
            raise ValueError("oracle_model_create rejected the config or tensor count")

    def __del__(self):
        if getattr(self, "_h", None):
            lib().oracle_model_destroy(self._h)
            self._h = None

    def new_cache(self) -> "OracleCache":
        return OracleCache(self)

    def forward(self, token: int, cache: "OracleCache", masked: Sequence[int] = (),
                trace: bool = False):
        V = self.cfg.vocab_size
        logits = np.empty(V, dtype=np.float32)
        m = np.asarray(masked, dtype=np.uint32) if len(masked) else None
        pos = len(cache)
        tr = (np.empty((self.cfg.num_layers, self.cfg.num_heads, pos + 1), dtype=np.float32)
              if trace else None)
        rc = lib().oracle_forward_ext(self._h, cache._h, token, _p(m), 0 if m is None else len(m),
                                      _p(logits), _p(tr))
        if rc:
            raise ValueError(f"oracle forward error {rc}")
        return (logits, tr) if trace else logits

    def generate(self, cache, seed: bytes, temperature: float, prompt, n_gen: int):
        p = np.asarray(prompt, dtype=np.uint32)
        out = np.zeros(max(n_gen, 1), dtype=np.uint32)
        last = np.empty(self.cfg.vocab_size, dtype=np.float32)
        s = np.frombuffer(seed, dtype=np.uint8).copy()
        words = lib().oracle_generate(self._h, cache._h, _p(s), temperature, _p(p), p.size, n_gen,
                                      _p(out), _p(last))
        if words < 0:
            raise ValueError(f"oracle generate error {words}")
        return [int(x) for x in out[:n_gen]], int(words), last

    def checkout(self, cache, seed: bytes, temperature: float, history, prompt_len: int):
        h = np.asarray(history, dtype=np.uint32)
        s = np.frombuffer(seed, dtype=np.uint8).copy()
        sd = ctypes.c_uint32(0)
        last = np.empty(self.cfg.vocab_size, dtype=np.float32)
        r = lib().oracle_checkout(self._h, cache._h, _p(s), temperature, _p(h), h.size, prompt_len,
                                  ctypes.byref(sd), _p(last))
        if r < -1:
            raise ValueError(f"oracle checkout error {r}")
        return int(r), int(sd.value), last


class OracleCache:
    def __init__(self, model: OracleModel):
        self.model = model
        self._h = lib().oracle_cache_create(model._h)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().oracle_cache_destroy(self._h)
            self._h = None

    def __len__(self) -> int:
        return int(lib().oracle_cache_len(self._h))

    def truncate(self, n: int) -> None:
        lib().oracle_cache_truncate(self._h, n)

    def read(self, layer: int):
        c = self.model.cfg
        kvd = c.num_kv_heads * c.head_dim
        n = len(self)
        k = np.empty((n, kvd), dtype=np.float32)
        v = np.empty((n, kvd), dtype=np.float32)
        lib().oracle_cache_read(self._h, layer, _p(k), _p(v))
        return k, v
