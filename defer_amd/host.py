"""ctypes binding of the C++ host side in include/defer_host.h (libdefer_host.so).

``Session`` mirrors the reference's ``Session`` (engine.rs:23-137, 241-274)
on the device path; ``Wal`` its write-ahead log (wal.rs:8-255); the free
functions its ChaCha8 word source and hashes. Like ``defer_amd.gpu``, this
module raises if the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence, Tuple

import numpy as np

from . import gpu

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdefer_host.so")

OK = 0
E_INVALID = 1
E_IO = 2
E_WAL = 3
E_CHECKPOINT = 4
E_DIVERGENCE = 5
E_GPU = 6
E_MODEL = 7


class DeferHostError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"defer_host error {code}: {msg}")
        self.code = code


class Divergence(DeferHostError):
    """DeferError::Divergence (error.rs): replay re-sampled another token."""


class WalHeader(ctypes.Structure):
    _fields_ = [
        ("model_signature", ctypes.c_uint8 * 32),
        ("base_seed", ctypes.c_uint8 * 32),
        ("temperature", ctypes.c_float),
        ("prompt_len", ctypes.c_uint32),
        ("start_rng_word_pos", ctypes.c_uint64),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it first (defer_amd/build.py)")
    gpu.lib()  # the host library links against libdefer_gpu.so
    L = ctypes.CDLL(LIB_PATH)
    u8p, u32, u64, sz, vp, f32 = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t,
                                  ctypes.c_void_p, ctypes.c_float)
    P = ctypes.POINTER
    L.defer_host_last_error.restype = ctypes.c_char_p
    L.defer_host_crc32.argtypes = [u8p, sz]
    L.defer_host_crc32.restype = u32
    L.defer_host_sha256.argtypes = [u8p, sz, u8p]
    L.defer_host_sha256.restype = None
    L.defer_host_cache_fingerprint.argtypes = [vp, u8p]
    L.defer_host_cache_fingerprint.restype = ctypes.c_int
    L.defer_host_seed_from_u64.argtypes = [u64, u8p]
    L.defer_host_seed_from_u64.restype = None
    L.defer_host_chacha8_words.argtypes = [u8p, u64, sz, vp]
    L.defer_host_chacha8_words.restype = None
    L.defer_host_words_per_sample.argtypes = [f32]
    L.defer_host_words_per_sample.restype = u32
    L.defer_host_wal_create.argtypes = [ctypes.c_char_p, P(WalHeader), vp, sz, ctypes.c_int, P(vp)]
    L.defer_host_wal_resume.argtypes = [ctypes.c_char_p, ctypes.c_int, P(vp)]
    L.defer_host_wal_append.argtypes = [vp, u32, u64]
    L.defer_host_wal_next_step.argtypes = [vp]
    L.defer_host_wal_next_step.restype = u32
    L.defer_host_wal_close.argtypes = [vp]
    L.defer_host_wal_close.restype = None
    L.defer_host_wal_read.argtypes = [ctypes.c_char_p, P(WalHeader), vp, P(sz), P(u64), P(ctypes.c_int)]
    L.defer_host_session_create.argtypes = [vp, u8p, f32, u32, P(vp)]
    L.defer_host_session_destroy.argtypes = [vp]
    L.defer_host_session_destroy.restype = None
    L.defer_host_session_prompt.argtypes = [vp, vp, sz]
    L.defer_host_session_step.argtypes = [vp, P(u32)]
    L.defer_host_session_generate.argtypes = [vp, u32, vp, sz, vp, P(u32)]
    L.defer_host_session_generate_logged.argtypes = [vp, u32, vp, sz, vp, vp, P(u32)]
    L.defer_host_session_history.argtypes = [vp, vp]
    L.defer_host_session_history.restype = sz
    L.defer_host_session_prompt_len.argtypes = [vp]
    L.defer_host_session_prompt_len.restype = u32
    L.defer_host_session_rng_word_pos.argtypes = [vp]
    L.defer_host_session_rng_word_pos.restype = u64
    L.defer_host_session_cache.argtypes = [vp]
    L.defer_host_session_cache.restype = vp
    L.defer_host_session_checkout.argtypes = [vp, u8p, f32, vp, sz, u32, u64, u32, P(vp)]
    L.defer_host_checkpoint_save.argtypes = [ctypes.c_char_p, P(WalHeader), vp, sz]
    L.defer_host_checkpoint_load.argtypes = [ctypes.c_char_p, P(WalHeader), vp, P(sz)]
    L.defer_host_session_checkpoint.argtypes = [vp, u8p, P(WalHeader)]
    L.defer_host_session_checkout_file.argtypes = [vp, u8p, ctypes.c_char_p, u32, P(vp)]
    L.defer_host_st_open.argtypes = [ctypes.c_char_p, P(vp)]
    L.defer_host_st_close.argtypes = [vp]
    L.defer_host_st_close.restype = None
    L.defer_host_st_count.argtypes = [vp]
    L.defer_host_st_count.restype = sz
    L.defer_host_st_name.argtypes = [vp, sz]
    L.defer_host_st_name.restype = ctypes.c_char_p
    L.defer_host_st_shape.argtypes = [vp, sz, P(u64), sz]
    L.defer_host_st_shape.restype = sz
    L.defer_host_st_data.argtypes = [vp, sz, P(sz)]
    L.defer_host_st_data.restype = ctypes.POINTER(ctypes.c_float)
    L.defer_host_st_meta.argtypes = [vp, ctypes.c_char_p]
    L.defer_host_st_meta.restype = ctypes.c_char_p
    L.defer_host_st_signature.argtypes = [vp, u8p]
    L.defer_host_st_signature.restype = None
    L.defer_host_model_load.argtypes = [ctypes.c_char_p, u32, P(vp), vp, u8p]
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != OK:
        msg = lib().defer_host_last_error().decode(errors="replace")
        raise (Divergence if rc == E_DIVERGENCE else DeferHostError)(rc, msg)


def _buf(b: bytes):
    return ctypes.c_char_p(b)


def crc32(data: bytes) -> int:
    return int(lib().defer_host_crc32(_buf(data), len(data)))


def sha256(data: bytes) -> bytes:
    out = ctypes.create_string_buffer(32)
    lib().defer_host_sha256(_buf(data), len(data), out)
    return out.raw


def cache_fingerprint(cache: "gpu.GpuCache") -> bytes:
    """KvCache::fingerprint (model.rs:233-242) of a device cache: SHA-256 of
    len (u64 LE), then per layer all keys, then all values (f32 LE bits)."""
    out = (ctypes.c_uint8 * 32)()
    _check(lib().defer_host_cache_fingerprint(cache._h, out))
    return bytes(out)


def seed_from_u64(seed: int) -> bytes:
    out = ctypes.create_string_buffer(32)
    lib().defer_host_seed_from_u64(int(seed), out)
    return out.raw


def chacha8_words(seed: bytes, word_pos: int, n: int) -> np.ndarray:
    assert len(seed) == 32
    out = np.zeros(n, dtype=np.uint32)
    lib().defer_host_chacha8_words(_buf(seed), int(word_pos), int(n), out.ctypes.data)
    return out


def words_per_sample(temperature: float) -> int:
    return int(lib().defer_host_words_per_sample(float(temperature)))


def _header(signature: bytes, seed: bytes, temperature: float, prompt_len: int,
            start_rng: int) -> WalHeader:
    h = WalHeader()
    h.model_signature[:] = list(signature)
    h.base_seed[:] = list(seed)
    h.temperature = temperature
    h.prompt_len = prompt_len
    h.start_rng_word_pos = start_rng
    return h


class Wal:
    """WalWriter (wal.rs:199-235)."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def create(cls, path: str, signature: bytes, seed: bytes, temperature: float, prompt_len: int,
               start_rng: int, prefix: Sequence[int], durable: bool = False) -> "Wal":
        h = _header(signature, seed, temperature, prompt_len, start_rng)
        p = np.ascontiguousarray(np.asarray(prefix, dtype=np.uint32))
        out = ctypes.c_void_p()
        _check(lib().defer_host_wal_create(path.encode(), ctypes.byref(h), p.ctypes.data, len(p),
                                           int(durable), ctypes.byref(out)))
        return cls(out)

    @classmethod
    def resume(cls, path: str, durable: bool = False) -> "Wal":
        out = ctypes.c_void_p()
        _check(lib().defer_host_wal_resume(path.encode(), int(durable), ctypes.byref(out)))
        return cls(out)

    def append(self, token: int, rng_word_pos: int) -> None:
        _check(lib().defer_host_wal_append(self._h, int(token), int(rng_word_pos)))

    @property
    def next_step(self) -> int:
        return int(lib().defer_host_wal_next_step(self._h))

    def close(self) -> None:
        if self._h:
            lib().defer_host_wal_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def read(path: str) -> dict:
        """WalLog::parse + to_checkpoint: header fields, history, rng position, torn flag."""
        h = WalHeader()
        n = ctypes.c_size_t(0)
        _check(lib().defer_host_wal_read(path.encode(), ctypes.byref(h), None, ctypes.byref(n), None, None))
        hist = np.zeros(max(n.value, 1), dtype=np.uint32)
        rng = ctypes.c_uint64()
        torn = ctypes.c_int()
        _check(lib().defer_host_wal_read(path.encode(), ctypes.byref(h), hist.ctypes.data,
                                         ctypes.byref(n), ctypes.byref(rng), ctypes.byref(torn)))
        return {
            "model_signature": bytes(h.model_signature),
            "base_seed": bytes(h.base_seed),
            "temperature": float(h.temperature),
            "prompt_len": int(h.prompt_len),
            "start_rng_word_pos": int(h.start_rng_word_pos),
            "history": [int(x) for x in hist[: n.value]],
            "rng_word_pos": int(rng.value),
            "torn_tail": bool(torn.value),
        }


def read_safetensors(path: str) -> dict:
    """SafeTensors::load (safetensors.rs:142-237) through the C++ reader:
    {"names": [...on-disk order], "tensors": {name: f32 array}, "metadata":
    {...} for the keys asked, "signature": SHA-256 of the file}."""
    h = ctypes.c_void_p()
    _check(lib().defer_host_st_open(path.encode(), ctypes.byref(h)))
    try:
        names, tensors = [], {}
        for i in range(lib().defer_host_st_count(h)):
            name = lib().defer_host_st_name(h, i).decode()
            dims = (ctypes.c_uint64 * 8)()
            rank = lib().defer_host_st_shape(h, i, dims, 8)
            n = ctypes.c_size_t()
            ptr = lib().defer_host_st_data(h, i, ctypes.byref(n))
            arr = np.ctypeslib.as_array(ptr, shape=(n.value,)).copy() if n.value else np.zeros(0, np.float32)
            tensors[name] = arr.reshape([int(dims[k]) for k in range(rank)])
            names.append(name)
        sig = (ctypes.c_uint8 * 32)()
        lib().defer_host_st_signature(h, sig)
        meta = lib().defer_host_st_meta(h, b"defer.config")
        return {"names": names, "tensors": tensors, "signature": bytes(sig),
                "defer.config": meta.decode() if meta else None}
    finally:
        lib().defer_host_st_close(h)


def load_model(path: str, max_seq_len: int = 0):
    """Model::load (model.rs:285-298): (GpuModel, config dict, signature)."""
    from . import gpu

    h = ctypes.c_void_p()
    cfg = gpu.Config()
    sig = (ctypes.c_uint8 * 32)()
    _check(lib().defer_host_model_load(path.encode(), int(max_seq_len), ctypes.byref(h),
                                       ctypes.byref(cfg), sig))
    m = gpu.GpuModel.__new__(gpu.GpuModel)
    m.cfg = cfg
    m._h = h
    return m, cfg.to_dict(), bytes(sig)


class Checkpoint:
    """DeferCheckpoint files (checkpoint.rs:4-136). The header struct has the
    WAL header's layout (signature, seed, temperature, prompt_len, u64 word
    position)."""

    @staticmethod
    def save(path: str, signature: bytes, seed: bytes, temperature: float, prompt_len: int,
             rng_word_pos: int, history: Sequence[int]) -> None:
        h = _header(signature, seed, temperature, prompt_len, rng_word_pos)
        t = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
        _check(lib().defer_host_checkpoint_save(path.encode(), ctypes.byref(h),
                                                t.ctypes.data if len(t) else None, len(t)))

    @staticmethod
    def load(path: str) -> dict:
        h = WalHeader()
        n = ctypes.c_size_t(0)
        _check(lib().defer_host_checkpoint_load(path.encode(), ctypes.byref(h), None, ctypes.byref(n)))
        hist = np.zeros(max(n.value, 1), dtype=np.uint32)
        _check(lib().defer_host_checkpoint_load(path.encode(), ctypes.byref(h), hist.ctypes.data,
                                                ctypes.byref(n)))
        return {
            "model_signature": bytes(h.model_signature),
            "base_seed": bytes(h.base_seed),
            "temperature": float(h.temperature),
            "prompt_len": int(h.prompt_len),
            "rng_word_pos": int(h.start_rng_word_pos),
            "history": [int(x) for x in hist[: n.value]],
        }


class Session:
    """Session (engine.rs:23-137) driving the device path."""

    def __init__(self, model: "gpu.GpuModel", seed: bytes, temperature: float, capacity: int = 0,
                 _handle=None):
        self.model = model
        if _handle is not None:
            self._h = _handle
            return
        out = ctypes.c_void_p()
        _check(lib().defer_host_session_create(model._h, _buf(seed), float(temperature),
                                               int(capacity), ctypes.byref(out)))
        self._h = out

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().defer_host_session_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prompt(self, tokens: Sequence[int]) -> None:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        _check(lib().defer_host_session_prompt(self._h, t.ctypes.data, len(t)))

    def step(self) -> int:
        out = ctypes.c_uint32()
        _check(lib().defer_host_session_step(self._h, ctypes.byref(out)))
        return int(out.value)

    def generate(self, max_tokens: int, stop: Sequence[int] = (), wal: Optional["Wal"] = None) -> list:
        """Session::generate; with `wal`, each token's record is appended and
        flushed as the device commits it (defer_host_session_generate_logged)."""
        s = np.ascontiguousarray(np.asarray(stop, dtype=np.uint32))
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        n = ctypes.c_uint32()
        sp = s.ctypes.data if len(s) else None
        if wal is None:
            rc = lib().defer_host_session_generate(self._h, int(max_tokens), sp, len(s),
                                                   out.ctypes.data, ctypes.byref(n))
        else:
            rc = lib().defer_host_session_generate_logged(self._h, int(max_tokens), sp, len(s),
                                                          wal._h, out.ctypes.data, ctypes.byref(n))
        self.last_n = int(n.value)
        _check(rc)
        return [int(x) for x in out[: n.value]]

    @property
    def history(self) -> list:
        n = lib().defer_host_session_history(self._h, None)
        out = np.zeros(max(n, 1), dtype=np.uint32)
        lib().defer_host_session_history(self._h, out.ctypes.data)
        return [int(x) for x in out[:n]]

    @property
    def prompt_len(self) -> int:
        return int(lib().defer_host_session_prompt_len(self._h))

    @property
    def rng_word_pos(self) -> int:
        return int(lib().defer_host_session_rng_word_pos(self._h))

    @property
    def cache(self) -> "gpu.GpuCache":
        """The session's device cache (owned by the session)."""
        c = gpu.GpuCache.__new__(gpu.GpuCache)
        c.model = self.model
        c._h = ctypes.c_void_p(lib().defer_host_session_cache(self._h))
        c.close = lambda: None  # the session destroys it
        return c

    def checkpoint(self, signature: bytes, path: str) -> None:
        """Session::checkpoint (engine.rs:223-232) saved to `path`."""
        h = WalHeader()
        _check(lib().defer_host_session_checkpoint(self._h, _buf(signature), ctypes.byref(h)))
        t = np.ascontiguousarray(np.asarray(self.history, dtype=np.uint32))
        _check(lib().defer_host_checkpoint_save(path.encode(), ctypes.byref(h),
                                                t.ctypes.data if len(t) else None, len(t)))

    @classmethod
    def checkout_file(cls, model: "gpu.GpuModel", signature: bytes, path: str,
                      capacity: int = 0) -> "Session":
        """Session::checkout (engine.rs:241-274) of a checkpoint file."""
        ck = Checkpoint.load(path)
        out = ctypes.c_void_p()
        _check(lib().defer_host_session_checkout_file(model._h, _buf(signature), path.encode(),
                                                      int(capacity), ctypes.byref(out)))
        return cls(model, ck["base_seed"], ck["temperature"], _handle=out)

    @classmethod
    def checkout(cls, model: "gpu.GpuModel", seed: bytes, temperature: float, history: Sequence[int],
                 prompt_len: int, rng_word_pos: int, capacity: int = 0) -> "Session":
        h = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
        out = ctypes.c_void_p()
        _check(lib().defer_host_session_checkout(model._h, _buf(seed), float(temperature), h.ctypes.data,
                                                 len(h), int(prompt_len), int(rng_word_pos), int(capacity),
                                                 ctypes.byref(out)))
        return cls(model, seed, temperature, _handle=out)
