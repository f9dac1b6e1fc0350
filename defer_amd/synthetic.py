"""Synthetic Llama-shaped models and inputs.

The reference ships one fixture generator (synthetic.rs:12-59: uniform
weights from a ChaCha8 stream, byte-tokenizer vocabulary). The benchmark
shapes here use a different, documented initialisation:

* every matrix and the embedding: N(0, 0.02) float32. Tensor i of the
  canonical order (model.rs:322-347) draws from its own stream,
  ``numpy.random.Generator(PCG64(SeedSequence(seed).spawn(n)[i]))``, via
  ``standard_normal(dtype=float32) * float32(0.02)``;
* RMSNorm weights: 1.0 (synthetic.rs:44, 49, 54);
* prompts: token ids uniform in [0, V) from ``Generator(PCG64(seed))``.

Shapes are named by what they are; ``CONFIGS`` maps each to the reference's
config fields (model.rs:23-39).
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from typing import List

import numpy as np


def _cfg(vocab, hidden, inter, layers, heads, kv_heads, head_dim, theta, tied, max_seq=8192,
         eps=1e-5, act=0, bias=0):
    return {
        "vocab_size": vocab,
        "hidden_size": hidden,
        "intermediate_size": inter,
        "num_layers": layers,
        "num_heads": heads,
        "num_kv_heads": kv_heads,
        "head_dim": head_dim,
        "rms_norm_eps": eps,
        "rope_theta": theta,
        "max_seq_len": max_seq,
        "tie_word_embeddings": 1 if tied else 0,
        "activation": act,
        "has_bias": bias,
    }


CONFIGS = {
    # synthetic.rs:12-29 (the reference's test model; untied, theta 1e4)
    "tiny": _cfg(256, 64, 160, 2, 4, 2, 16, 10000.0, False, max_seq=1024),
    "smollm2-135m": _cfg(49152, 576, 1536, 30, 9, 3, 64, 100000.0, True),
    "smollm2-360m": _cfg(49152, 960, 2560, 32, 15, 5, 64, 100000.0, True),
    "llama-3.2-1b": _cfg(128256, 2048, 8192, 16, 32, 8, 64, 500000.0, True),
    "llama-3-8b": _cfg(128256, 4096, 14336, 32, 32, 8, 128, 500000.0, False),
}


def tensor_specs(cfg: dict) -> List[tuple]:
    """(name, shape, is_norm) in the canonical order of model.rs:322-347."""
    h, V, ff = cfg["hidden_size"], cfg["vocab_size"], cfg["intermediate_size"]
    q = cfg["num_heads"] * cfg["head_dim"]
    kv = cfg["num_kv_heads"] * cfg["head_dim"]
    specs = [("model.embed_tokens.weight", (V, h), False)]
    for i in range(cfg["num_layers"]):
        p = f"model.layers.{i}"
        specs.append((f"{p}.input_layernorm.weight", (h,), True))
        specs.append((f"{p}.self_attn.q_proj.weight", (q, h), False))
        if cfg["has_bias"]:
            specs.append((f"{p}.self_attn.q_proj.bias", (q,), False))
        specs.append((f"{p}.self_attn.k_proj.weight", (kv, h), False))
        if cfg["has_bias"]:
            specs.append((f"{p}.self_attn.k_proj.bias", (kv,), False))
        specs.append((f"{p}.self_attn.v_proj.weight", (kv, h), False))
        if cfg["has_bias"]:
            specs.append((f"{p}.self_attn.v_proj.bias", (kv,), False))
        specs.append((f"{p}.self_attn.o_proj.weight", (h, q), False))
        specs.append((f"{p}.post_attention_layernorm.weight", (h,), True))
        specs.append((f"{p}.mlp.gate_proj.weight", (ff, h), False))
        specs.append((f"{p}.mlp.up_proj.weight", (ff, h), False))
        specs.append((f"{p}.mlp.down_proj.weight", (h, ff), False))
    specs.append(("model.norm.weight", (h,), True))
    if not cfg["tie_word_embeddings"]:
        specs.append(("lm_head.weight", (V, h), False))
    return specs


def make_weights(cfg: dict, seed: int = 0, std: float = 0.02, threads: int = 8) -> List[np.ndarray]:
    """N(std) matrices, unit norms; deterministic for (cfg, seed)."""
    specs = tensor_specs(cfg)
    children = np.random.SeedSequence(seed).spawn(len(specs))
    scale = np.float32(std)

    def one(i: int) -> np.ndarray:
        _, shape, is_norm = specs[i]
        if is_norm:
            return np.ones(shape, dtype=np.float32)
        g = np.random.Generator(np.random.PCG64(children[i]))
        a = g.standard_normal(size=shape, dtype=np.float32)
        a *= scale
        return a

    with ThreadPoolExecutor(max_workers=threads) as ex:
        return list(ex.map(one, range(len(specs))))


def make_prompt(vocab: int, n: int, seed: int) -> np.ndarray:
    """n token ids uniform in [0, vocab)."""
    g = np.random.Generator(np.random.PCG64(seed))
    return g.integers(0, vocab, size=n, dtype=np.uint32)


def weight_bytes_streamed(cfg: dict) -> int:
    """f32 bytes one token streams: every matrix once, the lm_head (or the
    tied embedding) once, norms once; the embedding row gather is h floats."""
    h, V, ff = cfg["hidden_size"], cfg["vocab_size"], cfg["intermediate_size"]
    q = cfg["num_heads"] * cfg["head_dim"]
    kv = cfg["num_kv_heads"] * cfg["head_dim"]
    per_layer = (q + 2 * kv) * h + h * q + 3 * ff * h + 2 * h
    if cfg["has_bias"]:
        per_layer += q + 2 * kv
    total = cfg["num_layers"] * per_layer + V * h + h + h
    return 4 * total
