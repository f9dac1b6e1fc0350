#!/usr/bin/env python3
"""Writes the oracle's results for each benchmark configuration as fixtures.

TEST INFRASTRUCTURE: runs the CPU oracle (oracle/liboracle.so, the C
restatement of the reference's forward pass and sampler) on the synthetic
workloads and stores what the GPU parity tests compare against. Run it in the
build container (the oracle needs minutes to hours of one core per
configuration); the GPU box only reads the `.npz` files.

    python tests/golden/make_fixtures.py c1 c2 c3 c4 c5

Every fixture holds, per sampled step: the token, and how close the choice
was (greedy: the gap between the two largest logits; T > 0: the distance in
probability between the draw r and the nearer edge of the chosen token's CDF
interval, formed in the reference's own float arithmetic), so a test can tell
a real mismatch from a rounding-boundary case. The T > 0 sessions (c1 B, c2,
c3) also hold the argmax and top-2 gap after every fed position, so the GPU
can be teacher-forced along the oracle's history and checked at each one.
Last-position logits are stored as every 8th value plus the 32 largest.

Workloads (weights N(0, 0.02) from seed 0, defer_amd.synthetic):
  c1  135M shape: 32-token prompt (seed 42); session A 128 greedy tokens;
      session B 128 tokens at T = 0.7 with seed 42.
  c2  135M shape: 512-token prompt (seed 7) + 1536 tokens at T = 0.7, seed 7;
      plus the argmax and top-2 gap at every one of the 2048 positions.
  c3  360M shape: 128-token prompt (seed 1) + 4096 tokens at T = 0.8, seed 1,
      with the argmax and gap at all 4224 positions; then 16 greedy tokens
      past position 4224 from the same cache.
  c4  1B shape: session k's 256-token prompt (seed 1000 + k) + 256 greedy
      tokens, for sessions 0 and 63.
  c5  8B shape: 64-token prompt (seed 0) + 512 greedy tokens.
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle_py as O  # noqa: E402
from defer_amd import synthetic  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
STRIDE = 8
TOPK = 32


def top2_gap(logits: np.ndarray) -> float:
    i = int(np.argmax(logits))
    rest = np.delete(logits, i)
    return float(logits[i] - np.max(rest))


def cdf_margin(logits: np.ndarray, T: float, word: int, tok: int) -> float:
    """Distance of the draw r from the edges of token tok's CDF interval, in
    the reference's own arithmetic (sampler.rs:43-109: float32 sequential
    total, normalisation and cumulative sum; oracle_sample_margin), so it is
    >= 0 for the token the oracle chose."""
    got, m = O.sample_margin(logits, T, word)
    assert got == tok
    return m


def logits_summary(prefix: str, logits: np.ndarray) -> dict:
    idx = np.argsort(-logits, kind="stable")[:TOPK].astype(np.uint32)
    return {
        f"{prefix}_logits_strided": logits[::STRIDE].astype(np.float32),
        f"{prefix}_top_idx": idx,
        f"{prefix}_top_val": logits[idx].astype(np.float32),
    }


def run_session(om, prompt, n_gen: int, T: float, seed_u64: int, say, per_position=None):
    """Session::prompt then n_gen steps (engine.rs:62-137) on the oracle,
    with the per-step diagnostics. per_position (a dict, optional) gets the
    argmax and top-2 gap of the logits after every fed position."""
    seed = O.seed_from_u64(seed_u64)
    cache = om.new_cache()
    logits = None
    am, gp = [], []

    def note(lg):
        if per_position is not None:
            am.append(int(np.argmax(lg)))
            gp.append(top2_gap(lg))

    for t in prompt:
        logits = om.forward(int(t), cache)
        note(logits)
    toks, words, close = [], [], []
    t0 = time.time()
    for g in range(n_gen):
        w = O.chacha8_word(seed, g) if T != 0.0 else 0
        tok = O.sample_token(logits, T, w)
        close.append(top2_gap(logits) if T == 0.0 else cdf_margin(logits, T, w, tok))
        toks.append(tok)
        words.append(w)
        logits = om.forward(tok, cache)
        note(logits)
        if g % 64 == 63:
            say(f"  {g + 1}/{n_gen} tokens, {time.time() - t0:.0f} s")
    if per_position is not None:
        per_position["argmax"] = np.asarray(am, np.uint32)
        per_position["gap"] = np.asarray(gp, np.float64)
    return cache, np.asarray(toks, np.uint32), np.asarray(words, np.uint32), \
        np.asarray(close, np.float64), logits


def say_for(name):
    def say(msg):
        print(f"[{name}] {msg}", flush=True)
    return say


def fixture_c1():
    say = say_for("c1")
    cfg = synthetic.CONFIGS["smollm2-135m"]
    om = O.OracleModel(cfg, synthetic.make_weights(cfg, 0))
    prompt = synthetic.make_prompt(cfg["vocab_size"], 32, seed=42)
    out = {"prompt": prompt}
    say("session A: 128 greedy")
    _, ta, _, ga, la = run_session(om, prompt, 128, 0.0, 42, say)
    out.update(greedy_tokens=ta, greedy_gap=ga, **logits_summary("greedy_last", la))
    say("session B: 128 at T=0.7, seed 42")
    pp = {}
    _, tb, wb, mb, lb = run_session(om, prompt, 128, 0.7, 42, say, pp)
    out.update(sampled_tokens=tb, sampled_words=wb, sampled_margin=mb,
               sampled_argmax=pp["argmax"], sampled_gap=pp["gap"],
               **logits_summary("sampled_last", lb))
    return out


def fixture_c2():
    say = say_for("c2")
    cfg = synthetic.CONFIGS["smollm2-135m"]
    om = O.OracleModel(cfg, synthetic.make_weights(cfg, 0))
    prompt = synthetic.make_prompt(cfg["vocab_size"], 512, seed=7)
    seed = O.seed_from_u64(7)
    cache = om.new_cache()
    argmax, gap = [], []
    logits = None
    t0 = time.time()
    for i, t in enumerate(prompt):
        logits = om.forward(int(t), cache)
        argmax.append(int(np.argmax(logits)))
        gap.append(top2_gap(logits))
        if i % 128 == 127:
            say(f"  prompt {i + 1}/512, {time.time() - t0:.0f} s")
    toks, words, margin = [], [], []
    for g in range(1536):
        w = O.chacha8_word(seed, g)
        tok = O.sample_token(logits, 0.7, w)
        margin.append(cdf_margin(logits, 0.7, w, tok))
        toks.append(tok)
        words.append(w)
        logits = om.forward(tok, cache)
        argmax.append(int(np.argmax(logits)))
        gap.append(top2_gap(logits))
        if g % 128 == 127:
            say(f"  sampled {g + 1}/1536, {time.time() - t0:.0f} s")
    return {
        "prompt": prompt, "tokens": np.asarray(toks, np.uint32),
        "words": np.asarray(words, np.uint32), "margin": np.asarray(margin, np.float64),
        "argmax": np.asarray(argmax, np.uint32), "gap": np.asarray(gap, np.float64),
        **logits_summary("last", logits),
    }


def fixture_c3():
    say = say_for("c3")
    cfg = synthetic.CONFIGS["smollm2-360m"]
    om = O.OracleModel(cfg, synthetic.make_weights(cfg, 0))
    prompt = synthetic.make_prompt(cfg["vocab_size"], 128, seed=1)
    say("128 prompt + 4096 at T=0.8, seed 1")
    pp = {}
    cache, toks, words, margin, logits = run_session(om, prompt, 4096, 0.8, 1, say, pp)
    out = {"prompt": prompt, "tokens": toks, "words": words, "margin": margin,
           "argmax": pp["argmax"], "gap": pp["gap"], **logits_summary("sampled_last", logits)}
    say("16 greedy tokens past position 4224")
    tail, gaps = [], []
    for _ in range(16):
        tok = O.argmax(logits)
        gaps.append(top2_gap(logits))
        tail.append(tok)
        logits = om.forward(tok, cache)
    out.update(tail_tokens=np.asarray(tail, np.uint32), tail_gap=np.asarray(gaps, np.float64),
               **logits_summary("tail_last", logits))
    return out


def fixture_c4():
    say = say_for("c4")
    cfg = synthetic.CONFIGS["llama-3.2-1b"]
    om = O.OracleModel(cfg, synthetic.make_weights(cfg, 0))
    out = {}
    for k in (0, 63):
        say(f"session {k}: 256 prompt + 256 greedy")
        prompt = synthetic.make_prompt(cfg["vocab_size"], 256, seed=1000 + k)
        _, t, _, g, lg = run_session(om, prompt, 256, 0.0, 0, say)
        out.update({f"s{k}_prompt": prompt, f"s{k}_tokens": t, f"s{k}_gap": g,
                    **logits_summary(f"s{k}_last", lg)})
    return out


def fixture_c5():
    say = say_for("c5")
    cfg = synthetic.CONFIGS["llama-3-8b"]
    om = O.OracleModel(cfg, synthetic.make_weights(cfg, 0))
    prompt = synthetic.make_prompt(cfg["vocab_size"], 64, seed=0)
    say("64 prompt + 512 greedy")
    _, t, _, g, lg = run_session(om, prompt, 512, 0.0, 0, say)
    return {"prompt": prompt, "tokens": t, "gap": g, **logits_summary("last", lg)}


FIXTURES = {"c1": fixture_c1, "c2": fixture_c2, "c3": fixture_c3, "c4": fixture_c4,
            "c5": fixture_c5}


def main(names):
    for name in names:
        t0 = time.time()
        data = FIXTURES[name]()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"[{name}] wrote {path} ({os.path.getsize(path)} bytes) in {time.time() - t0:.0f} s",
              flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or list(FIXTURES))
