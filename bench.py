#!/usr/bin/env python3
"""Benchmark: verified GPU replay of a 2048-token session, SmolLM2-135M shape, f32.

Workload (the replay/checkout configuration of the headline metric): a
135M-shaped Llama with N(0, 0.02) weights from seed 0; a 512-token prompt of
uniform-random ids; 1536 tokens sampled at temperature 0.7 with seed 7,
generated on the GPU and logged to a write-ahead log. One step is one
checkout of that log: all 2048 positions are rebuilt on the GPU and every
sampled position is re-sampled from its predecessor's logits and compared
with the record. The library runs the checkout through its batched path
(every position's forward as rows of MFMA GEMMs in the one-token reduction
order, the one-token attention and sampler per row), whose results are bit
for bit those of feeding the positions one at a time: the first step's
rebuilt cache and logits must equal the generating session's.

Prints one JSON line. `value` is replayed positions per second with the
weights, the history and the rng words already in HBM / host memory when the
timed region starts. `roofline` prices the dominant kernel class of a step
(by event-timed device time: the GEMMs or the attention), whose launches the
library times with HIP events on its own stream during the first timed step,
against MI355X's dense f32 peak. `config` also carries the token-by-token replay rate (one
persistent-kernel launch, priced against HBM bandwidth) and the batch-1
decode rates. `cpu_baseline` is the single-threaded C restatement of the
reference (the oracle) timed on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

CFG_NAME = "smollm2-135m"
PROMPT_LEN = 512
SAMPLED = 1536
TEMPERATURE = 0.7
SEED = 7
PEAK_GBS = 8000.0
PEAK_F32_TFLOPS = 157.3


def algorithmic_bytes(cfg: dict, weight_bytes: int, first_pos: int, n_pos: int) -> int:
    """Bytes one forward per position must move: every weight once, the
    cached K/V of positions 0..p once per GQA group, the new K/V row, the
    logits."""
    L = cfg["num_layers"]
    kv = cfg["num_kv_heads"] * cfg["head_dim"]
    V = cfg["vocab_size"]
    total = 0
    for p in range(first_pos, first_pos + n_pos):
        total += weight_bytes + 4 * 2 * L * kv * (p + 1) + 4 * 2 * L * kv + 4 * V
    return total


def measured_traffic(profile: str = "k_persistent_replay_135m.md",
                     key: str = "traffic_bytes_per_launch") -> int | None:
    """HBM bytes from a committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE, each scaled by a 1 GiB copy's reading)."""
    p = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith(key + ":"):
            return int(line.split(":")[1])
    return None


def cpu_baseline(cfg: dict, weights, history, budget_s: float = 12.0) -> dict:
    """The oracle (C, one thread) replaying the session's first positions
    until `budget_s` of CPU work is spent."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_py as O

    om = O.OracleModel(cfg, weights)
    cache = om.new_cache()
    n = 0
    t0 = time.perf_counter()
    while n < len(history) and time.perf_counter() - t0 < budget_s:
        om.forward(int(history[n]), cache)
        n += 1
    dt = time.perf_counter() - t0
    cores = os.cpu_count() or 0
    return {
        "value": n / dt,
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": f"oracle replay of positions 0..{n - 1} of the same session "
                  f"(prompt forwards, 1 thread, {dt:.1f} s; host has {cores} cores)",
    }


def c1_decode(model, cfg: dict, H) -> dict:
    """Batch-1 decode of the CPU-runnable configuration: a 32-token prompt,
    128 greedy tokens then 128 at T = 0.7 (seed 42), device time of the two
    generate calls."""
    from defer_amd import synthetic

    prompt = synthetic.make_prompt(cfg["vocab_size"], 32, seed=42)
    model.set_batching(0)
    s = H.Session(model, H.seed_from_u64(42), 0.0, capacity=512)
    s.prompt(prompt)
    s.generate(128)
    ms = model.last_device_ms()
    s.close()
    s = H.Session(model, H.seed_from_u64(42), TEMPERATURE, capacity=512)
    s.prompt(prompt)
    s.generate(128)
    s.generate(128)
    ms += model.last_device_ms()
    s.close()
    model.set_batching(16)
    tok_s = 256 / (ms / 1e3)
    return {"tok_s": round(tok_s, 2), "us": round(1e6 / tok_s, 1)}


def sessions_workload(args) -> int:
    """The many-session configuration: a Llama-3.2-1B-shaped model (16 layers,
    h 2048, 32/8 heads, ff 8192, vocab 128256, tied, N(0,0.02) weights from
    seed 0); 64 sessions, each a 256-token uniform-random prompt (batched
    prefill) then 256 greedy tokens, all 64 sessions stepping together (one
    MFMA GEMM batch per step, each session bit-identical to its batch-1 run).
    One step of the benchmark = one lockstep token for all 64 sessions; value
    = generated tokens per second over the whole job."""
    from defer_amd import gpu as G
    from defer_amd import synthetic

    cfg = synthetic.CONFIGS["llama-3.2-1b"]
    n_sess, n_prompt = 64, 256
    n_gen = args.steps
    model = G.GpuModel(G.Config.from_dict(cfg), synthetic.make_weights(cfg, 0))
    caches = [model.new_cache(n_prompt + n_gen + args.warmup + 1) for _ in range(n_sess)]
    for k, c in enumerate(caches):
        model.prompt(c, synthetic.make_prompt(cfg["vocab_size"], n_prompt, seed=1000 + k))
    for _ in range(args.warmup):
        model.step_batch(caches, 0.0)
    model.set_profiling(True)
    model.batch_stats(reset=True)
    t0 = time.perf_counter()
    for _ in range(n_gen):
        model.step_batch(caches, 0.0)
    dt = time.perf_counter() - t0
    prof = model.batch_stats(reset=True)
    model.set_profiling(False)
    # batch-1 rate of one session on the same model, for comparison
    one = model.new_cache(n_prompt + 64)
    model.set_batching(0)
    model.prompt(one, synthetic.make_prompt(cfg["vocab_size"], n_prompt, seed=1000))
    model.generate(one, 32, 0.0)
    b1_ms = model.last_device_ms()
    model.set_batching(16)
    achieved = prof["gemm_flop"] / (prof["gemm_ms"] / 1e3) / 1e12
    line = {
        "metric": "many-session lockstep decode tok/s (f32)",
        "value": round(n_sess * n_gen / dt, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": n_gen,
        "warmup": args.warmup,
        "ms_per_step": round(dt / n_gen * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,0.02) weights from seed 0, uniform-random prompt ids)",
        "config": {
            "workload": "Llama-3.2-1B-shaped model, 64 sessions x (256-token prompt + greedy "
                        "tokens), all sessions stepping together",
            "sessions": n_sess,
            "gemm_ms_per_step": round(prof["gemm_ms"] / n_gen, 3),
            "attention_ms_per_step": round(prof["attn_ms"] / n_gen, 3),
            "batch1_decode_tok_s": round(32 / (b1_ms / 1e3), 2),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "k_gemm (MFMA f32 GEMMs)",
            "achieved": round(achieved, 3),
            "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F32_TFLOPS, 4),
            "traffic": None,
        },
    }
    for c in caches:
        c.close()
    one.close()
    model.close()
    print(json.dumps(line), flush=True)
    return 0


def c1_workload(args) -> int:
    """Batch-1 decode of the CPU-runnable configuration alone (c1_decode: a
    32-token prompt, 128 greedy tokens, then 128 at T = 0.7; positions 32..288
    timed); roofline = the persistent kernel's algorithmic bytes over the
    device time of the two timed generate calls."""
    from defer_amd import gpu as G
    from defer_amd import host as H
    from defer_amd import synthetic

    cfg = synthetic.CONFIGS[CFG_NAME]
    model = G.GpuModel(G.Config.from_dict(cfg), synthetic.make_weights(cfg, 0))
    c1 = c1_decode(model, cfg, H)
    ms = 256 / c1["tok_s"] * 1e3
    wbytes = synthetic.weight_bytes_streamed(cfg)
    achieved = algorithmic_bytes(cfg, wbytes, 32, 256) / (ms / 1e3) / 1e9
    line = {
        "metric": "batch-1 decode tok/s (f32) + achieved HBM GB/s as % of peak",
        "value": c1["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": 256,
        "warmup": 0,
        "ms_per_step": round(ms / 256, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,0.02) weights from seed 0, uniform-random prompt ids)",
        "config": {
            "workload": "SmolLM2-135M-shaped decode: 32-token prompt, 128 greedy tokens, then "
                        "128 at T=0.7 (seed 42), one token at a time",
            "weight_bytes_per_token": wbytes,
            "weight_roofline_tok_s": round(PEAK_GBS * 1e9 / wbytes, 1),
            "weight_roofline_frac": round(c1["tok_s"] * wbytes / (PEAK_GBS * 1e9), 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_persistent",
            "achieved": round(achieved, 2),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": None,
        },
    }
    model.close()
    print(json.dumps(line), flush=True)
    return 0


def decode_workload(args, name: str) -> int:
    """Batch-1 decode of the long-context (SmolLM2-360M shape: 128-token prompt,
    4096 tokens at T=0.8, seed 1) or the large-model configuration
    (Llama-3-8B shape, 32 GB of weights: 64-token prompt, 512 greedy tokens).
    value = decoded tokens per second (device time of the generate call);
    roofline = the persistent kernel's algorithmic bytes over that time."""
    from defer_amd import gpu as G
    from defer_amd import host as H
    from defer_amd import synthetic

    if name == "long":
        cfg_name, n_prompt, n_gen, T, seed = "smollm2-360m", 128, 4096, 0.8, 1
    else:
        cfg_name, n_prompt, n_gen, T, seed = "llama-3-8b", 64, 512, 0.0, 0
    cfg = synthetic.CONFIGS[cfg_name]
    t0 = time.perf_counter()
    model = G.GpuModel(G.Config.from_dict(cfg), synthetic.make_weights(cfg, 0))
    setup_s = time.perf_counter() - t0
    s = H.Session(model, H.seed_from_u64(seed), T, capacity=n_prompt + n_gen)
    s.prompt(synthetic.make_prompt(cfg["vocab_size"], n_prompt, seed=seed))
    toks = s.generate(n_gen)
    ms = model.last_device_ms()
    assert len(toks) == n_gen
    wbytes = synthetic.weight_bytes_streamed(cfg)
    algo = algorithmic_bytes(cfg, wbytes, n_prompt, n_gen)
    achieved = algo / (ms / 1e3) / 1e9
    line = {
        "metric": "batch-1 decode tok/s (f32) + achieved HBM GB/s as % of peak",
        "value": round(n_gen / (ms / 1e3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": n_gen,
        "warmup": 0,
        "ms_per_step": round(ms / n_gen, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,0.02) weights from seed 0, uniform-random prompt ids)",
        "config": {
            "workload": f"{cfg_name}-shaped decode: {n_prompt}-token prompt + {n_gen} tokens at "
                        f"T={T}, seed {seed}, one token at a time",
            "weight_bytes_per_token": wbytes,
            "weight_roofline_tok_s": round(PEAK_GBS * 1e9 / wbytes, 1),
            "weight_roofline_frac": round(n_gen / (ms / 1e3) * wbytes / (PEAK_GBS * 1e9), 4),
            "setup_s": round(setup_s, 1),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_persistent",
            "achieved": round(achieved, 2),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": None,
        },
    }
    s.close()
    model.close()
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=["replay", "sessions", "c1", "long", "8b"],
                    default="replay",
                    help="replay: the 2048-position checkout (default, the headline); "
                         "sessions: 64 Llama-3.2-1B-shaped sessions in lockstep; "
                         "c1: 135M-shaped batch-1 decode of 256 tokens; "
                         "long: 360M-shaped decode of 4096 tokens; 8b: 8B-shaped decode")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device once (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.copy_probe:
        import torch

        n = args.copy_probe * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n * 4}), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported "
              "(the single-GPU path is the whole product: one GPU's share at its real shape)",
              file=sys.stderr)
        return 2

    if args.workload == "sessions":
        return sessions_workload(args)
    if args.workload == "c1":
        return c1_workload(args)
    if args.workload in ("long", "8b"):
        return decode_workload(args, args.workload)

    from defer_amd import gpu as G
    from defer_amd import host as H
    from defer_amd import synthetic

    cfg = synthetic.CONFIGS[CFG_NAME]
    weights = synthetic.make_weights(cfg, 0)
    model = G.GpuModel(G.Config.from_dict(cfg), weights)
    signature = H.sha256(b"".join(w.tobytes() for w in weights))
    seed = H.seed_from_u64(SEED)
    prompt = synthetic.make_prompt(cfg["vocab_size"], PROMPT_LEN, seed=SEED)
    n_pos = PROMPT_LEN + SAMPLED

    # The session, generated on the GPU and logged (untimed setup; its decode
    # rate is reported beside the replay rate). Everything outside the timed
    # replays runs token by token, so every GEMM launch of the run belongs to
    # a replay and a kernel trace of the run prices exactly those.
    live = H.Session(model, seed, TEMPERATURE, capacity=n_pos)
    model.set_batching(0)
    live.prompt(prompt)
    model.set_batching(16)
    toks = live.generate(SAMPLED)
    decode_ms = model.last_device_ms()
    assert len(toks) == SAMPLED
    wal_path = os.path.join(tempfile.mkdtemp(prefix="defer-bench-"), "session.wal")
    wal = H.Wal.create(wal_path, signature, seed, TEMPERATURE, PROMPT_LEN, 0, prompt)
    for i, t in enumerate(toks):
        wal.append(t, (i + 1) * H.words_per_sample(TEMPERATURE))
    wal.close()
    log = H.Wal.read(wal_path)
    assert log["history"] == live.history and not log["torn_tail"]

    def replay():
        return H.Session.checkout(model, log["base_seed"], log["temperature"], log["history"],
                                  log["prompt_len"], log["rng_word_pos"], capacity=n_pos)

    # Token-by-token replay (one persistent launch), timed once beside.
    model.set_batching(0)
    t0 = time.perf_counter()
    replay().close()
    tbt_s = time.perf_counter() - t0
    tbt_dev_s = model.last_device_ms() / 1e3
    model.set_batching(16)

    for _ in range(args.warmup):
        replay().close()
    # HIP events around every GEMM and attention launch of the first timed
    # step (the kernels' event-timed durations); the other steps run without
    # them, since each event pair adds a few microseconds between launches.
    model.set_profiling(True)
    model.batch_stats(reset=True)
    times, dev_ms = [], []
    first = None
    prof = None
    for k in range(args.steps):
        t0 = time.perf_counter()
        s = replay()
        times.append(time.perf_counter() - t0)
        dev_ms.append(model.last_device_ms())
        if prof is None:
            prof = model.batch_stats(reset=True)
            model.set_profiling(False)
        if first is None:
            first = s
        else:
            s.close()
    prof_steps = 1
    # Verification of the first timed step (outside the timed region).
    a, b = first.cache, live.cache
    for layer in range(cfg["num_layers"]):
        for x, y in zip(a.read(layer), b.read(layer)):
            if not np.array_equal(x.view(np.uint32), y.view(np.uint32)):
                raise SystemExit(f"replayed cache differs from the generated one at layer {layer}")
    if not np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32)):
        raise SystemExit("replayed logits differ from the generated session's")
    first.close()

    total_s = sum(times)
    value = args.steps * n_pos / total_s
    wbytes = synthetic.weight_bytes_streamed(cfg)
    algo = algorithmic_bytes(cfg, wbytes, 0, n_pos)
    tbt_gbs = algo / tbt_dev_s / 1e9
    # Dominant kernel class of the batched replay, by event-timed device time.
    cls = "gemm" if prof["gemm_ms"] >= prof["attn_ms"] else "attn"
    k_ms, k_flop, k_n = prof[cls + "_ms"], prof[cls + "_flop"], prof[cls + "_launches"]
    achieved = (k_flop / k_n) / (k_ms / k_n / 1e3) / 1e12
    c1 = c1_decode(model, cfg, H)
    line = {
        "metric": "batch-1 decode tok/s (f32) + achieved HBM GB/s as % of peak; replay tok/s",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_s / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,0.02) weights from seed 0, uniform-random prompt ids)",
        "config": {
            "workload": "SmolLM2-135M-shaped replay: 2048-token session (512 prompt + 1536 sampled "
                        "at T=0.7, seed 7), every position rebuilt and every sampled position "
                        "re-sampled and verified on the GPU (batched path, bit-identical to "
                        "token by token)",
            "positions_per_step": n_pos,
            "replay_device_ms": round(float(np.mean(dev_ms)), 3),
            "gemm_ms_per_step": round(prof["gemm_ms"] / prof_steps, 3),
            "attention_ms_per_step": round(prof["attn_ms"] / prof_steps, 3),
            "event_timed_steps": prof_steps,
            "token_by_token_replay_tok_s": round(n_pos / tbt_s, 2),
            "token_by_token_replay_hbm_gbs": round(tbt_gbs, 2),
            "token_by_token_replay_hbm_frac": round(tbt_gbs / PEAK_GBS, 4),
            "token_by_token_replay_traffic": measured_traffic(),
            "decode_tok_s_ctx_512_2048": round(SAMPLED / (decode_ms / 1e3), 2),
            "c1_decode_tok_s": c1["tok_s"],
            "c1_decode_us_per_token": c1["us"],
            "c1_weight_roofline_frac": round(c1["tok_s"] * wbytes / (PEAK_GBS * 1e9), 4),
            "weight_roofline_tok_s": round(PEAK_GBS * 1e9 / wbytes, 1),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "k_gemm (MFMA f32 GEMMs)" if cls == "gemm" else "k_b_attn (attention items)",
            "achieved": round(achieved, 3),
            "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F32_TFLOPS, 4),
            # HBM bytes of one replay's k_gemm launches (PMC, committed profile)
            "traffic": (measured_traffic("k_gemm_replay_135m.md", "gemm_traffic_bytes_per_replay")
                        if cls == "gemm" else None),
        },
    }
    # Device objects are released here, not during interpreter shutdown.
    live.close()
    model.close()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, weights, log["history"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    rc = main()
    if rc:
        sys.exit(rc)
