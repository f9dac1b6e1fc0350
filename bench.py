#!/usr/bin/env python3
"""Benchmark: batch-1 f32 decode of a SmolLM2-135M-shaped model on one MI355X.

The default workload is the north-star configuration: a 135M-shaped Llama
(hidden 576, 30 layers, 9/3 heads, head_dim 64, ff 1536, vocab 49152, tied)
with N(0, 0.02) weights from seed 0 and a 32-token uniform-random prompt;
session A generates 128 greedy tokens, session B 128 tokens at T = 0.7 with
seed 42, one token at a time. One step of the benchmark is both sessions:
their prompts are fed untimed (as the reference's `defer run` excludes load
and prompt from its tok/s, main.rs:261-312) and the two generate calls --
256 tokens at positions 32..160 -- are timed on the host clock.

Prints one JSON line. `value` is decoded tokens per second over the K timed
steps. `roofline` prices the persistent decode kernel (`k_persistent`, one
launch per generate call) against the 8 TB/s HBM peak: its algorithmic bytes
(every weight once per token, the cached K/V once per GQA group, the new K/V
row and the logits) over its HIP-event-timed duration on the library's
stream; `traffic` is its HBM bytes per launch from the committed rocprofv3
PMC profile. `config` also carries the weight-streaming roofline fraction and
the replay figures (the 2048-position checkout, batched and token by token).
`cpu_baseline` is the oracle -- the single-threaded C restatement of the
reference's loops -- timed on the same workload, pinned to one core, before
the GPU is touched.

Other workloads (--workload): replay (the 2048-position checkout as its own
line), sessions (64 Llama-3.2-1B-shaped sessions in lockstep), long
(360M-shaped 4096-token decode), 8b (8B-shaped decode).
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
EXEC_MODES = {"persistent": 0, "graph": 1, "eager": 2}
# Per-layer phase kernels in launch order (k_phase's `ph` argument), then
# the final norm + lm_head + logits phase.
PHASES = ("qkv", "attn", "comb", "o", "gate_up", "down")


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


def host_cpu() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_c1(cfg: dict, weights, prompt, budget_s: float = 15.0) -> dict:
    """The oracle (C, one thread, pinned to one core) on the decode workload:
    session A's greedy tokens, then session B's tokens at T = 0.7, prompts
    untimed, until `budget_s` of timed decoding is spent."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_py as O

    om = O.OracleModel(cfg, weights)
    saved = os.sched_getaffinity(0)
    core = min(saved)
    os.sched_setaffinity(0, {core})
    n, spent = 0, 0.0
    try:
        for T, seed in ((0.0, 42), (TEMPERATURE, 42)):
            cache = om.new_cache()
            logits = None
            for t in prompt:
                logits = om.forward(int(t), cache)
            s = O.seed_from_u64(seed)
            t0 = time.perf_counter()
            for g in range(128):
                w = O.chacha8_word(s, g) if T != 0.0 else 0
                tok = O.sample_token(logits, T, w)
                logits = om.forward(tok, cache)
                n += 1
                if time.perf_counter() - t0 + spent > budget_s:
                    break
            spent += time.perf_counter() - t0
            if spent > budget_s:
                break
    finally:
        os.sched_setaffinity(0, saved)
    return {
        "value": round(n / spent, 2),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": f"oracle (C restatement of ops.rs/model.rs/sampler.rs, -O2, no FMA contraction) "
                  f"decoding {n} tokens of the same two sessions from position 32 (greedy, then "
                  f"T=0.7), prompts untimed, {spent:.1f} s on core {core}; host: {host_cpu()}, "
                  f"{os.cpu_count()} logical cores",
    }


def c1_step(model, prompt, H, wal_dir) -> tuple:
    """One step of the decode workload: sessions A (greedy) and B (T = 0.7,
    seed 42), 128 generated tokens each, every token logged to the session's
    WAL as the device commits it (one 29-byte record written and flushed,
    wal.rs:241-250), inside the timed region as `defer run` times its
    generate loop with its appends (main.rs:261-303); the WAL is created
    before, as cmd_run creates it before run_generation. Returns (host
    seconds of the two generate calls, device ms of their two launches as a
    (greedy, sampled) pair, tokens of A, tokens of B)."""
    wall, dev, out = 0.0, [], []
    for k, T in enumerate((0.0, TEMPERATURE)):
        s = H.Session(model, H.seed_from_u64(42), T, capacity=512)
        s.prompt(prompt)
        wal = H.Wal.create(os.path.join(wal_dir, f"session{k}.wal"), bytes(32), H.seed_from_u64(42), T,
                           len(prompt), 0, prompt)
        t0 = time.perf_counter()
        toks = s.generate(128, wal=wal)
        wall += time.perf_counter() - t0
        dev.append(model.last_device_ms())
        wal.close()
        assert len(toks) == 128
        out.append(toks)
        s.close()
    return wall, tuple(dev), out[0], out[1]


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
    n_prof = 4  # untimed steps with HIP events around the GEMMs and attention
    model = G.GpuModel(G.Config.from_dict(cfg), synthetic.make_weights(cfg, 0))
    caches = [model.new_cache(n_prompt + n_gen + args.warmup + n_prof + 1) for _ in range(n_sess)]
    for k, c in enumerate(caches):
        model.prompt(c, synthetic.make_prompt(cfg["vocab_size"], n_prompt, seed=1000 + k))
    for _ in range(args.warmup):
        model.step_batch(caches, 0.0)
    t0 = time.perf_counter()
    for _ in range(n_gen):
        model.step_batch(caches, 0.0)
    dt = time.perf_counter() - t0
    # The GEMM / attention split from separate steps: each event pair adds a
    # few microseconds between launches, which the timed steps do not carry.
    model.set_profiling(True)
    model.batch_stats(reset=True)
    for _ in range(n_prof):
        model.step_batch(caches, 0.0)
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
            "gemm_ms_per_step": round(prof["gemm_ms"] / n_prof, 3),
            "attention_ms_per_step": round(prof["attn_ms"] / n_prof, 3),
            "batch1_decode_tok_s": round(32 / (b1_ms / 1e3), 2),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "k_gemm (MFMA f32 GEMMs)",
            "achieved": round(achieved, 3),
            "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F32_TFLOPS, 4),
            "traffic": measured_traffic("k_gemm_lockstep_1b.md", "gemm_traffic_bytes_per_step"),
        },
    }
    for c in caches:
        c.close()
    one.close()
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
            "traffic": measured_traffic("k_persistent_decode_8b.md" if name == "8b"
                                        else "k_persistent_decode_360m.md"),
        },
    }
    s.close()
    model.close()
    print(json.dumps(line), flush=True)
    return 0


def replay_measure(model, cfg: dict, weights, H, steps: int, warmup: int) -> dict:
    """The replay configuration: a 2048-token session (512 prompt + 1536
    sampled at T=0.7, seed 7) generated on the GPU and logged to a WAL, then
    checked out `steps` times through the batched path (every position
    rebuilt, every sampled position re-sampled and verified; bit-identical to
    the token-by-token path, which is timed once beside). The first timed
    checkout's cache and logits are compared bit for bit with the generating
    session's."""
    n_pos = PROMPT_LEN + SAMPLED
    signature = H.sha256(b"".join(w.tobytes() for w in weights))
    seed = H.seed_from_u64(SEED)
    prompt = synthetic_prompt(cfg, PROMPT_LEN, SEED)
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

    model.set_batching(0)
    t0 = time.perf_counter()
    replay().close()
    tbt_s = time.perf_counter() - t0
    tbt_dev_s = model.last_device_ms() / 1e3
    model.set_batching(16)
    for _ in range(warmup):
        replay().close()
    # One untimed checkout with HIP events around every GEMM and attention
    # launch (each event adds a few microseconds between launches), for the
    # GEMM / attention split; its result is the one compared bit for bit.
    model.set_profiling(True)
    model.batch_stats(reset=True)
    first = replay()
    prof = model.batch_stats(reset=True)
    model.set_profiling(False)
    times, dev_ms = [], []
    for _ in range(steps):
        t0 = time.perf_counter()
        s = replay()
        times.append(time.perf_counter() - t0)
        dev_ms.append(model.last_device_ms())
        s.close()
    a, b = first.cache, live.cache
    for layer in range(cfg["num_layers"]):
        for x, y in zip(a.read(layer), b.read(layer)):
            if not np.array_equal(x.view(np.uint32), y.view(np.uint32)):
                raise SystemExit(f"replayed cache differs from the generated one at layer {layer}")
    if not np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32)):
        raise SystemExit("replayed logits differ from the generated session's")
    first.close()
    live.close()
    wbytes = synthetic_weight_bytes(cfg)
    algo = algorithmic_bytes(cfg, wbytes, 0, n_pos)
    gemm_tflops = prof["gemm_flop"] / (prof["gemm_ms"] / 1e3) / 1e12
    return {
        "replay_positions": n_pos,
        "replay_tok_s": round(steps * n_pos / sum(times), 2),
        "replay_ms": round(sum(times) / steps * 1e3, 3),
        "replay_device_ms": round(float(np.mean(dev_ms)), 3),
        "replay_gemm_ms": round(prof["gemm_ms"], 3),
        "replay_gemm_tflops": round(gemm_tflops, 2),
        "replay_gemm_mfma_frac": round(gemm_tflops / PEAK_F32_TFLOPS, 4),
        "replay_attention_ms": round(prof["attn_ms"], 3),
        "token_by_token_replay_tok_s": round(n_pos / tbt_s, 2),
        "token_by_token_replay_hbm_gbs": round(algo / tbt_dev_s / 1e9, 2),
        "token_by_token_replay_hbm_frac": round(algo / tbt_dev_s / 1e9 / PEAK_GBS, 4),
        "decode_tok_s_ctx_512_2048": round(SAMPLED / (decode_ms / 1e3), 2),
    }


def synthetic_prompt(cfg: dict, n: int, seed: int):
    from defer_amd import synthetic

    return synthetic.make_prompt(cfg["vocab_size"], n, seed=seed)


def synthetic_weight_bytes(cfg: dict) -> int:
    from defer_amd import synthetic

    return synthetic.weight_bytes_streamed(cfg)


def replay_workload(args) -> int:
    """The replay configuration as its own line (value: replayed positions/s)."""
    from defer_amd import gpu as G
    from defer_amd import host as H
    from defer_amd import synthetic

    cfg = synthetic.CONFIGS[CFG_NAME]
    weights = synthetic.make_weights(cfg, 0)
    model = G.GpuModel(G.Config.from_dict(cfg), weights)
    r = replay_measure(model, cfg, weights, H, args.steps, args.warmup)
    model.close()
    line = {
        "metric": "verified replay positions/s (f32), 2048-position checkout",
        "value": r["replay_tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["replay_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,0.02) weights from seed 0, uniform-random prompt ids)",
        "config": {"workload": "SmolLM2-135M-shaped checkout of a 2048-token session (512 prompt "
                               "+ 1536 sampled at T=0.7, seed 7), batched path", **r},
        "roofline": {
            "bound": "mfma",
            "kernel": "k_gemm (MFMA f32 GEMMs)",
            "achieved": r["replay_gemm_tflops"],
            "peak": PEAK_F32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": r["replay_gemm_mfma_frac"],
            "traffic": measured_traffic("k_gemm_replay_135m.md", "gemm_traffic_bytes_per_replay"),
        },
    }
    print(json.dumps(line), flush=True)
    return 0


def _read_csv(d: str, suffix: str) -> list:
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def _pmc_per_dispatch(d: str, counter: str) -> dict:
    """Dispatch_Id -> the counter's value (KiB), from counter_collection.csv."""
    out = {}
    for r in _read_csv(d, "counter_collection.csv"):
        if r["Counter_Name"] == counter:
            out[int(r["Dispatch_Id"])] = out.get(int(r["Dispatch_Id"]), 0.0) + float(r["Counter_Value"])
    return out


def phase_table(trace_dir: str, fetch_dir: str | None = None, write_dir: str | None = None,
                copy_fetch_dir: str | None = None, copy_write_dir: str | None = None,
                steps: int = 1, warmup: int = 0) -> int:
    """Per-phase durations, algorithmic HBM bytes and (with PMC dirs) measured
    bytes of the decode workload run with `--exec eager`, from rocprofv3
    output. Every op of that run launches k_samp_a, k_op, L x 6 phase
    kernels, the lm_head phase kernel and k_commit; the run is (warmup +
    steps) x two sessions x (32 prompt ops at positions 0..31, then 128
    generate ops at positions 32..159). Only the generate ops are tabled."""
    from defer_amd import synthetic

    cfg = synthetic.CONFIGS[CFG_NAME]
    L, h, V = cfg["num_layers"], cfg["hidden_size"], cfg["vocab_size"]
    ff = cfg["intermediate_size"]
    q = cfg["num_heads"] * cfg["head_dim"]
    kv = cfg["num_kv_heads"] * cfg["head_dim"]
    trace = [r for r in _read_csv(trace_dir, "kernel_trace.csv") if "k_phase" in r["Kernel_Name"]]
    trace.sort(key=lambda r: int(r["Dispatch_Id"]))
    per_op = L * len(PHASES) + 1
    n_ops = (warmup + steps) * 2 * 160
    if len(trace) != n_ops * per_op:
        raise SystemExit(f"{len(trace)} k_phase dispatches, expected {n_ops * per_op} "
                         f"({n_ops} ops x {per_op}) for --steps {steps} --warmup {warmup}")
    fetch = _pmc_per_dispatch(fetch_dir, "FETCH_SIZE") if fetch_dir else None
    write = _pmc_per_dispatch(write_dir, "WRITE_SIZE") if write_dir else None
    f_scale = w_scale = 1.0
    if copy_fetch_dir and copy_write_dir:
        cf = [v for v in _pmc_per_dispatch(copy_fetch_dir, "FETCH_SIZE").values()]
        cw = [v for v in _pmc_per_dispatch(copy_write_dir, "WRITE_SIZE").values()]
        f_scale, w_scale = 1048576.0 / max(cf), 1048576.0 / max(cw)
    # algorithmic bytes per dispatch, by phase (weights, the K/V rows read or
    # written, the vectors are the phase's own input/output)
    wq = 4 * (q + 2 * kv) * h + 4 * h

    def algo(ph: int, pos: int) -> int:
        if ph == 0:
            return wq + 4 * 2 * kv                 # qkv rows + norm; new K/V row written
        if ph == 1:
            return 4 * 2 * kv * (pos + 1)          # cached K/V of positions 0..pos, once
        if ph == 2:
            return 4 * q                           # the combined attention output
        if ph == 3:
            return 4 * h * q
        if ph == 4:
            return 4 * 2 * ff * h + 4 * h
        if ph == 5:
            return 4 * h * ff
        return 4 * V * h + 4 * h + 4 * V           # lm_head, final norm, logits

    names = list(PHASES) + ["lm_head"]
    acc = {k: [0, 0.0, 0, 0.0, 0.0] for k in names}  # n, us, algo B, fetch B, write B
    for op in range(n_ops):
        pos = op % 160
        if pos < 32:
            continue
        for j in range(per_op):
            r = trace[op * per_op + j]
            ph = j % len(PHASES) if j < L * len(PHASES) else len(PHASES)
            a = acc[names[ph]]
            a[0] += 1
            a[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            a[2] += algo(ph, pos)
            did = int(r["Dispatch_Id"])
            if fetch is not None:
                a[3] += fetch.get(did, 0.0) * f_scale * 1024
            if write is not None:
                a[4] += write.get(did, 0.0) * w_scale * 1024
    print(f"| Phase | Dispatches | Avg us | Algorithmic B/dispatch | GB/s | % of {PEAK_GBS:.0f} |"
          + (" HBM B/dispatch (PMC) | PMC / algorithmic |" if fetch is not None else ""))
    print("|---|---:|---:|---:|---:|---:|" + ("---:|---:|" if fetch is not None else ""))
    tot = [0, 0.0, 0, 0.0, 0.0]
    for k in names:
        n, us, ab, fb, wb = acc[k]
        for i, v in enumerate(acc[k]):
            tot[i] += v
        gbs = ab / (us * 1e3)
        line = f"| {k} | {n} | {us / n:.2f} | {ab / n:,.0f} | {gbs:.1f} | {100 * gbs / PEAK_GBS:.2f} |"
        if fetch is not None:
            line += f" {(fb + wb) / n:,.0f} | {(fb + wb) / ab:.2f} |"
        print(line)
    n_tok = n_ops * 128 // 160
    print(f"\nGenerate ops: {n_tok}; phase-kernel time per token {tot[1] / n_tok:.1f} us; "
          f"algorithmic {tot[2] / n_tok / 1e6:.1f} MB per token = "
          f"{tot[2] / (tot[1] * 1e3):.1f} GB/s over the phase kernels' own time"
          + (f"; FETCH_SIZE x {f_scale:.5f}, WRITE_SIZE x {w_scale:.5f}" if fetch is not None else ""))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=["c1", "replay", "sessions", "long", "8b"],
                    default="c1",
                    help="c1: 135M-shaped batch-1 decode (default, the headline); replay: the "
                         "2048-position checkout; sessions: 64 Llama-3.2-1B-shaped sessions in "
                         "lockstep; long: 360M-shaped decode of 4096 tokens; 8b: 8B-shaped decode")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-replay", action="store_true",
                    help="skip the replay figures in the decode line's config")
    ap.add_argument("--exec", choices=list(EXEC_MODES), default="persistent",
                    help="how a token step runs: one persistent kernel (default), a captured "
                         "graph of per-phase kernels, or the same kernels launched one by one")
    ap.add_argument("--phase-table", nargs="+", metavar="DIR",
                    help="no GPU: print the per-phase table of a rocprofv3 run of "
                         "`--exec eager` (DIR = its --kernel-trace output; optional FETCH_SIZE, "
                         "WRITE_SIZE dirs of the same command and of `--copy-probe 1024`)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device once (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.phase_table:
        return phase_table(*args.phase_table, steps=args.steps, warmup=args.warmup)
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
    if args.workload == "replay":
        return replay_workload(args)
    if args.workload in ("long", "8b"):
        return decode_workload(args, args.workload)

    from defer_amd import synthetic

    cfg = synthetic.CONFIGS[CFG_NAME]
    weights = synthetic.make_weights(cfg, 0)
    prompt = synthetic.make_prompt(cfg["vocab_size"], 32, seed=42)
    # The CPU baseline runs first, before anything touches the GPU.
    cpu = None if args.no_cpu else cpu_baseline_c1(cfg, weights, prompt)

    from defer_amd import gpu as G
    from defer_amd import host as H

    model = G.GpuModel(G.Config.from_dict(cfg), weights)
    model.set_exec(EXEC_MODES[args.exec])
    model.set_batching(0)
    ref = None
    import tempfile

    wal_dir = tempfile.mkdtemp(prefix="defer-bench-")
    for _ in range(args.warmup):
        ref = c1_step(model, prompt, H, wal_dir)[2:]
    wall, dev, dev_g, dev_t = 0.0, 0.0, 0.0, 0.0
    for _ in range(args.steps):
        w, d, ta, tb = c1_step(model, prompt, H, wal_dir)
        wall += w
        dev += d[0] + d[1]
        dev_g += d[0]
        dev_t += d[1]
        if ref is not None and (ta, tb) != ref:
            raise SystemExit("decode is not repeatable: tokens differ between steps")
        ref = (ta, tb)
    model.set_batching(16)
    model.set_exec(EXEC_MODES["persistent"])
    n_tok = 256 * args.steps
    wbytes = synthetic.weight_bytes_streamed(cfg)
    algo = 2 * algorithmic_bytes(cfg, wbytes, 32, 128) * args.steps
    achieved = algo / (dev / 1e3) / 1e9
    value = n_tok / wall
    secondary = {} if args.no_replay else replay_measure(model, cfg, weights, H, 3, 1)
    model.close()
    line = {
        "metric": "batch-1 decode tok/s (f32) + achieved HBM GB/s as % of peak; replay tok/s",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,0.02) weights from seed 0, uniform-random prompt ids)",
        "config": {
            "workload": "SmolLM2-135M-shaped batch-1 decode: 32-token prompt; session A 128 "
                        "greedy tokens, session B 128 tokens at T=0.7 (seed 42), every token "
                        "appended to the session's WAL inside the timed region; one step = both "
                        "sessions (256 tokens at positions 32..160, prompts untimed)",
            "tokens_per_step": 256,
            "exec": args.exec,
            "us_per_token": round(wall / n_tok * 1e6, 1),
            "device_us_per_token": round(dev / n_tok * 1e3, 1),
            "device_us_per_token_greedy": round(dev_g / (n_tok / 2) * 1e3, 1),
            "device_us_per_token_sampled": round(dev_t / (n_tok / 2) * 1e3, 1),
            "weight_bytes_per_token": wbytes,
            "weight_roofline_tok_s": round(PEAK_GBS * 1e9 / wbytes, 1),
            "weight_roofline_frac": round(value * wbytes / (PEAK_GBS * 1e9), 4),
            **secondary,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_persistent (one launch per 128-token generate call)"
                      if args.exec == "persistent" else
                      f"k_phase ({args.exec}: 184 launches per token, the device time of all)",
            "achieved": round(achieved, 2),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": measured_traffic("k_persistent_decode_135m.md", "traffic_bytes_per_launch")
                       if args.exec == "persistent" else None,
        },
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    rc = main()
    if "defer_amd.gpu" in sys.modules and "torch" not in sys.modules:
        # Every handle is closed: release the device (the runtime's queues,
        # the cooperative one included) before the interpreter exits.
        sys.modules["defer_amd.gpu"].shutdown()
    if rc:
        sys.exit(rc)
