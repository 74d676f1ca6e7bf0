#!/usr/bin/env python3
"""Batch-1 greedy decode of the MiniCPM5-2.4B-shaped Q4_K_M model on one MI355X.

Workload (the full 2.4B-shaped model): 40 layers, hidden 2304,
32 q / 8 kv heads of 64, FFN 5760 SwiGLU, vocab 130560 with a tied Q6_K LM
head, Q6_K attn_v / ffn_down, Q4_K elsewhere, F32 norms; random-init weights
N(0, 0.02) from a fixed seed; a 32-token random-ID prompt, then greedy decode.
A step is one decoded token (one captured hipGraph replay of the whole
forward plus argmax on the device) through the engine's default decode path:
every layer of the token in one persistent launch where that launch has an
instance compiled for the shape (this one, on 256 CUs), else five launches
per layer.  --warmup steps run untimed, then exactly --steps steps are timed
between device synchronisations.

Printed: one JSON line with tokens/s, the achieved HBM bandwidth of the
dominant kernel against the 8 TB/s peak (HIP events around its launches, on
the engine stream), and the reference's CPU path timed on this host's cores;
beside them the same decode through the other decode path, the long-context
prefill and sampled decode, and the single-op configurations (one GEMV cold
and warm, the FFN block, QKV + attention) with, for each GEMV class of the
five-launch path, one read-only launch of its bytes as the floor a single
launch of that size can reach.
"""
import argparse
import platform
import subprocess
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "minicpm5.cpp_amd", "python"))

import mcpm  # noqa: E402

HBM_PEAK_GBPS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16
# HBM bytes per launch by kernel class from rocprofv3 FETCH_SIZE / WRITE_SIZE
# runs, scaled by the same counters on a device copy of known size
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_2p4b_traffic.json")
SEED = 20260105  # base seed 20260101 + 4, the full-model workload's index
PROMPT = 32


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Decode kernels of this workload by class (the shapes the launch picker
# chooses for the 2.4B-shaped model; names as rocprofv3 prints them, less
# namespaces and arguments).
PROFILE_CLASSES = {
    # the default decode path: every layer of a token in one launch, the
    # instance compiled for this shape with XCD-local hand-offs
    "layers": "k_decode_persist<true, true>",
    "qkv": "k_gemv<3, 1, true, 2, false>",
    "attn": "k_attention_q8k",
    "oproj": "k_gemv<0, 2, true, 0, true>",
    # contexts of at most 64 positions: the attention inside the O projection
    "oproj_attn": "k_gemv<6, 2, true, 0, true>",
    "gate_up": "k_gemv<3, 3, true, 0, false>",
    "down": "k_gemv<2, 2, true, 1, true>",
    "lm_head": "k_gemv<4, 4, false, 1, false>",
}
COPY_KERNEL = "__amd_rocclr_copyBuffer"


def summarize_profiles(stats_csv, fetch_csv, write_csv, calib_bytes, out_path, run):
    """Per-class figures from three rocprofv3 runs of `bench.py --eager`: the
    kernel-trace statistics (average launch duration) and the FETCH_SIZE and
    WRITE_SIZE counters (KiB per dispatch, averaged over a class's
    dispatches), the counters scaled by what they read for the run's device
    copies of calib_bytes (the largest copy dispatch).  Classes with no
    launch in these runs keep what out_path already holds for them (the
    other decode path's runs); each class names the run it comes from."""
    import csv

    def short(name):
        name = name.replace("(anonymous namespace)::", "").replace("void ", "").replace("mcpm::", "")
        return name.split("(")[0].strip()

    stats = {short(r["Name"]): r for r in csv.DictReader(open(stats_csv))}

    def counter(path, cname):
        per, calib = {}, 0.0
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != cname:
                continue
            k, v = short(r["Kernel_Name"]), float(r["Counter_Value"])
            if k == COPY_KERNEL:
                calib = max(calib, v)
            per.setdefault(k, []).append(v)
        return {k: sum(v) / len(v) for k, v in per.items()}, {k: len(v) for k, v in per.items()}, calib

    fetch, nf, cf = counter(fetch_csv, "FETCH_SIZE")
    write, _, cw = counter(write_csv, "WRITE_SIZE")
    ff = calib_bytes / (cf * 1024) if cf else None
    fw = calib_bytes / (cw * 1024) if cw else None
    old = {}
    if os.path.exists(out_path):
        with open(out_path) as f:
            old = json.load(f)
    classes = old.get("classes", {})
    for cls, kern in PROFILE_CLASSES.items():
        if kern not in stats:
            continue
        e = {"kernel": kern, "run": run, "kernel_calls": int(stats[kern]["Calls"]),
             "kernel_avg_us": round(float(stats[kern]["AverageNs"]) / 1000.0, 3)}
        if kern in fetch and ff:
            e.update(dispatches=nf[kern], fetch_kib=round(fetch[kern], 1), write_kib=round(write.get(kern, 0.0), 1),
                     fetch_bytes=int(fetch[kern] * 1024 * ff), write_bytes=int(write.get(kern, 0.0) * 1024 * (fw or 1.0)))
        classes[cls] = e
    runs = old.get("runs", {})
    runs[run] = {"kernel_stats": os.path.basename(stats_csv),
                 "copy_calibration": {"bytes": calib_bytes, "fetch_kib": cf, "write_kib": cw,
                                      "fetch_factor": round(ff, 5) if ff else None,
                                      "write_factor": round(fw, 5) if fw else None}}
    out = {"workload": "greedy decode, 2.4B-shaped Q4_K_M decoder, eager launches", "runs": runs,
           "classes": {k: classes[k] for k in PROFILE_CLASSES if k in classes}}
    with open(out_path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    return out


def kernel_breakdown(eng, n_tokens=8):
    """Per-class average launch duration: HIP events recorded around each
    kernel of the class on the engine stream.  Timing a class makes the token
    run eagerly (kernel by kernel, not as one graph replay), so these
    durations include each launch's own start-up and exceed the kernels'
    share of a graph-replayed step; classes with no launch are left out."""
    out = {}
    for kc, name in enumerate(mcpm.KC_NAMES):
        eng.set_kernel_timing(kc)
        eng.decode_steps(n_tokens)
        eng.sync()
        ms, n = eng.kernel_time()
        eng.set_kernel_timing(-1)
        if n == 0:
            continue
        per_launch_us = 1000.0 * ms / max(n, 1)
        launches_per_token = n / n_tokens
        out[name] = {"avg_us": per_launch_us, "launches_per_token": launches_per_token,
                     "us_per_token": per_launch_us * launches_per_token,
                     "bytes_per_launch": eng.kernel_bytes(kc)}
    return out


PATH_LAUNCH = {"persistent": "one launch per token for every layer (one work group per CU), hipGraph per token",
               "five_launch": "five launches per layer (QKV, attention, O, gate/up, down), hipGraph per token"}


def other_path_measure(eng, prompt, steps, warmup, default_tps):
    """The same decode (prompt, warmup, then `steps` timed steps) through the
    decode path the default does not take, on the same engine and KV cache,
    graph replay as the default: five launches per layer where the default
    is the persistent launch (mcpm_engine_set_persistent mode 0; with their
    per-class kernel timings), else the persistent launch wherever the shape
    fits (mode 1; None where it does not).  The default mode is restored."""
    persistent_default = eng.uses_persistent()
    eng.set_persistent(0 if persistent_default else 1)
    try:
        if not persistent_default and not eng.uses_persistent():
            return None, None
        eng.generate_greedy(prompt, 1 + warmup)
        eng.sync()
        t0 = time.perf_counter()
        eng.decode_steps(steps)
        eng.sync()
        dt = time.perf_counter() - t0
        name = "five_launch" if persistent_default else "persistent"
        out = {"path": name, "tokens_per_s": round(steps / dt, 2), "ms_per_step": round(1e3 * dt / steps, 4),
               "over_default": round(steps / dt / default_tps, 4), "launch": PATH_LAUNCH[name]}
        return out, kernel_breakdown(eng) if persistent_default else None
    finally:
        eng.set_persistent(mcpm.PERSIST_AUTO)


def prefill_measure(eng, cfg, n_prompt=1024, reps=3):
    """The long-context configuration's prompt: n_prompt random token ids
    through the batched prefill (MFMA GEMMs).  Times the prefill of the first
    n_prompt-1 tokens (KV cache only) and the time to the first token (that
    prefill plus the last prompt token's forward and argmax)."""
    eng.init_kv_cache(1536)
    prompt = np.random.default_rng(SEED + 1).integers(0, cfg.vocab, n_prompt).astype(np.int32)
    eng.prefill(prompt[:n_prompt - 1])
    eng.sync()
    t_pf, t_ttft = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        eng.prefill(prompt[:n_prompt - 1])
        eng.sync()
        t_pf.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        eng.generate_greedy(prompt, 1)
        eng.sync()
        t_ttft.append(time.perf_counter() - t0)
    pf, ttft = float(np.median(t_pf)), float(np.median(t_ttft))
    # algorithmic GEMM work: every layer's projections for n_prompt-1 tokens,
    # the last layer's q/k/v only (nothing after them reaches the KV cache)
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    qkv = (qd + 2 * kvd) * cfg.dim
    layer = qkv + cfg.dim * qd + 2 * cfg.ffn * cfg.dim + cfg.dim * cfg.ffn
    macs = (n_prompt - 1) * ((cfg.n_layers - 1) * layer + qkv)
    tflops = 2.0 * macs / pf / 1e12
    return {"prompt_tokens": n_prompt, "prefill_ms": round(pf * 1e3, 2),
            "prefill_tokens_per_s": round((n_prompt - 1) / pf, 1),
            "time_to_first_token_ms": round(ttft * 1e3, 2),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": FP16_MFMA_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                         "flop_per_pass": 2 * macs}}


def sampled_measure(eng, cfg, n_prompt=1024, n_gen=512, temperature=0.8, top_p=0.95):
    """The long-context configuration's decode: after an n_prompt-token prompt
    (batched prefill), n_gen tokens drawn by the device sampler (temperature,
    top-p), the KV cache growing to n_prompt + n_gen.  The decode rate is
    (n_gen - 1) over the difference between the n_gen-token and the 1-token
    runs (both include the same prefill); the greedy loop at the same
    positions is timed the same way, for the sampler's share."""
    eng.init_kv_cache(n_prompt + n_gen + 4)
    prompt = np.random.default_rng(SEED + 2).integers(0, cfg.vocab, n_prompt).astype(np.int32)

    def run(fn, n):
        t0 = time.perf_counter()
        fn(n)
        eng.sync()
        return time.perf_counter() - t0

    sampled = lambda n: eng.generate_sampled(prompt, n, temperature, top_p, SEED)
    greedy = lambda n: eng.generate_greedy(prompt, n)
    run(sampled, 8)  # warm-up: graphs, sampler scratch
    ts = run(sampled, n_gen) - run(sampled, 1)
    tg = run(greedy, n_gen) - run(greedy, 1)
    return {"prompt_tokens": n_prompt, "tokens": n_gen, "temperature": temperature, "top_p": top_p,
            "context_at_end": n_prompt + n_gen - 1, "tokens_per_s": round((n_gen - 1) / ts, 1),
            "ms_per_token": round(1e3 * ts / (n_gen - 1), 4),
            "greedy_tokens_per_s_same_positions": round((n_gen - 1) / tg, 1)}


def ops_measure(ctx, eng, cfg, bd, cold_mb=640):
    """The single-op configurations, kernel time from HIP events at each
    kernel's start and end:
      C1  one Q4_K GEMV 5760 x 2304 with the ties-even Q8_K quantize prologue
          (mcpm_gemv_q4_K), warm (one weight copy, resident in the 256 MB
          Infinity Cache) and cold (a rotation over cold_mb of copies);
      C2  the FFN block as the engine runs it (RMSNorm + Q8_K + gate/up +
          SwiGLU, then Q8_K + down + residual: two fused kernels), per layer
          of the decode measured above, weights streamed from HBM;
      C3  QKV (with RoPE and the KV append) + attention at contexts 512, 2048
          and 4096 (the engine's kernels after a prompt of that length)."""
    out = {}
    rows, cols = 5760, 2304
    w = mcpm.synth_normal(SEED + 10, 1, rows * cols, 0.0, 0.02).reshape(rows, cols)
    native = mcpm.quantize_rows(mcpm.TYPE_Q4_K, w)
    n_copies = max(1, -(-(cold_mb << 20) // native.nbytes))
    copies = [ctx.tensor(native, mcpm.TYPE_Q4_K, cols, rows) for _ in range(n_copies)]
    x = ctx.upload(mcpm.synth_normal(SEED + 10, 2, cols))
    y = ctx.alloc(rows * 4)
    c1_bytes = native.nbytes + cols * 4 + rows * 4

    def timed(seq, reps):
        ctx.set_op_timing(True)
        for _ in range(reps):
            for t in seq:
                mcpm.check(ctx.lib.mcpm_gemv_q4_K(ctx.h, t.h, x.ptr, y.ptr, rows, cols))
        ms, n = ctx.op_time()
        ctx.set_op_timing(False)
        return 1e3 * ms / max(n, 1)

    timed(copies[:1], 20)
    c1 = {"bytes": c1_bytes}
    for name, seq, reps in (("warm", copies[:1], 400), ("cold", copies, 4)):
        us = timed(seq, reps)
        gbps = c1_bytes / (us * 1e-6) / 1e9
        c1[name] = {"us": round(us, 3), "GBps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4)}
    c1["cold"]["rotation_MB"] = round(n_copies * native.nbytes / 1e6, 1)
    out["c1_gemv_q4k_5760x2304"] = c1
    for t in copies:
        t.free()
    x.free()
    y.free()

    gu, dn = bd["gate_up"], bd["down"]
    c2_us = gu["avg_us"] + dn["avg_us"]
    c2_bytes = gu["bytes_per_launch"] + dn["bytes_per_launch"]
    out["c2_ffn_block"] = {"us": round(c2_us, 3), "bytes": c2_bytes,
                           "GBps": round(c2_bytes / (c2_us * 1e-6) / 1e9, 1),
                           "frac": round(c2_bytes / (c2_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                           "kernels_us": {"gate_up": round(gu["avg_us"], 3), "down": round(dn["avg_us"], 3)}}

    kvd = cfg.n_kv_heads * cfg.head_dim
    qkv_w = eng.kernel_bytes(mcpm.KC_QKV)
    c3 = {}
    eng.set_persistent(0)  # the five launches' QKV and attention kernels
    eng.init_kv_cache(4096 + 64)
    for ctx_len in (512, 2048, 4096):
        prompt = np.random.default_rng(SEED + ctx_len).integers(0, cfg.vocab, ctx_len).astype(np.int32)
        eng.generate_greedy(prompt, 1)
        eng.sync()
        us = {}
        for kc, name in ((mcpm.KC_QKV, "qkv"), (mcpm.KC_ATTN, "attn")):
            eng.set_kernel_timing(kc)
            eng.decode_steps(4)
            eng.sync()
            ms, n = eng.kernel_time()
            eng.set_kernel_timing(-1)
            us[name] = 1e3 * ms / max(n, 1)
        # KV read at about ctx_len + 4 positions, plus the new row's append
        b = qkv_w + 2 * (ctx_len + 4) * kvd * 4 + 2 * kvd * 4
        t = us["qkv"] + us["attn"]
        c3[str(ctx_len)] = {"us": round(t, 3), "qkv_us": round(us["qkv"], 3), "attn_us": round(us["attn"], 3),
                            "bytes": b, "GBps": round(b / (t * 1e-6) / 1e9, 1),
                            "frac": round(b / (t * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    out["c3_qkv_attention"] = c3
    eng.set_persistent(mcpm.PERSIST_AUTO)
    return out


def read_floor_measure(ctx, bd, pool_mb=1024, grids=(512, 1024, 2048, 4096)):
    """The floor of one launch that reads as many bytes as a GEMV class: a
    read-only kernel (mcpm_stream_read: 16-byte non-temporal loads, a
    grid-stride loop) over the class's bytes per launch, each launch on the
    next region of a pool_mb rotation (so the bytes come from HBM, as the
    weights do in decode), the best of a few grid sizes; kernel durations from
    HIP events at each kernel's start and end, as the class timings are."""
    pool_bytes = pool_mb << 20
    pool = ctx.alloc(pool_bytes)
    sink = ctx.alloc(max(grids) * 4)
    out = {"pool_MB": round(pool_bytes / 1e6, 1), "classes": {}}
    gemv_us = floor_us = 0.0
    try:
        mcpm.check(ctx.lib.mcpm_fill_device(ctx.h, pool.ptr, 1, pool_bytes))
        for name in ("qkv", "oproj", "gate_up", "down", "lm_head"):
            d = bd[name]
            nbytes = -(-d["bytes_per_launch"] // 16) * 16
            nreg = pool_bytes // nbytes
            reps = max(16, min(400, (4 << 30) // nbytes))

            def run(n, g):
                for r in range(n):
                    mcpm.check(ctx.lib.mcpm_stream_read(ctx.h, pool.ptr + (r % nreg) * nbytes, nbytes, g,
                                                        sink.ptr))

            best = None
            for g in grids:
                run(8, g)
                ctx.op_time()
                ctx.set_op_timing(True)
                run(reps, g)
                ms, n = ctx.op_time()
                ctx.set_op_timing(False)
                us = 1e3 * ms / max(n, 1)
                if best is None or us < best[0]:
                    best = (us, g)
            lpt = d["launches_per_token"]
            gemv_us += d["avg_us"] * lpt
            floor_us += best[0] * lpt
            out["classes"][name] = {"bytes": nbytes, "floor_us": round(best[0], 3), "grid": best[1],
                                    "floor_GBps": round(nbytes / (best[0] * 1e-6) / 1e9, 1),
                                    "kernel_us": round(d["avg_us"], 3),
                                    "floor_over_kernel": round(best[0] / d["avg_us"], 4) if d["avg_us"] else None}
    finally:
        sink.free()
        pool.free()
    out["gemv_us_per_token"] = round(gemv_us, 1)
    out["floor_us_per_token"] = round(floor_us, 1)
    out["floor_over_gemv_per_token"] = round(floor_us / gemv_us, 4)
    return out


def host_cpu():
    """CPU model, sockets, physical cores (lscpu) and the CPUs this process may
    run on."""
    info = {"model": platform.processor() or "unknown", "sockets": None, "physical_cores": None}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    info["model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(l.split(":", 1) for l in out.splitlines() if ":" in l)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        if kv.get("Model name") and len(kv["Model name"]) > len(info["model"]):
            info["model"] = kv["Model name"]
        if kv.get("BIOS Model name"):
            info["bios_model"] = kv["BIOS Model name"]
        # where the model name is generic (a virtual machine's "AMD EPYC"),
        # the vendor, family, model and stepping still identify the part
        for key, name in (("Vendor ID", "vendor"), ("CPU family", "family"), ("Model", "model_number"),
                          ("Stepping", "stepping")):
            if kv.get(key):
                info[name] = kv[key]
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets or None
        info["physical_cores"] = sockets * per or None
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    info["allowed_cpus"] = len(os.sched_getaffinity(0))
    return info


def cpu_baseline(image, cfg_vocab, prompt, n_steps, budget_s=20.0):
    """The reference's own CPU ops (oracle/_ref: its src/ops compiled -O3
    -mavx2 -mfma -ffast-math -fopenmp, driven through the restated forward)
    when built, else the oracle's C restatement, on the benchmark's own
    workload: the same 32-token prompt, then greedy decode steps (all 256
    when they fit the time budget).  Run with the reference CLI's team of 8
    threads (src/main.cpp:34 -> include/omp_config.h) and with one thread per
    physical core this process may use (at most 16, the box's CPU share),
    OMP_PROC_BIND=close, OMP_PLACES=cores; `value` is the 8-thread run."""
    os.environ["OMP_PROC_BIND"] = "close"  # read when the OpenMP runtime starts (first oracle load below)
    os.environ["OMP_PLACES"] = "cores"
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    host = host_cpu()
    kind = "reference" if O.reference() is not None else "port"
    lib = O.reference() if kind == "reference" else None
    phys = host["physical_cores"] or host["allowed_cpus"]
    team = min(16, phys, host["allowed_cpus"])
    runs = []
    for threads in sorted({8, team}):
        if lib is not None:
            lib.ref_set_threads(threads)
        else:
            O.oracle().or_set_threads(threads)
        model = O.OracleModel(image, use_reference_ops=(kind == "reference"))
        model.init_kv(len(prompt) + n_steps + 1)
        lg = np.empty(cfg_vocab, np.float32)
        t0 = time.perf_counter()
        for p, t in enumerate(prompt):
            tok = model.forward(int(t), p, lg)
        t1 = time.perf_counter()
        n = 0
        while n < n_steps and time.perf_counter() - t1 < budget_s:
            tok = model.forward(tok, len(prompt) + n, lg)
            n += 1
        t2 = time.perf_counter()
        model.close()
        runs.append({"threads": threads, "decode_tokens_per_s": n / (t2 - t1), "decode_steps": n,
                     "prompt_tokens_per_s": len(prompt) / (t1 - t0)})
        log(f"  CPU {kind} {threads} threads: {n / (t2 - t1):.1f} tok/s over {n} decode steps")
    main_run = next(r for r in runs if r["threads"] == 8)
    src = ("oracle/_ref: the reference's src/ops compiled -O3 -mavx2 -mfma -mf16c -ffast-math -fopenmp"
           if kind == "reference" else "the oracle's C port")
    # "cores" is the OpenMP team of the `value` run (threads, one per core
    # with OMP_PLACES=cores); cpu.physical_cores is the host's core count
    return {"value": main_run["decode_tokens_per_s"], "unit": "tokens/s", "cores": 8, "threads": 8, "kind": kind,
            "sample": f"the benchmark's 32-token prompt, then {main_run['decode_steps']} greedy decode steps of the "
                      f"same 2.4B-shaped model (budget {budget_s:.0f} s), {src}; 8 OpenMP threads as the "
                      f"reference CLI forces, OMP_PROC_BIND=close OMP_PLACES=cores",
            "cpu": host, "runs": runs}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mix", type=int, default=0, help="0: Q6_K v/down in every layer; 1: llama.cpp layers")
    ap.add_argument("--eager", action="store_true", help="launch kernels one by one instead of a graph replay")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 1024-token prefill measurement")
    ap.add_argument("--no-other-path", "--no-persistent", dest="no_other_path", action="store_true",
                    help="skip the same decode through the decode path the default does not take (five launches "
                         "per layer where the default is the persistent launch)")
    ap.add_argument("--no-sampled", action="store_true",
                    help="skip the sampled decode after a 1024-token prompt (device sampler)")
    ap.add_argument("--no-ops", action="store_true",
                    help="skip the single-op configurations (one GEMV cold/warm, FFN block, QKV + attention)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run device-to-device copies of this many MB (the reference kernel of known "
                         "size for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--summarize-profiles", nargs=3, metavar=("STATS_CSV", "FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/decode_2p4b_traffic.json from rocprofv3 outputs and exit (no GPU)")
    ap.add_argument("--profile-run", default="default decode path",
                    help="with --summarize-profiles: the name the classes of these runs are filed under")
    args = ap.parse_args()
    if args.summarize_profiles:
        out = summarize_profiles(*args.summarize_profiles, (args.copy_calibration_mb or 256) << 20, TRAFFIC_FILE,
                                 args.profile_run)
        print(json.dumps(out["classes"]))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(batch-1 decode of one model runs on one GPU)", file=sys.stderr)
        sys.exit(2)

    cfg = mcpm.config_2p4b()
    log("synthesizing the 2.4B-shaped model")
    t = time.perf_counter()
    image = mcpm.synth_gguf(cfg, seed=SEED, mix=args.mix)
    log(f"  {image.nbytes / 1e9:.3f} GB GGUF in {time.perf_counter() - t:.1f} s")
    ctx = mcpm.Context(0)
    n_cu, arch = ctx.info()
    eng = mcpm.Engine(ctx, image=image)
    if args.eager:
        eng.set_graph(False)
    log(f"loaded into HBM on {arch} ({n_cu} CUs){' eager launches' if args.eager else ''}")
    total_steps = args.warmup + args.steps + 8 * len(mcpm.KC_NAMES)
    eng.init_kv_cache(PROMPT + total_steps + 8)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, PROMPT).astype(np.int32)

    # prefill + warmup (untimed), then exactly --steps timed steps
    eng.generate_greedy(prompt, 1 + args.warmup)
    eng.sync()
    t0 = time.perf_counter()
    eng.decode_steps(args.steps)
    eng.sync()
    t1 = time.perf_counter()
    dt = t1 - t0
    tps = args.steps / dt
    wbytes = eng.weight_bytes_per_token()
    path = "persistent" if eng.uses_persistent() else "five_launch"
    log(f"decode ({path.replace('_', ' ')}): {args.steps} tokens in {dt * 1e3:.1f} ms -> {tps:.1f} tok/s, "
        f"{wbytes * tps / 1e9:.1f} GB/s effective")

    # per-kernel durations with HIP events (eager launches of the same kernels)
    bd = kernel_breakdown(eng)
    dom = max(bd, key=lambda k: bd[k]["us_per_token"])
    d = bd[dom]
    for k, v in bd.items():
        log(f"  {k:8s} {v['avg_us']:8.2f} us x {v['launches_per_token']:.0f}/token "
            f"= {v['us_per_token']:8.1f} us/token  "
            f"{v['bytes_per_launch'] / (v['avg_us'] * 1e-6) / 1e9 if v['bytes_per_launch'] and v['avg_us'] else 0:7.1f} GB/s")

    other, bd_five = None, None
    if not args.no_other_path and not args.eager:
        other, bd_five = other_path_measure(eng, prompt, args.steps, args.warmup, tps)
        if other:
            log(f"{other['path'].replace('_', ' ')} path, same decode: {other['tokens_per_s']:.1f} tok/s "
                f"({other['over_default']:.3f} of the default path)")
    if path == "five_launch":
        bd_five = bd
    elif bd_five is None and not args.no_ops:
        # the single-op figures and the read floor take the five launches'
        # per-class timings, at the same contexts
        eng.set_persistent(0)
        eng.generate_greedy(prompt, 1 + args.warmup)
        eng.decode_steps(args.steps)
        bd_five = kernel_breakdown(eng)
        eng.set_persistent(mcpm.PERSIST_AUTO)
    if bd_five is not bd and bd_five:
        log("  five launches per layer, per class:")
        for k, v in bd_five.items():
            log(f"  {k:8s} {v['avg_us']:8.2f} us x {v['launches_per_token']:.0f}/token = {v['us_per_token']:8.1f} us/token")

    if args.copy_calibration_mb > 0:
        nbytes = args.copy_calibration_mb << 20
        src, dst = mcpm.DeviceBuffer(ctx, nbytes), mcpm.DeviceBuffer(ctx, nbytes)
        ctx.lib.mcpm_fill_device(ctx.h, src.ptr, 1, nbytes)
        for _ in range(4):
            mcpm.check(ctx.lib.mcpm_copy_device(ctx.h, dst.ptr, src.ptr, nbytes))
        src.free()
        dst.free()
        log(f"copy calibration: 4 device copies of {args.copy_calibration_mb} MiB")

    prefill = None
    if not args.no_prefill:
        prefill = prefill_measure(eng, cfg)
        log(f"prefill: {prefill['prompt_tokens'] - 1} tokens in {prefill['prefill_ms']:.1f} ms -> "
            f"{prefill['prefill_tokens_per_s']:.0f} tok/s ({prefill['roofline']['achieved']:.1f} TFLOP/s), "
            f"first token after {prefill['time_to_first_token_ms']:.1f} ms")

    sampled = None
    if not args.no_sampled:
        sampled = sampled_measure(eng, cfg)
        log(f"sampled decode after a {sampled['prompt_tokens']}-token prompt: {sampled['tokens_per_s']:.1f} tok/s "
            f"(T {sampled['temperature']}, top-p {sampled['top_p']}; greedy at the same positions "
            f"{sampled['greedy_tokens_per_s_same_positions']:.1f} tok/s)")

    ops = None
    if not args.no_ops:
        ops = ops_measure(ctx, eng, cfg, bd_five)
        c1 = ops["c1_gemv_q4k_5760x2304"]
        log(f"ops: C1 GEMV {c1['warm']['us']:.2f} us warm ({c1['warm']['GBps']:.0f} GB/s), "
            f"{c1['cold']['us']:.2f} us cold ({c1['cold']['GBps']:.0f} GB/s); "
            f"C2 FFN block {ops['c2_ffn_block']['us']:.2f} us; C3 QKV+attention "
            + ", ".join(f"{k}: {v['us']:.2f} us" for k, v in ops["c3_qkv_attention"].items()))
        rf = read_floor_measure(ctx, bd_five)
        ops["read_floor"] = rf
        log("read floor (one read-only launch of each GEMV class's bytes): "
            + ", ".join(f"{k} {v['floor_us']:.2f} us vs {v['kernel_us']:.2f}" for k, v in rf["classes"].items())
            + f"; GEMVs {rf['gemv_us_per_token']:.0f} us/token, floor {rf['floor_us_per_token']:.0f} us/token "
            f"({100 * rf['floor_over_gemv_per_token']:.0f} %)")

    traffic_classes = {}
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic_classes = json.load(f).get("classes", {})

    def roofline_of(cls, d):
        """The class's achieved HBM rate (algorithmic bytes per launch over
        this run's HIP-event launch time), with the committed rocprofv3
        figures for it: read + written bytes per launch, and its average
        launch time from the kernel statistics of the same decode path."""
        tr = traffic_classes.get(cls, {})
        a = d["bytes_per_launch"] / (d["avg_us"] * 1e-6) / 1e9
        prof = None
        if tr.get("kernel_avg_us"):
            pa = d["bytes_per_launch"] / (tr["kernel_avg_us"] * 1e-6) / 1e9
            src = "decode_2p4b_persistent_kernel_stats.md" if "persistent" in tr.get("run", "") \
                else "decode_2p4b_kernel_stats.md"
            prof = {"source": "profiles/" + src, "avg_launch_us": tr["kernel_avg_us"], "achieved": round(pa, 1),
                    "frac": round(pa / HBM_PEAK_GBPS, 4)}
        return {"bound": "hbm", "kernel": cls, "achieved": round(a, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(a / HBM_PEAK_GBPS, 4),
                "traffic": int(tr["fetch_bytes"] + tr["write_bytes"]) if "fetch_bytes" in tr else None,
                "bytes_per_launch": d["bytes_per_launch"], "avg_launch_us": round(d["avg_us"], 3),
                "timing": "eager launches of the class, HIP events around each kernel on the engine stream",
                "rocprof": prof}

    roofline = roofline_of(dom, d)
    if bd_five is not bd and bd_five:
        # the five launches' dominant GEMV class, for comparison
        d5 = max(bd_five, key=lambda k: bd_five[k]["us_per_token"])
        roofline["five_launch_dominant"] = roofline_of(d5, bd_five[d5])

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        cpu = cpu_baseline(image, cfg.vocab, prompt, 256)
        log(f"  cpu: {cpu['value']:.2f} tok/s ({cpu['kind']}, {cpu['cores']} threads, {cpu['cpu']['model']})")

    res = {
        "metric": "decode tokens/s, batch 1, 2.4B Q4_K_M shape; GEMV achieved HBM GB/s vs peak",
        "value": round(tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot (Q4_K/Q6_K x Q8_K), fp32 scale/accumulate",
        "data": "synthetic: random-init weights N(0,0.02) seed 20260105, random-ID prompt",
        "config": {"workload": "greedy decode, batch 1, 2.4B-shaped Q4_K_M decoder", "layers": cfg.n_layers,
                   "hidden": cfg.dim, "heads": f"{cfg.n_heads}q/{cfg.n_kv_heads}kv x {cfg.head_dim}",
                   "ffn": cfg.ffn, "vocab": cfg.vocab, "quant_mix": "literal" if args.mix == 0 else "llama",
                   "launch": "eager" if args.eager else "hipGraph per token", "decode_path": path,
                   "prompt_tokens": PROMPT, "context_at_end": PROMPT + args.warmup + args.steps,
                   "weight_bytes_per_token": wbytes, "effective_GBps": round(wbytes * tps / 1e9, 1),
                   "token_roofline_frac": round(wbytes * tps / 1e9 / HBM_PEAK_GBPS, 4),
                   "eager_kernels_us_per_token": {k: round(v["us_per_token"], 2) for k, v in bd.items()},
                   "eager_kernels_sum_us_per_token": round(sum(v["us_per_token"] for v in bd.values()), 1),
                   "eager_sum_over_graph_step": round(sum(v["us_per_token"] for v in bd.values())
                                                      / (1e6 * dt / args.steps), 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode_paths": {"default": path, path: {"tokens_per_s": round(tps, 2), "launch": PATH_LAUNCH[path]},
                         **({other["path"]: other} if other else {})},
        "prefill": prefill,
        "sampled_decode": sampled,
        "ops": ops,
    }
    print(json.dumps(res), flush=True)
    eng.free()
    ctx.close()


if __name__ == "__main__":
    main()
