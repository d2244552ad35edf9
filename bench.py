#!/usr/bin/env python3
"""MTP speculative-decode throughput on one MI355X, plus the 4-bit qmv roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload e2e|qmv]

Workload "e2e" (default): a random-init Qwen3.5-9B-shaped model (32 layers, 24
Gated DeltaNet + 8 gated attention, hidden 4096, MLP 12288, vocab 248320, 4-bit
group-64 MLX-layout weights) with an MTP draft head sharing the lm_head. A
4096-token prompt of seeded uniform ids is prefilled (untimed), then W warmup
cycles run, then exactly K timed MTP cycles (draft k=3 greedy, verify 4 tokens,
accept at T=0.7, roll back; the cycle is captured once as a HIP graph and
replayed). value = tokens emitted in the timed cycles / time.

Every line also carries:
  roofline: the 4-bit GEMV of 12288 x 4096 (one M=1 qmv), timed with HIP events
    over back-to-back launches that rotate through >= 600 MB of weight copies
    (so HBM, not the 256 MB Infinity Cache, serves them); algorithmic bytes
    0.5625*N*K + 2K + 2N = 28,344,320 per launch;
  cpu_baseline: the oracle's C restatement (OpenMP) of the cycle's quantized
    matmuls, timed on this host on one cycle's worth of shapes and scaled to
    tokens per second with the GPU run's tokens per cycle.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (str(REPO / "qvex-3.5_amd"), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "MTP spec-decode tok/s (9B-shape, 4-bit, k=3); 4-bit qmv HBM GB/s vs peak"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- qmv roofline

def qmv_time(M, N, K, iters=None, tile=None, seed_tag=0):
    """Average µs per launch of back-to-back qmv launches captured in one HIP graph,
    rotating over enough weight copies that every launch reads HBM."""
    import torch
    from qvex import kernels, synth
    dev = torch.device("cuda:0")
    w, s, b = synth.qmv_weights(N, K, tag=seed_tag)
    x = synth.qmv_x(M, K, tag=seed_tag)
    wd = torch.from_numpy(w.view(np.int32)).to(dev)
    sd = torch.from_numpy(s.view(np.int16)).to(dev).view(torch.bfloat16)
    bd = torch.from_numpy(b.view(np.int16)).to(dev).view(torch.bfloat16)
    xd = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
    wbytes = 0.5625 * N * K
    ncopy = max(2, int(np.ceil(600e6 / wbytes)) + 1)
    W = [wd] + [torch.empty_like(wd).random_() for _ in range(ncopy - 1)]
    S = [sd] + [sd.clone() for _ in range(ncopy - 1)]
    B = [bd] + [bd.clone() for _ in range(ncopy - 1)]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    iters = iters or max(2 * ncopy, 40)
    kernels.quantized_matmul(xd, W[0], S[0], B[0], out=y, tile=tile)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            kernels.quantized_matmul(xd, W[i % ncopy], S[i % ncopy], B[i % ncopy], out=y, tile=tile)
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / iters)
    del g, W, S, B
    torch.cuda.empty_cache()
    algo = 0.5625 * N * K + 2 * M * K + 2 * M * N
    return best, algo


def read_roof_calibration(nbytes=28344320 // 16 * 16, copies=24, reps=3):
    """Stream-read `copies` distinct buffers of nbytes with qvex_read_roof: a
    kernel of known traffic, for scaling PMC byte counters (FETCH_SIZE)."""
    import torch
    from qvex import kernels
    buf = torch.empty(copies * nbytes // 4, dtype=torch.int32, device="cuda:0").random_()
    sink = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    for _ in range(reps):
        for c in range(copies):
            kernels.read_roof(buf[c * nbytes // 4:(c + 1) * nbytes // 4], sink, 2048)
    torch.cuda.synchronize()
    return nbytes


PROFILE = REPO / "profiles" / "qmv_gemv_12288x4096_m1.json"


def roofline_qmv0():
    us, algo = qmv_time(1, 12288, 4096)
    ach = algo / (us * 1e-6) / 1e9
    out = {"kernel": "qvex_qmv_w4g64 (M=1, N=12288, K=4096)", "bound": "hbm",
           "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
           "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
           "algorithmic_bytes_per_launch": int(algo), "avg_launch_us": round(us, 3)}
    # HBM bytes per launch come from rocprofv3 FETCH_SIZE/WRITE_SIZE passes of this
    # same command (calibrated on a read of known size), kept in profiles/
    if PROFILE.exists():
        prof = json.loads(PROFILE.read_text())
        out["traffic"] = prof["traffic_bytes_per_launch"]
        out["traffic_source"] = f"{PROFILE.relative_to(REPO)} ({prof['calibration']})"
        out["rocprof_avg_launch_us"] = prof["avg_us"]
    return out


def qmv_shapes():
    """GB/s of the verify-cycle shapes (M=4 verify rows, M=1 draft rows)."""
    out = {}
    for name, (M, N, K) in {"lm_head_m1": (1, 248320, 4096), "lm_head_m4": (4, 248320, 4096),
                            "gate_up_m4": (4, 24576, 4096), "down_m4": (4, 4096, 12288),
                            "gdn_in_proj_m4": (4, 12352, 4096)}.items():
        us, algo = qmv_time(M, N, K)
        out[name] = {"us": round(us, 2), "GB/s": round(algo / (us * 1e-6) / 1e9, 1),
                     "frac": round(algo / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    return out


# ---------------------------------------------------------------- CPU baseline

def cycle_shapes(cfg, k):
    """(M, N, K, count) of every quantized matmul of one MTP cycle."""
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
    kd = cfg.linear_num_key_heads * cfg.linear_key_head_dim
    vd = cfg.linear_num_value_heads * cfg.linear_value_head_dim
    n_gdn = sum(cfg.is_linear(i) for i in range(cfg.num_hidden_layers))
    n_att = cfg.num_hidden_layers - n_gdn
    W = k + 1
    qkv = Hq * 2 * D + 2 * Hkv * D
    return [
        (W, 2 * kd + 2 * vd + 2 * cfg.linear_num_value_heads, H, n_gdn),   # GDN in_proj
        (W, H, vd, n_gdn),                                                  # GDN out_proj
        (W, qkv, H, n_att), (W, H, Hq * D, n_att),                          # attention
        (W, 2 * I, H, cfg.num_hidden_layers), (W, H, I, cfg.num_hidden_layers),  # MLP
        (W, V, H, 1),                                                       # lm_head (verify)
        (1, H, 2 * H, k), (1, qkv, H, k), (1, H, Hq * D, k),                # MTP head per draft
        (1, 2 * I, H, k), (1, H, I, k), (1, V, H, k),
    ]


def cpu_baseline(cfg, k, tokens_per_cycle):
    import oracle
    from qvex import synth
    threads = min(int(os.environ.get("OMP_NUM_THREADS", "16")), len(os.sched_getaffinity(0)))
    total = 0.0
    for (M, N, K, count) in cycle_shapes(cfg, k):
        w, s, b = synth.qmv_weights(N, K, tag=7)
        x = synth.qmv_x(M, K, tag=7)
        oracle.qmv_f32(x[:1], w[:64], s[:64], b[:64], threads)      # warm the thread pool
        t0 = time.perf_counter()
        oracle.qmv_f32(x, w, s, b, threads)
        dt = time.perf_counter() - t0
        total += dt * count
    return {"value": round(tokens_per_cycle / total, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"one MTP cycle (k={k}) of 4-bit quantized matmuls ({len(cycle_shapes(cfg, k))} shapes, "
                      f"each timed once, scaled by its count) through the C restatement with {threads} "
                      f"OpenMP threads; {total:.2f} s per cycle; other ops (<2% of bytes) not included",
            "host_cpus": os.cpu_count(), "host_affinity": len(os.sched_getaffinity(0))}


# ---------------------------------------------------------------- end to end

def run_e2e(args):
    import torch
    from qvex.model import Config, random_model
    from qvex.mtp import random_mtp
    from qvex.sampler import Sampler, SamplingParams
    from qvex.speculative import GraphedMTPCycle, MTPDecoder, mtp_prefill
    from qvex import synth

    cfg = Config.qwen35_9b()
    dev = torch.device("cuda:0")
    max_ctx = args.prompt + (args.warmup + args.steps + 2) * (args.k + 1) + 64
    t0 = time.perf_counter()
    model = random_model(cfg, seed=synth.SEED_E2E, device=dev, max_context=max_ctx, max_width=args.k + 1)
    mtp = random_mtp(model, seed=synth.SEED_E2E + 1)
    torch.cuda.synchronize()
    log(f"model built in {time.perf_counter() - t0:.1f}s")
    ids = synth.rng(synth.SEED_E2E, 5).integers(0, cfg.vocab_size, size=args.prompt).astype(np.int32)
    ids_t = torch.from_numpy(ids).reshape(1, -1).to(dev)
    cache, mcache = model.make_cache(), mtp.make_cache()
    t0 = time.perf_counter()
    logits, hidden = model(ids_t, cache, return_hidden=True)
    last_h = mtp_prefill(mtp, mcache, hidden, ids_t, None)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"prefill {args.prompt} tokens in {prefill_s:.2f}s")
    sampler = Sampler(SamplingParams(temperature=args.temperature, top_k=0, top_p=1.0, seed=synth.SEED_E2E), cfg.vocab_size)
    stats = {}
    dec = MTPDecoder(model, sampler, cache, logits[0, -1], last_h, mtp, mcache, k=args.k, stats=stats)
    runner = dec
    if not args.eager:
        dec.cycle()                        # one eager cycle, then capture the cycle as a HIP graph
        t0 = time.perf_counter()
        runner = GraphedMTPCycle(dec)
        log(f"cycle captured as a HIP graph in {time.perf_counter() - t0:.2f}s")
    for _ in range(args.warmup):
        runner.cycle()
    torch.cuda.synchronize()
    e0 = stats["emitted"]
    a0, c0 = stats["accepted"], stats["cycles"]
    t0 = time.perf_counter()
    for i in range(args.steps):
        runner.cycle()
        if (i + 1) % 64 == 0:
            log(f"cycle {i + 1}/{args.steps}")
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    emitted = stats["emitted"] - e0
    acc = stats["accepted"] - a0
    cycles = stats["cycles"] - c0
    return {"value": emitted / dt, "ms_per_step": dt / args.steps * 1e3, "tokens": emitted,
            "tokens_per_cycle": emitted / cycles, "acceptance": acc / (cycles * args.k),
            "prefill_s": prefill_s}, cfg


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="e2e", choices=["e2e", "qmv"])
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--k", type=int, default=3)
    ap.add_argument("--temperature", type=float, default=0.7)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch every kernel from Python (no HIP graph)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (collectives are out of scope); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    from qvex import _C
    _C.lib()  # fail loudly without the HIP library

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic: random-init weights generated in the MLX 4-bit group-64 layout, "
                    "seeded uniform prompt ids"}
    if args.workload == "e2e":
        res, cfg = run_e2e(args)
        line.update({"value": round(res["value"], 2), "unit": "tok/s", "ms_per_step": round(res["ms_per_step"], 3)})
        line["config"] = {"workload": "MTP speculative decode, Qwen3.5-9B shape (32 layers: 24 Gated DeltaNet "
                                      "+ 8 gated attention, hidden 4096, MLP 12288, vocab 248320), 4-bit g64 "
                                      "weights, MTP head drafting k=3, T=0.7, 4096-token prompt",
                          "k": args.k, "prompt_tokens": args.prompt, "temperature": args.temperature,
                          "cycles_timed": args.steps, "hip_graph": not args.eager}
        line["tokens_per_cycle"] = round(res["tokens_per_cycle"], 4)
        line["acceptance"] = round(res["acceptance"], 4)
        line["prefill_s"] = round(res["prefill_s"], 2)
    else:
        from qvex.model import Config
        cfg = Config.qwen35_9b()
        res = None
    log("qmv roofline")
    line["roofline"] = roofline_qmv0()
    if args.workload == "qmv":
        line["read_roof_calibration_bytes"] = read_roof_calibration()
        line.update({"value": line["roofline"]["achieved"], "unit": "GB/s",
                     "ms_per_step": line["roofline"]["avg_launch_us"] / 1e3,
                     "config": {"workload": "4-bit group-64 GEMV, x bf16 [1,4096], W [12288,4096]"}})
    if not args.no_shapes:
        line["qmv_shapes"] = qmv_shapes()
    if not args.no_cpu_baseline:
        log("cpu baseline")
        tpc = res["tokens_per_cycle"] if res else 1.0
        line["cpu_baseline"] = cpu_baseline(cfg, args.k, tpc)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
