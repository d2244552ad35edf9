#!/usr/bin/env python3
"""MTP speculative-decode throughput on one MI355X, plus the 4-bit qmv roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload e2e|qmv|gdn|gdn_verify|mixer|attn|spec] [--accept-all]

Workload "e2e" (default): a random-init Qwen3.5-9B-shaped model (32 layers, 24
Gated DeltaNet + 8 gated attention, hidden 4096, MLP 12288, vocab 248320, 4-bit
group-64 MLX-layout weights) with an MTP draft head sharing the lm_head. A
4096-token prompt of seeded uniform ids is prefilled (untimed), then the
speculative.decode() generator - the reference's API, iterated as its MTP
benchmark does (bench/mtp_bench.py:49-55) - runs W warmup cycles (the first
captures the cycle as a HIP graph) and exactly K timed MTP cycles (draft k=3
greedy, verify 4 tokens, accept at T=0.7 with top-k 20 / top-p 0.8 as the
reference's MTP benchmark, roll back): one graph replay and one host read per
cycle. value = tokens emitted in the timed cycles / time.
graphed_run: the same cycles through GraphedMTPCycle.run (each launched before
  the previous result is read), from the same prompt and seed;
cycle_roofline: the cycle's algorithmic HBM bytes (weights, DeltaNet states, KV)
  at 8 TB/s against the measured cycle;
accept_all: a labelled diagnostic, greedy with the shared lm_head zeroed, so
  every draft is accepted (k + 1 tokens a cycle, the n = k commit path).

Every line also carries:
  roofline: the dominant kernel of the cycle, the packed 4-bit MFMA qmv on the
    fused gate/up projection at the 4 verify rows with SwiGLU in its epilogue
    (N=24576, K=4096), timed with HIP events over back-to-back launches that
    rotate through >= 600 MB of weight copies (so HBM, not the 256 MB Infinity
    Cache, serves them); algorithmic bytes 0.5625*N*K + 2MK + 2M(N/2) =
    56,754,176 per launch;
  qmv_config0: the same for the single 4-bit GEMV of 12288 x 4096 (M=1,
    28,344,320 bytes per launch);
  qmv_shapes: the decode cycle's other matmul shapes, and the config-0 GEMV on
    the packed copy QLinear runs it on;
  cpu_baseline: the oracle's C restatement (OpenMP) of the cycle's quantized
    matmuls, timed on this host on one cycle's worth of shapes and scaled to
    tokens per second with the GPU run's tokens per cycle;
  cpu_baselines: the same restatement beside each config's GPU figure
    (config-0 GEMV, config-2 verify recurrence, config-3 accept on a sample of
    steps), on all host threads, best of repeated runs;
  cycle_kernels: the cycle's split DeltaNet mixer and verify attention (one
    layer at the 9B shape, isolated, rotating caches) with their HBM fractions.

--accept-all makes that diagnostic the line's value (labelled, not the headline).

The other workloads run one kernel family in a loop for rocprofv3 counter
passes (profiles/): gdn (chunked DeltaNet prefill), gdn_verify (the config-2
recurrence), mixer (the cycle's split DeltaNet mixer at the 9B shape), attn
(the verify attention's q/k norm + RoPE, partial and combine at a 4352-token
context), spec (config 3); readprobe prints the single-launch read ceiling by
load path (VGPR against direct-to-LDS loads).
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

def qmv_time(M, N, K, iters=None, tile=None, seed_tag=0, packed=False, swiglu=False):
    """Average µs per launch of back-to-back qmv launches captured in one HIP graph,
    rotating over enough weight copies that every launch reads HBM. packed=True
    times the tile-packed MFMA kernel (what QLinear runs for 1..4 rows)."""
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
    if packed:
        PK = [kernels.pack_w4(W[i], S[i], B[i], swiglu=swiglu) for i in range(ncopy)]
        del W, S, B
        W = S = B = None
        def launch(i):   # rows in chunks of 8, as QLinear runs 9..15-row calls
            for m0 in range(0, M, 8):
                kernels.quantized_matmul_packed(xd[m0:m0 + 8], PK[i % ncopy], N, out=y[m0:m0 + 8], tile=tile,
                                                swiglu=swiglu)
    else:
        PK = None
        launch = lambda i: kernels.quantized_matmul(xd, W[i % ncopy], S[i % ncopy], B[i % ncopy], out=y, tile=tile)
    y = torch.empty((M, N // 2 if swiglu else N), dtype=torch.bfloat16, device=dev)
    iters = iters or max(2 * ncopy, 40)
    launch(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            launch(i)
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
    del g, W, S, B, PK
    torch.cuda.empty_cache()
    algo = 0.5625 * N * K + 2 * M * K + 2 * M * (N // 2 if swiglu else N)
    return best, algo


def read_ceiling_us(nbytes, blocks=2048, iters=200):
    """The single-launch HBM read ceiling for a buffer of nbytes: qvex_read_roof
    (grid-stride 16-byte loads; 2048 blocks of 256 threads = 32 waves on each of
    the 256 CUs) replayed back to back from a HIP graph over rotating copies
    (> 600 MB, so HBM serves them), as the products are timed. A sweep of 256 to
    4096 blocks and 1 to 16 loads in flight per lane found this shape fastest for
    9.4 to 57 MB."""
    import torch
    from qvex import kernels
    n = nbytes // 16 * 16
    copies = int(np.ceil(600e6 / n)) + 1
    bufs = [torch.empty(n // 4, dtype=torch.int32, device="cuda:0").fill_(i) for i in range(copies)]
    sink = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    kernels.read_roof(bufs[0], sink, blocks)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            kernels.read_roof(bufs[i % copies], sink, blocks)
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
    del g, bufs
    torch.cuda.empty_cache()
    return best


def read_probe_table(sizes_kib=(9216, 27648, 55296)):
    """Single-launch read ceiling by load path: qvex_read_probe with VGPR loads
    against gfx950's direct-to-LDS loads (global_load_lds_dwordx4), same access
    pattern (every wave issues all its 1 KiB units before waiting), 2..16 units
    per wave, 4 or 8 waves per block, beside qvex_read_roof's grid-stride read;
    graphs of back-to-back launches over > 600 MB of copies. Sizes 9.4, 28.3 and
    56.6 MB (the o_proj, config-0 and gate/up weight bytes, rounded to 128 KiB)."""
    import torch
    from qvex import kernels
    dev = torch.device("cuda:0")
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    out = {}
    for kib in sizes_kib:
        nb = kib * 1024
        copies = int(np.ceil(600e6 / nb)) + 1
        bufs = [torch.empty(nb // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(copies)]
        res = {"grid_stride_2048": _graph_time(lambda i: kernels.read_roof(bufs[i % copies], sink, 2048), 200)}
        for lds in (False, True):
            for it in (2, 4, 8, 16):
                for wpb in (4, 8):
                    res[f"{'lds' if lds else 'vgpr'}_it{it}_w{wpb}"] = _graph_time(
                        lambda i, it=it, lds=lds, wpb=wpb: kernels.read_probe(bufs[i % copies], sink, it, lds, wpb), 200)
        best = {path: min(v for k, v in res.items() if k.startswith(path)) for path in ("vgpr", "lds", "grid")}
        out[f"{nb / 1e6:.1f}MB"] = {"us": {k: round(v, 2) for k, v in res.items()},
                                    "best_us": {k: round(v, 2) for k, v in best.items()},
                                    "best_TB_s": {k: round(nb / v / 1e6, 2) for k, v in best.items()}}
        del bufs
        torch.cuda.empty_cache()
    return out


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


# Kernels with a roofline entry: (M, N, K, packed, profile summary). "gate_up_m4" is
# the dominant kernel of the decode cycle (the fused gate/up projection of every
# layer at the 4 verify rows); "config0" is the single M=1 GEMV of 12288 x 4096.
ROOF_KERNELS = {
    "gate_up_m4": (4, 24576, 4096, "swiglu", "qmv_packed_swiglu_24576x4096_m4.json",
                   "qvex_qmv_w4g64_packed_swiglu (M=4, N=24576, K=4096; verify gate_up + SwiGLU)"),
    "config0": (1, 12288, 4096, False, "qmv_gemv_12288x4096_m1.json",
                "qvex_qmv_w4g64 (M=1, N=12288, K=4096)"),
}


def roofline(name):
    M, N, K, packed, prof_name, label = ROOF_KERNELS[name]
    us, algo = qmv_time(M, N, K, packed=bool(packed), swiglu=packed == "swiglu")
    ach = algo / (us * 1e-6) / 1e9
    ceil = read_ceiling_us(int(algo))
    out = {"kernel": label, "bound": "hbm",
           "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
           "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
           "algorithmic_bytes_per_launch": int(algo), "avg_launch_us": round(us, 3),
           "read_ceiling_us": round(ceil, 3), "frac_of_read_ceiling": round(ceil / us, 3)}
    # HBM bytes per launch come from rocprofv3 FETCH_SIZE/WRITE_SIZE passes of
    # `bench.py --workload qmv --qmv NAME` (calibrated on a read of known size), kept in profiles/
    prof = REPO / "profiles" / prof_name
    if prof.exists():
        p = json.loads(prof.read_text())
        out["traffic"] = p["traffic_bytes_per_launch"]
        out["traffic_source"] = f"{prof.relative_to(REPO)} ({p['calibration']})"
        out["rocprof_avg_launch_us"] = p["avg_us"]
    return out


def qmv_shapes():
    """Config-1 shapes as the decode cycle runs them: the packed MFMA kernel for
    1..4 rows (M=4 verify, M=1 draft / plain decode), and for M=5 (a verify of 4
    drafts) as two row halves over one read of the weights; config0_packed_m1 is
    the config-0 GEMV on the copy QLinear packs once at load (what a decode step
    runs for that weight; qmv_config0 times the MLX-layout kernel)."""
    out = {}
    shapes = {"lm_head_m1": (1, 248320, 4096), "lm_head_m4": (4, 248320, 4096),
              "gate_up_swiglu_m4": (4, 24576, 4096), "down_m4": (4, 4096, 12288),
              "gdn_in_proj_m4": (4, 12352, 4096), "attn_qkv_m4": (4, 10240, 4096),
              "o_proj_m4": (4, 4096, 4096), "mtp_fc_m1": (1, 4096, 8192),
              "gate_up_swiglu_m5": (5, 24576, 4096), "config0_packed_m1": (1, 12288, 4096)}
    for name, (M, N, K) in shapes.items():
        us, algo = qmv_time(M, N, K, packed=True, swiglu="swiglu" in name)
        ceil = read_ceiling_us(int(0.5625 * N * K))
        out[name] = {"us": round(us, 2), "GB/s": round(algo / (us * 1e-6) / 1e9, 1),
                     "frac": round(algo / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                     "read_ceiling_us": round(ceil, 2), "frac_of_read_ceiling": round(ceil / us, 3),
                     "kernel": "packed" if M <= 4 else "packed, two row halves over one weight read"}
    return out


def _graph_time(fn, iters, reps=5):
    """Best-of-reps average µs per call of fn(i), i = 0..iters-1, captured once as a
    HIP graph and replayed between HIP events (no host launch cost in the timing,
    as in the decode cycle)."""
    import torch
    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / iters)
    del g
    return best


def _event_time(fn, iters, reps=3):
    """Best-of-reps average µs per call of fn(i), i = 0..iters-1, between HIP events
    on the current stream (every call launches on that stream)."""
    import torch
    fn(0)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(iters):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / iters)
    return best


def spec_config3(S=256, k=4, V=248320, temperature=0.7):
    """Fused accept/resample over S verify steps in one launch on the seeded
    config-3 inputs of synth.spec_inputs (target ~N(0,3) plus +8 spikes, draft =
    target + N(0,1), draft ids from softmax(draft/T), uniforms U(0,1)): the same
    bytes tests/test_spec_gpu.py checks bit for bit against the oracle for all
    256 steps. Bytes (2k+1)*V*4 per step."""
    import torch
    from qvex import kernels, synth
    dev = torch.device("cuda:0")
    threads = min(16, len(os.sched_getaffinity(0)))
    inp = synth.spec_inputs(range(S), k=k, V=V, temperature=temperature, threads=threads)
    target = torch.from_numpy(inp["target"]).to(dev)
    draft = torch.from_numpy(inp["draft"]).to(dev)
    draft_ids = torch.from_numpy(inp["draft_ids"]).to(dev)
    u_acc = torch.from_numpy(inp["u_accept"]).to(dev)
    u_smp = torch.from_numpy(inp["u_sample"]).to(dev)
    del inp
    ws = kernels.spec_workspace(S, k, V, True, dev)
    n = torch.empty(S, dtype=torch.int32, device=dev)
    tok = torch.empty(S, dtype=torch.int32, device=dev)
    us = _event_time(lambda i: kernels.spec_accept(target, draft, draft_ids, u_acc, u_smp, temperature,
                                                    n_accept=n, out_token=tok, workspace=ws), 5)
    nbytes = (2 * k + 1) * V * 4 * S
    acc = float(n.float().mean())
    del target, draft
    torch.cuda.empty_cache()
    return {"kernel": "qvex_spec_accept (3 kernels: rowstats, decide, sample)", "steps": S, "k": k, "V": V,
            "inputs": f"synth.spec_inputs(range({S}), k={k}) (seed {synth.SEED_SPEC}, the tested inputs)",
            "us": round(us, 1), "us_per_step": round(us / S, 3), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "bytes": nbytes,
            "mean_accept": round(acc, 3)}


def gdn_config2_verify(T=5, Hk=16, Hv=32, D=128, copies=40):
    """Gated DeltaNet verify form: T tokens of one layer (Hk=16, Hv=32, d=128) with
    a state snapshot per token; rotates over `copies` state/snapshot buffers so the
    2 MiB state is read from HBM; bytes = state + T snapshots + q,k,v,y,a,b."""
    import torch
    from qvex import kernels
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1002)
    bf = torch.bfloat16
    q = torch.nn.functional.normalize(torch.randn((1, T, Hk, D), generator=g, device=dev), dim=-1).to(bf)
    kk = torch.nn.functional.normalize(torch.randn((1, T, Hk, D), generator=g, device=dev), dim=-1).to(bf)
    v = torch.randn((1, T, Hv, D), generator=g, device=dev).to(bf)
    a = torch.randn((1, T, Hv), generator=g, device=dev).to(bf)
    b = torch.randn((1, T, Hv), generator=g, device=dev).to(bf)
    A_log = torch.zeros(Hv, device=dev)
    dt = torch.zeros(Hv, device=dev, dtype=bf)
    states = [torch.randn((1, Hv, D, D), generator=g, device=dev) * 0.02 for _ in range(copies)]
    snaps = [torch.empty((T, 1, Hv, D, D), device=dev) for _ in range(copies)]
    y = torch.empty((1, T, Hv, D), device=dev, dtype=bf)
    us = _graph_time(lambda i: kernels.gated_delta_snapshots(q, kk, v, a, b, A_log, dt, states[i % copies],
                                                              snapshots=snaps[i % copies], y=y), 4 * copies)
    nbytes = (1 + T) * Hv * D * D * 4 + 2 * T * Hk * D * 2 + 2 * T * Hv * D * 2 + 2 * T * Hv * 2
    return {"kernel": "qvex_gdn_recurrent (T=5, per-token snapshots)", "us": round(us, 2),
            "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "bytes": nbytes}


def gdn_config2_prefill(T=4096, Hk=16, Hv=32, D=128, C=64, recurrent=True):
    """Gated DeltaNet prefill form, T = 4096 tokens of one layer (Hk = 16, Hv = 32,
    d = 128) through the chunked MFMA kernel (chunk 64); work counted as the
    canonical chunked FLOPs Hv*(T/C)*(4C^2 Dk + 4C^2 Dv + 6 C Dk Dv) = 21.47 GFLOP.
    The recurrent kernel on the same input is timed beside it."""
    import torch
    from qvex import _C, kernels
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1002)
    bf = torch.bfloat16
    q = torch.nn.functional.normalize(torch.randn((1, T, Hk, D), generator=g, device=dev), dim=-1).to(bf)
    kk = torch.nn.functional.normalize(torch.randn((1, T, Hk, D), generator=g, device=dev), dim=-1).to(bf)
    v = torch.randn((1, T, Hv, D), generator=g, device=dev).to(bf)
    a = torch.randn((1, T, Hv), generator=g, device=dev).to(bf)
    b = torch.randn((1, T, Hv), generator=g, device=dev).to(bf)
    A_log = torch.zeros(Hv, device=dev)
    dt = torch.zeros(Hv, device=dev, dtype=bf)
    s0 = torch.randn((1, Hv, D, D), generator=g, device=dev) * 0.02
    s1 = torch.empty_like(s0)
    y = torch.empty((1, T, Hv, D), device=dev, dtype=bf)
    ws = torch.empty(int(_C.lib().qvex_gdn_chunked_workspace_bytes(1, T, Hv, D, D, C)), dtype=torch.uint8, device=dev)
    us = _event_time(lambda i: kernels.gated_delta_chunked(q, kk, v, a, b, A_log, dt, s0, state_out=s1, y=y,
                                                           workspace=ws), 10)
    flops = Hv * (T // C) * (4 * C * C * D + 4 * C * C * D + 6 * C * D * D)
    out = {"kernel": "qvex_gdn_chunked (prep + scan, chunk 64)", "T": T, "us": round(us, 1),
           "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 2), "frac_of_bf16_peak": round(flops / (us * 1e-6) / 2.5e15, 4),
           "flops": flops}
    if recurrent:
        ur = _event_time(lambda i: kernels.gated_delta(q, kk, v, a, b, A_log, dt, s0), 3)
        out["recurrent_us"] = round(ur, 1)
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


def _best_of(fn, reps=3):
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def cpu_baselines(k_spec=4, steps_sample=4):
    """The oracle's C restatement beside each config's GPU figure, on all host
    threads (best of 3): config 0 (the 12288 x 4096 GEMV, fp32 accumulate),
    config 2 verify (T = 5 recurrence with snapshots, 32 heads of 128), config 2
    prefill (T = 4096, one run), config 3 (the fused accept on a sample of
    `steps_sample` of its 256 steps, scaled)."""
    import oracle
    from qvex import synth
    threads = min(int(os.environ.get("OMP_NUM_THREADS", "16")), len(os.sched_getaffinity(0)))
    out = {"cores": threads, "kind": "port"}
    w, s, b = synth.qmv_weights(12288, 4096, tag=9)
    x = synth.qmv_x(1, 4096, tag=9)
    oracle.qmv_f32(x, w[:64], s[:64], b[:64], threads)
    t = _best_of(lambda: oracle.qmv_f32(x, w, s, b, threads))
    out["config0_gemv"] = {"us": round(t * 1e6, 1), "GB/s": round(28344320 / t / 1e9, 2)}
    inp = synth.gdn_inputs(5, seed=9, Hk=16, Hv=32)
    f = synth.bf16_to_f32
    args = [f(inp[n]) for n in ("q", "k", "v", "a", "b")]
    t = _best_of(lambda: oracle.gated_delta_f32(*args, inp["A_log"], f(inp["dt_bias"]), inp["state"], snaps=True,
                                                 threads=threads))
    out["config2_verify"] = {"us": round(t * 1e6, 1), "GB/s": round(12.71e6 / t / 1e9, 2)}
    # config-2 prefill: the recurrence of engine/kernels.py:34-63 over all 4096
    # tokens (the chunked GPU kernel regroups the same arithmetic), run once
    inp = synth.gdn_inputs(4096, seed=9, Hk=16, Hv=32)
    args = [f(inp[n]) for n in ("q", "k", "v", "a", "b")]
    t0 = time.perf_counter()
    oracle.gated_delta_f32(*args, inp["A_log"], f(inp["dt_bias"]), inp["state"], snaps=False, threads=threads)
    t = time.perf_counter() - t0
    flops = 32 * (4096 // 64) * (4 * 64 * 64 * 128 * 2 + 6 * 64 * 128 * 128)
    out["config2_prefill"] = {"us": round(t * 1e6, 1), "TFLOP/s": round(flops / t / 1e12, 4),
                              "sample": "T = 4096, 32 value heads of 128, one run (no chunking: the recurrence)"}
    sp = synth.spec_inputs(range(steps_sample), k=k_spec, V=248320)
    t = _best_of(lambda: oracle.spec_accept(sp["target"], sp["draft"], sp["draft_ids"], sp["u_accept"],
                                             sp["u_sample"], float(np.float32(1.0) / np.float32(0.7)),
                                             threads=threads), reps=2)
    out["config3_accept"] = {"us_per_step": round(t * 1e6 / steps_sample, 1),
                             "us_256_steps": round(t * 1e6 / steps_sample * 256, 1),
                             "sample": f"{steps_sample} of the 256 steps (k={k_spec}, V=248320, draft logits)"}
    return out


# ---------------------------------------------------------------- single-kernel workloads (profiling)

def mixer_verify(copies=24, iters=96):
    """The decode cycle's split DeltaNet mixer (qvex_gdn_decode_split, the model's
    workgroups per value head) at the 9B shape for a 4-token verify with snapshots, over
    rotating recurrent caches (state ring + conv ring, ~19 MB each); bytes = the
    state read + 4 snapshots written = 10 MiB per call."""
    import torch
    from qvex.model import Config, random_model
    cfg = Config.qwen35_9b()
    cfg.num_hidden_layers = 1
    m = random_model(cfg, seed=5, device="cuda:0", max_context=256, max_width=4)
    gdn = m.layers[0].mixer
    caches = [m.make_cache(max_width=4) for _ in range(copies)]
    g = torch.Generator(device="cuda:0")
    g.manual_seed(5)
    proj = (torch.randn((4, gdn.in_proj.N), generator=g, device="cuda:0")).to(torch.bfloat16)
    us = _graph_time(lambda i: gdn.mix_split(proj, caches[i % copies][0]), iters)
    nbytes = 5 * 32 * 128 * 128 * 4
    return {"kernel": f"qvex_gdn_decode_split ({gdn.split_blocks} blocks per head, T=4 with snapshots)",
            "us": round(us, 2),
            "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "bytes": nbytes}


def attn_verify(L=4, pos0=4348, copies=24, iters=96, kps=128):
    """The verify attention of one layer at the 9B shape (16 q / 4 kv heads of 256,
    L = 4 rows at positions 4348..4351) over rotating KV caches: the fused decode
    step (qvex_attention_decode: norms, RoPE and the KV append inside the split
    kernel, then the combine), beside the two-launch path it replaces
    (qvex_attn_qk_rope, then qvex_attention); bytes = the K and V read for the
    4352 keys (17.8 MB per call)."""
    import torch
    from qvex import _C
    from qvex.kernels import _ptr, _stream
    dev = torch.device("cuda:0")
    Hq, Hkv, D, rot = 16, 4, 256, 64
    cap = 4608
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    proj = torch.randn((L, Hq * 2 * D + 2 * Hkv * D), generator=g, device=dev).to(torch.bfloat16)
    qn = torch.ones(D, dtype=torch.bfloat16, device=dev)
    kc = [torch.randn((Hkv, cap, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    vc = [torch.randn((Hkv, D, cap), generator=g, device=dev).to(torch.bfloat16) for _ in range(copies)]
    pos = torch.tensor([pos0], dtype=torch.int32, device=dev)
    q = torch.empty((L, Hq, D), dtype=torch.bfloat16, device=dev)
    out = torch.empty((L, Hq * D), dtype=torch.bfloat16, device=dev)
    need = int(_C.lib().qvex_attn_workspace_bytes(L, Hq, Hkv, D, pos0 + L, kps))
    ws = torch.empty((need + 3) // 4, dtype=torch.float32, device=dev)

    def two_launch(i):
        c = i % copies
        _C.call("qvex_attn_qk_rope", _ptr(proj), proj.stride(0), _ptr(qn), _ptr(qn), _ptr(pos), L, Hq, Hkv, D, rot,
                1e7, 1e-6, _ptr(q), _ptr(kc[c]), _ptr(vc[c]), cap, _ptr(tab), tab.shape[0], _stream())
        _C.call("qvex_attention", _ptr(q), _ptr(kc[c]), _ptr(vc[c]), _ptr(pos), L, Hq, Hkv, D, cap, pos0 + L, pos0 + L, kps,
                _ptr(proj), proj.stride(0), _ptr(out), _ptr(ws), ws.numel() * 4, _stream())

    from qvex.model import rope_table
    tab = rope_table(rot, 1e7, cap, dev)

    def fused(i):
        c = i % copies
        _C.call("qvex_attention_decode", _ptr(proj), proj.stride(0), _ptr(qn), _ptr(qn), _ptr(pos), L, Hq, Hkv, D,
                rot, 1e-6, _ptr(tab), tab.shape[0], _ptr(kc[c]), _ptr(vc[c]), cap, pos0 + L, kps, _ptr(out), _ptr(ws),
                ws.numel() * 4, _stream())
    us2 = _graph_time(two_launch, iters)
    us = _graph_time(fused, iters)
    nbytes = 2 * Hkv * (pos0 + L) * D * 2
    return {"kernel": "qvex_attention_decode (decode partial + combine)", "ctx": pos0 + L, "us": round(us, 2),
            "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "bytes": nbytes, "two_launch_us": round(us2, 2)}


# ---------------------------------------------------------------- end to end

def cycle_bytes(model, mtp, k, ctx):
    """Algorithmic HBM bytes of one MTP cycle (k drafts, k + 1 verify rows) at
    context ctx: every main-model weight byte once (the verify, lm_head
    included), the MTP head's products and the shared lm_head once per draft,
    the DeltaNet states read once and written after each verify token, and the
    verify attention's K and V of the ctx keys in every attention layer."""
    cfg = model.cfg
    w = lambda q: 0.5625 * q.N * q.K
    main = sum(w(q) for q in model.qlinears())
    draft = k * (sum(w(q) for q in mtp.qlinears()) + w(model.lm_head))
    n_gdn = sum(cfg.is_linear(i) for i in range(cfg.num_hidden_layers))
    n_att = cfg.num_hidden_layers - n_gdn
    state = cfg.linear_num_value_heads * cfg.linear_value_head_dim * cfg.linear_key_head_dim * 4
    gdn = n_gdn * state * (1 + (k + 1))
    kv = n_att * 2 * cfg.num_key_value_heads * ctx * cfg.head_dim * 2
    return {"main_weights": int(main), "drafting": int(draft), "gdn_state": int(gdn), "kv": int(kv),
            "total": int(main + draft + gdn + kv)}


def _pull(gen, toks, stats, cycles):
    """Iterate the decode() generator until `cycles` cycles have run and every
    token they emitted has been taken."""
    while stats["cycles"] < cycles or len(toks) < stats["emitted"]:
        toks.append(next(gen))


def time_decode(model, mtp, caches, logits, last_h, sampler, k, warmup, steps):
    """The reference's API as its MTP benchmark drives it (bench/mtp_bench.py:
    49-55): iterate decode() and time the tokens of `steps` cycles after
    `warmup` cycles (the first of which captures the cycle's HIP graph). Each
    cycle is one graph replay and one host read of its result."""
    import torch
    from qvex.speculative import decode
    cache, mcache = caches
    stats = {}
    gen = decode(model, sampler, cache, logits[0, -1], last_h, mtp, mcache, stats=stats, k=k)
    toks = [next(gen)]
    _pull(gen, toks, stats, warmup)
    torch.cuda.synchronize()
    n0, a0, c0, g0 = len(toks), stats["accepted"], stats["cycles"], stats["graph_cycles"]
    t0 = time.perf_counter()
    _pull(gen, toks, stats, warmup + steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    gen.close()
    n, cycles = len(toks) - n0, stats["cycles"] - c0
    return {"value": n / dt, "ms_per_step": dt / steps * 1e3, "tokens": n, "tokens_per_cycle": n / cycles,
            "acceptance": (stats["accepted"] - a0) / (cycles * k), "graph_cycles": stats["graph_cycles"] - g0,
            "captures": stats["captures"]}, toks


def time_run(model, mtp, caches, logits, last_h, sampler, k, warmup, steps):
    """GraphedMTPCycle.run: each cycle launched before the previous cycle's result
    is read (two graphs alternating over pinned result slots), so the GPU never
    waits on the host between cycles; the upper bound of the decode() figure."""
    import torch
    from qvex.speculative import GraphedMTPCycle, MTPDecoder
    cache, mcache = caches
    stats = {}
    dec = MTPDecoder(model, sampler, cache, logits[0, -1], last_h, mtp, mcache, k=k, stats=stats)
    g = GraphedMTPCycle(dec)
    toks = [dec.first]
    for part in g.run(warmup):
        toks += part
    torch.cuda.synchronize()
    n0 = len(toks)
    t0 = time.perf_counter()
    for part in g.run(steps):
        toks += part
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    g.release()
    n = len(toks) - n0
    return {"value": n / dt, "ms_per_step": dt / steps * 1e3, "tokens": n}, toks


def run_e2e(args):
    import torch
    from qvex.model import Config, random_model
    from qvex.mtp import random_mtp
    from qvex.sampler import Sampler, SamplingParams
    from qvex.engine import prefill
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
    logits, last_h = prefill(model, ids_t, cache, mtp, mcache)      # 512-token chunks, MTP head per chunk
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"prefill {args.prompt} tokens in {prefill_s:.2f}s")
    clone = lambda: (cache.clone(), mcache.clone())                  # every measurement starts from the prompt

    def sampler(temperature):
        # the reference's MTP benchmark samples with top_k = 20, top_p = 0.8 (bench/mtp_bench.py:39)
        return Sampler(SamplingParams(temperature=temperature, top_k=args.top_k, top_p=args.top_p,
                                      seed=synth.SEED_E2E), cfg.vocab_size)

    def zero_head():
        # diagnostic: greedy with every logit 0, so drafts (token 0) are always accepted
        model.lm_head.scales.zero_()
        model.lm_head.biases.zero_()
        model.lm_head.repack()

    extra = {}
    if args.accept_all:
        zero_head()
    temperature = 0.0 if args.accept_all else args.temperature
    if args.eager:
        from qvex.speculative import MTPDecoder
        stats = {}
        dec = MTPDecoder(model, sampler(temperature), cache, logits[0, -1], last_h, mtp, mcache, k=args.k,
                         stats=stats)
        for _ in range(args.warmup):
            dec.cycle()
        torch.cuda.synchronize()
        e0, a0, c0 = stats["emitted"], stats["accepted"], stats["cycles"]
        t0 = time.perf_counter()
        for _ in range(args.steps):
            dec.cycle()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        n, cycles = stats["emitted"] - e0, stats["cycles"] - c0
        res = {"value": n / dt, "ms_per_step": dt / args.steps * 1e3, "tokens": n, "tokens_per_cycle": n / cycles,
               "acceptance": (stats["accepted"] - a0) / (cycles * args.k)}
    else:
        # the pipelined loop first: besides its own figure it brings the GPU to its
        # steady clocks before the headline's timed cycles (the first timed loop of
        # a process otherwise runs ~1.5 % slow)
        run, toks_run = time_run(model, mtp, clone(), logits, last_h, sampler(temperature), args.k, args.warmup,
                                 args.steps)
        log(f"GraphedMTPCycle.run: {run['value']:.1f} tok/s, {run['ms_per_step']:.3f} ms per cycle")
        res, toks = time_decode(model, mtp, clone(), logits, last_h, sampler(temperature), args.k, args.warmup,
                                args.steps)
        log(f"decode(): {res['value']:.1f} tok/s, {res['ms_per_step']:.3f} ms per cycle")
        extra["graphed_run"] = {"value": round(run["value"], 2), "unit": "tok/s",
                                "ms_per_step": round(run["ms_per_step"], 3),
                                "same_tokens_as_decode": toks_run == toks[:len(toks_run)],
                                "decode_over_run": round(res["value"] / run["value"], 4),
                                "how": "GraphedMTPCycle.run(K): each cycle launched before the previous result "
                                       "is read (no host gap); same seed and prompt as the decode() figure"}
        if not args.accept_all and not args.no_accept_all:
            zero_head()
            aa, _ = time_decode(model, mtp, clone(), logits, last_h, sampler(0.0), args.k, args.warmup, args.steps)
            log(f"accept-all diagnostic: {aa['value']:.1f} tok/s, {aa['ms_per_step']:.3f} ms per cycle")
            extra["accept_all"] = {"value": round(aa["value"], 2), "unit": "tok/s",
                                   "ms_per_step": round(aa["ms_per_step"], 3),
                                   "tokens_per_cycle": round(aa["tokens_per_cycle"], 4),
                                   "acceptance": round(aa["acceptance"], 4),
                                   "how": "DIAGNOSTIC: greedy with the shared lm_head zeroed, so every draft is "
                                          "accepted (k + 1 tokens, the n = k commit path, every cycle); decode() "
                                          "iterated as for the headline"}
    ctx = args.prompt + (args.warmup + args.steps // 2) * res["tokens_per_cycle"]
    cb = cycle_bytes(model, mtp, args.k, int(ctx))
    ms_peak = cb["total"] / (PEAK_HBM_GBS * 1e9) * 1e3
    extra["cycle_roofline"] = {"bound": "hbm", "bytes_per_cycle": cb["total"], "components": cb,
                               "context": int(ctx), "ms_at_peak": round(ms_peak, 4),
                               "ms_per_cycle": round(res["ms_per_step"], 4),
                               "frac": round(ms_peak / res["ms_per_step"], 4),
                               "tok_s_at_peak": round(res["tokens_per_cycle"] / ms_peak * 1e3, 1)}
    res["prefill_s"] = prefill_s
    res["extra"] = extra
    return res, cfg


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="e2e",
                    choices=["e2e", "qmv", "gdn", "gdn_verify", "mixer", "attn", "spec", "readprobe"])
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--k", type=int, default=3)
    ap.add_argument("--temperature", type=float, default=0.7)
    ap.add_argument("--top-k", type=int, default=20)
    ap.add_argument("--top-p", type=float, default=0.8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    ap.add_argument("--qmv", default="config0", choices=sorted(ROOF_KERNELS),
                    help="kernel timed by --workload qmv")
    ap.add_argument("--eager", action="store_true", help="launch every kernel from Python (no HIP graph)")
    ap.add_argument("--accept-all", action="store_true",
                    help="diagnostic: greedy, zeroed lm_head, every draft accepted (not the headline figure)")
    ap.add_argument("--no-accept-all", action="store_true",
                    help="skip the accept-all diagnostic that follows the headline")
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
                                      "weights, MTP head drafting k=3, T=0.7 (top-k 20, top-p 0.8), 4096-token prompt",
                          "k": args.k, "prompt_tokens": args.prompt, "temperature": args.temperature,
                          "top_k": args.top_k, "top_p": args.top_p,
                          "cycles_timed": args.steps, "hip_graph": not args.eager}
        if args.accept_all:
            line["metric"] = "diagnostic: MTP cycle with every draft accepted (greedy, zeroed lm_head), tok/s"
            line["config"]["temperature"] = 0.0
            line["config"]["workload"] += "; DIAGNOSTIC accept-all (not the headline)"
        line["config"]["timed_through"] = "MTPDecoder.cycle() op by op (--eager)" if args.eager else \
            "speculative.decode() generator (reference API; graph replay, one host read per cycle)"
        line["tokens_per_cycle"] = round(res["tokens_per_cycle"], 4)
        line["acceptance"] = round(res["acceptance"], 4)
        line["prefill_s"] = round(res["prefill_s"], 2)
        for key in ("graph_cycles", "captures"):
            if key in res:
                line[key] = res[key]
        line.update(res["extra"])
    else:
        from qvex.model import Config
        cfg = Config.qwen35_9b()
        res = None
    single = {"gdn_verify": gdn_config2_verify, "mixer": mixer_verify, "attn": attn_verify, "spec": spec_config3}
    if args.workload in single:
        r = single[args.workload]()
        line.update({"value": r["GB/s"], "unit": "GB/s", "ms_per_step": r["us"] / 1e3, args.workload: r,
                     "config": {"workload": r["kernel"]}})
        print(json.dumps(line), flush=True)
        return
    if args.workload == "readprobe":
        r = read_probe_table()
        best = r["28.3MB"]["best_us"]
        line.update({"value": round(28311552 / min(best.values()) / 1e3, 1), "unit": "GB/s",
                     "ms_per_step": min(best.values()) / 1e3, "read_probe": r,
                     "config": {"workload": "single-launch HBM read of 9.4 / 28.3 / 56.6 MB by load path"}})
        print(json.dumps(line), flush=True)
        return
    if args.workload == "gdn":
        # the chunked prefill kernel only (what the rocprofv3 MFMA passes under profiles/ run)
        r = gdn_config2_prefill(recurrent=False)
        line.update({"value": r["TFLOP/s"], "unit": "TFLOP/s", "ms_per_step": r["us"] / 1e3,
                     "dtype": "bf16 operands, fp32 state", "gdn_config2_prefill": r,
                     "config": {"workload": "Gated DeltaNet prefill, T=4096, Hk=16, Hv=32, d=128, chunk 64"}})
        print(json.dumps(line), flush=True)
        return
    if args.workload == "qmv":
        # one kernel only (what the rocprofv3 passes under profiles/ run)
        log(f"qmv roofline {args.qmv}")
        line["roofline"] = roofline(args.qmv)
        line["read_roof_calibration_bytes"] = read_roof_calibration()
        M, N, K = ROOF_KERNELS[args.qmv][:3]
        line.update({"value": line["roofline"]["achieved"], "unit": "GB/s",
                     "ms_per_step": line["roofline"]["avg_launch_us"] / 1e3,
                     "config": {"workload": f"4-bit group-64 qmv, x bf16 [{M},{K}], W [{N},{K}]"}})
    else:
        log("qmv roofline (dominant kernel of the cycle)")
        line["roofline"] = roofline("gate_up_m4")
        log("qmv roofline (config 0 GEMV)")
        line["qmv_config0"] = roofline("config0")
    if not args.no_shapes:
        log("config-1 shapes")
        line["qmv_shapes"] = qmv_shapes()
        log("config-2 verify (GDN) and config-3 sampler")
        line["gdn_config2_verify"] = gdn_config2_verify()
        line["spec_config3"] = spec_config3()
        log("config-2 prefill (chunked GDN)")
        line["gdn_config2_prefill"] = gdn_config2_prefill()
        log("the cycle's other hot kernels (DeltaNet mixer, verify attention)")
        att = attn_verify()
        gbs = att["bytes"] / (att["two_launch_us"] * 1e-6) / 1e9
        line["cycle_kernels"] = {
            "gdn_mixer": mixer_verify(),
            "attention": {"kernel": "qvex_attn_qk_rope + qvex_attention (the cycle's path: q/k norm, RoPE and KV "
                                    "append, then the split-K partial and the combine)",
                          "ctx": att["ctx"], "us": att["two_launch_us"], "GB/s": round(gbs, 1),
                          "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": att["bytes"],
                          "fused_decode_us": att["us"]},
        }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        tpc = res["tokens_per_cycle"] if res else 1.0
        line["cpu_baseline"] = cpu_baseline(cfg, args.k, tpc)
        if not args.no_shapes:
            log("cpu baselines per config")
            line["cpu_baselines"] = cpu_baselines()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
