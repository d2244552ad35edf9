"""Seeded synthetic inputs for the verify-path workloads (numpy PCG64).

All generators are pure numpy on the host so any consumer (GPU run, CPU
baseline, parity test) rebuilds identical bytes from the same seed. bf16
tensors are returned as uint16 bit patterns (round to nearest even).

Workloads (sizes of a Qwen3.5-9B-shaped model):
  qmv:   x ~ N(0,1) bf16 [M,K]; packed words uniform over 2^32 (every nibble
         uniform on 0..15, independent); scales ~ U(0.002, 0.02) bf16;
         biases = -8 * scale (exact in bf16).
  gdn:   q, k ~ N(0,1) then L2-normalised per head, bf16; v ~ N(0,1) bf16;
         a, b ~ N(0,1) bf16 with A_log = 0, dt_bias = 0, so the kernel's gates
         are g = exp(-softplus(a)) and beta = sigmoid(b); state ~ N(0, 0.02) fp32.
  spec:  target logits ~ N(0,3) + 8 at 1..3 seeded positions per row; draft =
         target + N(0,1); draft ids drawn from softmax(draft / T); uniforms
         U(0,1) fp32. Each verify step has its own seed stream, so any subset
         of steps can be regenerated alone.
"""

from __future__ import annotations

import numpy as np

SEED_QMV = 1000
SEED_SKINNY = 1001
SEED_GDN = 1002
SEED_SPEC = 1003
SEED_E2E = 1004

# Qwen3.5-9B-shaped model
HIDDEN = 4096
MLP = 12288
VOCAB = 248320
GDN_HK, GDN_HV, GDN_D = 16, 32, 128


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rng(seed, *stream) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, *stream])))


# ---------------------------------------------------------------- qmv

def qmv_weights(N: int, K: int, seed: int = SEED_QMV, tag: int = 0):
    """(w uint32 [N,K/8], scales bf16 bits [N,K/64], biases bf16 bits [N,K/64])."""
    assert K % 64 == 0
    g = rng(seed, 1, tag)
    w = g.integers(0, 2**32, size=(N, K // 8), dtype=np.uint32)
    s = bf16_bits(g.uniform(0.002, 0.02, size=(N, K // 64)).astype(np.float32))
    b = bf16_bits(-8.0 * bf16_to_f32(s))
    return w, s, b


def qmv_x(M: int, K: int, seed: int = SEED_QMV, tag: int = 0) -> np.ndarray:
    g = rng(seed, 2, tag)
    return bf16_bits(g.standard_normal((M, K), dtype=np.float32))


# Verify-width skinny GEMM shapes (K -> N) of one Qwen3.5-9B-shaped layer plus the lm_head.
SKINNY_SHAPES = {
    "o_proj": (4096, 4096),
    "qkvz": (4096, 8192),
    "gate": (4096, 12288),
    "down": (12288, 4096),
    "lm_head": (4096, 248320),
}
# The reference's fused projections (engine/model.py:243-246, 296).
FUSED_SHAPES = {
    "gdn_in_proj": (4096, 12352),
    "gate_up": (4096, 24576),
    "attn_q_proj": (4096, 8192),
    "attn_kv_proj": (4096, 1024),
    "mtp_fc": (8192, 4096),
}


# ---------------------------------------------------------------- Gated DeltaNet

def gdn_inputs(T: int, seed: int = SEED_GDN, B: int = 1, Hk: int = GDN_HK, Hv: int = GDN_HV,
               Dk: int = GDN_D, Dv: int = GDN_D):
    g = rng(seed, 3, T)

    def l2n(a):
        return a / np.linalg.norm(a, axis=-1, keepdims=True)

    q = bf16_bits(l2n(g.standard_normal((B, T, Hk, Dk))).astype(np.float32))
    k = bf16_bits(l2n(g.standard_normal((B, T, Hk, Dk))).astype(np.float32))
    v = bf16_bits(g.standard_normal((B, T, Hv, Dv), dtype=np.float32))
    a = bf16_bits(g.standard_normal((B, T, Hv), dtype=np.float32))
    b = bf16_bits(g.standard_normal((B, T, Hv), dtype=np.float32))
    A_log = np.zeros(Hv, np.float32)
    dt_bias = np.zeros(Hv, np.uint16)  # bf16 zeros
    state = (0.02 * g.standard_normal((B, Hv, Dv, Dk))).astype(np.float32)
    return dict(q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt_bias=dt_bias, state=state)


# ---------------------------------------------------------------- speculative acceptance

def _softmax64(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.float64)
    e = np.exp(z - z.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def spec_step(step: int, k: int, V: int, temperature: float, seed: int = SEED_SPEC):
    """One verify step: target [k+1,V], draft [k,V] fp32, draft ids [k] int32,
    u_accept [k] fp32, u_sample fp32 scalar."""
    g = rng(seed, 4, step)
    target = (3.0 * g.standard_normal((k + 1, V), dtype=np.float32)).astype(np.float32)
    for r in range(k + 1):
        npos = int(g.integers(1, 4))
        pos = g.choice(V, size=npos, replace=False)
        target[r, pos] += 8.0
    draft = (target[:k] + g.standard_normal((k, V), dtype=np.float32)).astype(np.float32)
    ids = np.empty(k, np.int32)
    p = _softmax64(draft / np.float32(temperature))
    for i in range(k):
        c = np.cumsum(p[i])
        ids[i] = min(int(np.searchsorted(c, g.random() * c[-1], side="right")), V - 1)
    u_accept = g.random(k, dtype=np.float32)
    u_sample = g.random(dtype=np.float32)
    return target, draft, ids, u_accept, np.float32(u_sample)


def spec_inputs(steps, k: int = 4, V: int = VOCAB, temperature: float = 0.7, seed: int = SEED_SPEC,
                threads: int = 1):
    """Stacked spec_step for the given step indices; with threads > 1 the steps
    are generated concurrently (each has its own seed stream, so the bytes do
    not depend on the thread count)."""
    steps = list(steps)
    S = len(steps)
    target = np.empty((S, k + 1, V), np.float32)
    draft = np.empty((S, k, V), np.float32)
    ids = np.empty((S, k), np.int32)
    ua = np.empty((S, k), np.float32)
    us = np.empty(S, np.float32)

    def one(i):
        target[i], draft[i], ids[i], ua[i], us[i] = spec_step(steps[i], k, V, temperature, seed)

    if threads > 1 and S > 1:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(min(threads, S)) as ex:
            list(ex.map(one, range(S)))
    else:
        for i in range(S):
            one(i)
    return dict(target=target, draft=draft, draft_ids=ids, u_accept=ua, u_sample=us)
