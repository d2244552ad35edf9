"""CPU restatement of QVex's MTP verify-path arithmetic — the oracle.

TEST INFRASTRUCTURE ONLY. This package is the checker for libqvex.so: only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import it, and
never as the thing being measured or shipped. The product path
(qvex-3.5_amd/qvex) does not import it and fails loudly without its HIP library.

Contents:
  * liboracle.so (oracle/*.c, built by oracle/Makefile): fp64 qmv, fp64/fp32
    Gated DeltaNet recurrence, fp32-emulation speculative acceptance;
  * numpy helpers: bf16 rounding, the MLX affine pack/unpack of any width
    (quant/quantize.py:71-75) with its fp64 dequant and product, and a numpy
    layer-level restatement (oracle.model) of the verify forward.

Pinning (what checks each function against something other than itself) is
listed per function below; each is exercised in tests/test_oracle.py.
  - qmv_f64: independent numpy dequant (np.unpackbits, quant/quantize.py:71-75)
    + float64 matmul; closed forms (q = 8 with b = -8s gives 0; x = e_k gives
    column k; s = 1, b = 0 gives an exact integer GEMV); golden fixtures.
  - pack_bits / unpack_bits / dequant_f64 / qmv_affine_f64 (any width):
    codes against a Python-integer stream (sum of q_k << bits*k, cut into
    32-bit words), hand-worked 2-, 3- and 8-bit words, pack_w4 at 4 bits,
    qmv_f64 (C) at 4-bit group 64, scale/bias shared within a group and a
    zero product where every code is the bias midpoint
    (tests/test_oracle_affine.py).
  - gated_delta_f64: matrix form S_t = g S (I - b k k^T) + b v k^T (a different
    formulation); delta-rule invariants (g = 1, b = 0 keeps S; g = 1, b = 1,
    |k| = 1 gives S k = v); T-step = T one-step calls; golden fixtures.
  - philox4x32_10 / philox_uniforms: the known-answer vectors published with
    Philox (Salmon et al. 2011); the uniform law (moments, equidistribution).
  - spec_accept: textbook rule checked by exhaustive enumeration on tiny
    vocabularies, p == q accepts all, p(d) = 0 rejects, greedy limit, chi^2 of
    the emitted-token law; orc_expf within 2 ulp of float64 exp.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# QVEX_ORACLE_LIB names another build of the same sources (the sanitizer build
# of `make asan`, which tests/test_oracle_asan.py runs the oracle tests on)
LIB_PATH = Path(os.environ["QVEX_ORACLE_LIB"]) if os.environ.get("QVEX_ORACLE_LIB") else HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile (always rebuilds)."""
    r = subprocess.run(["make", "-B", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int
        F = ctypes.c_float
        L.orc_qmv_w4g64_f64.argtypes = [P, P, P, P, P, I, I, I]
        L.orc_qmv_w4g64_f32.argtypes = [P, P, P, P, P, I, I, I, I]
        L.orc_gated_delta_f64.argtypes = [P] * 10 + [I] * 6
        L.orc_gated_delta_f32.argtypes = [P] * 10 + [I] * 7
        L.orc_spec_accept.argtypes = [P, P, P, P, P, F, P, P, I, I, I, I]
        L.orc_spec_accept_filtered.argtypes = [P, P, P, P, P, F, P, F, I, F, P, P, I, I, I, I]
        L.orc_philox4x32_10.argtypes = [P, P, P]
        L.orc_philox4x32_10.restype = None
        L.orc_philox_uniforms.argtypes = [ctypes.c_uint64, ctypes.c_uint64, I, P]
        L.orc_philox_uniforms.restype = None
        L.orc_row_filter.argtypes = [P, I, F, P, F, I, F, P]
        L.orc_row_filter.restype = None
        L.orc_expf.argtypes = [F]
        L.orc_expf.restype = F
        for fn in ("orc_qmv_w4g64_f64", "orc_qmv_w4g64_f32", "orc_gated_delta_f64",
                   "orc_gated_delta_f32", "orc_spec_accept", "orc_spec_accept_filtered"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- bf16

def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(a))


# ---------------------------------------------------------------- MLX 4-bit layout

def pack_w4(q: np.ndarray) -> np.ndarray:
    """uint8 codes [N, K] -> uint32 [N, K/8]: each row a little-endian bit stream
    of 4-bit codes (restates quant/quantize.py:71-75 for bits=4)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape
    bits = np.unpackbits(q[..., None], axis=-1, bitorder="little")[..., :4].reshape(N, K * 4)
    return np.ascontiguousarray(np.packbits(bits, axis=-1, bitorder="little").view(np.uint32))


def unpack_w4(w: np.ndarray, K: int) -> np.ndarray:
    """uint32 [N, K/8] -> uint8 codes [N, K] (inverse of pack_w4)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    N = w.shape[0]
    bits = np.unpackbits(w.view(np.uint8), axis=-1, bitorder="little").reshape(N, K, 4)
    return np.packbits(bits, axis=-1, bitorder="little")[..., 0]


def dequant_w4_f64(w, scales_bits, biases_bits, K) -> np.ndarray:
    """Dense float64 [N, K] weight = s * q + b per 64-wide group."""
    q = unpack_w4(w, K).astype(np.float64)
    s = np.repeat(bf16_to_f32(scales_bits).astype(np.float64), 64, axis=1)
    b = np.repeat(bf16_to_f32(biases_bits).astype(np.float64), 64, axis=1)
    return s * q + b


# ---------------------------------------------------------------- MLX affine layout, any width

def pack_bits(q: np.ndarray, bits: int) -> np.ndarray:
    """uint8 codes [N, K] -> uint32 [N, K*bits/32]: each row a little-endian bit
    stream of `bits`-bit codes (restates quant/quantize.py:71-75)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape
    assert (K * bits) % 32 == 0
    stream = np.unpackbits(q[..., None], axis=-1, bitorder="little")[..., :bits].reshape(N, K * bits)
    return np.ascontiguousarray(np.packbits(stream, axis=-1, bitorder="little").view(np.uint32))


def unpack_bits(w: np.ndarray, K: int, bits: int) -> np.ndarray:
    """uint32 [N, K*bits/32] -> uint8 codes [N, K] (inverse of pack_bits)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    N = w.shape[0]
    stream = np.unpackbits(w.view(np.uint8), axis=-1, bitorder="little").reshape(N, K, bits)
    pad = np.zeros((N, K, 8 - bits), np.uint8)
    return np.packbits(np.concatenate([stream, pad], axis=-1), axis=-1, bitorder="little")[..., 0]


def dequant_f64(w, scales_bits, biases_bits, K: int, bits: int, group_size: int) -> np.ndarray:
    """Dense float64 [N, K] weight = s * q + b per group (mx.dequantize)."""
    q = unpack_bits(w, K, bits).astype(np.float64)
    s = np.repeat(bf16_to_f32(scales_bits).astype(np.float64), group_size, axis=1)
    b = np.repeat(bf16_to_f32(biases_bits).astype(np.float64), group_size, axis=1)
    return s * q + b


def qmv_affine_f64(x_bits, w, scales_bits, biases_bits, bits: int, group_size: int,
                   row_block: int = 4096) -> np.ndarray:
    """fp64 y [M, N] = x @ dequant(W)^T for any width (mx.quantized_matmul,
    engine/model.py:87-91), dequantizing row_block weight rows at a time."""
    x = bf16_to_f32(np.ascontiguousarray(x_bits, dtype=np.uint16)).astype(np.float64)
    N = w.shape[0]
    K = x.shape[1]
    y = np.empty((x.shape[0], N), np.float64)
    for r0 in range(0, N, row_block):
        r1 = min(N, r0 + row_block)
        y[:, r0:r1] = x @ dequant_f64(w[r0:r1], scales_bits[r0:r1], biases_bits[r0:r1], K, bits, group_size).T
    return y


# ---------------------------------------------------------------- qmv

def qmv_f64(x_bits, w, scales_bits, biases_bits) -> np.ndarray:
    """fp64 y [M, N] of the 4-bit group-64 matmul (C loop, engine/kernels.py:121)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x_bits.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float64)
    lib().orc_qmv_w4g64_f64(_p(x_bits), _p(np.ascontiguousarray(w, np.uint32)),
                            _p(np.ascontiguousarray(scales_bits, np.uint16)),
                            _p(np.ascontiguousarray(biases_bits, np.uint16)), _p(y), M, N, K)
    return y


def qmv_f32(x_bits, w, scales_bits, biases_bits, threads: int = 1) -> np.ndarray:
    """fp32-accumulated, bf16-rounded y (bits) — the CPU baseline restatement."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x_bits.shape
    N = w.shape[0]
    assert M <= 8
    y = np.empty((M, N), np.uint16)
    lib().orc_qmv_w4g64_f32(_p(x_bits), _p(np.ascontiguousarray(w, np.uint32)),
                            _p(np.ascontiguousarray(scales_bits, np.uint16)),
                            _p(np.ascontiguousarray(biases_bits, np.uint16)), _p(y), M, N, K, threads)
    return y


# ---------------------------------------------------------------- Gated DeltaNet

def gated_delta_f64(q, k, v, a, b, A_log, dt_bias, state, snaps=True):
    """fp64 recurrence (engine/kernels.py:34-63). Inputs are float32 arrays holding
    the (bf16-representable) kernel inputs; state fp32/fp64 [B,Hv,Dv,Dk].
    Returns y [B,T,Hv,Dv], final state, snapshots [T,B,Hv,Dv,Dk] (or None)."""
    q, k, v, a, b = (np.ascontiguousarray(t, np.float32) for t in (q, k, v, a, b))
    A_log = np.ascontiguousarray(A_log, np.float32)
    dt_bias = np.ascontiguousarray(dt_bias, np.float32)
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2:]
    st = np.array(state, dtype=np.float64, order="C", copy=True)
    y = np.empty((B, T, Hv, Dv), np.float64)
    sn = np.empty((T, B, Hv, Dv, Dk), np.float64) if snaps else None
    lib().orc_gated_delta_f64(_p(q), _p(k), _p(v), _p(a), _p(b), _p(A_log), _p(dt_bias),
                              _p(st), _p(y), _p(sn), B, T, Hk, Hv, Dk, Dv)
    return y, st, sn


def gated_delta_f32(q, k, v, a, b, A_log, dt_bias, state, snaps=False, threads=1):
    q, k, v, a, b = (np.ascontiguousarray(t, np.float32) for t in (q, k, v, a, b))
    A_log = np.ascontiguousarray(A_log, np.float32)
    dt_bias = np.ascontiguousarray(dt_bias, np.float32)
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2:]
    st = np.array(state, dtype=np.float32, order="C", copy=True)
    y = np.empty((B, T, Hv, Dv), np.float32)
    sn = np.empty((T, B, Hv, Dv, Dk), np.float32) if snaps else None
    lib().orc_gated_delta_f32(_p(q), _p(k), _p(v), _p(a), _p(b), _p(A_log), _p(dt_bias),
                              _p(st), _p(y), _p(sn), B, T, Hk, Hv, Dk, Dv, threads)
    return y, st, sn


# ---------------------------------------------------------------- speculative acceptance

def spec_accept(target, draft, draft_ids, u_accept, u_sample, inv_temp, threads=1, seen=None,
                presence_penalty=0.0, top_k=0, top_p=1.0):
    """Bit-exact fp32 emulation of the fused acceptance kernel (see oracle/spec.c).
    target [S,k+1,V] fp32, draft [S,k,V] fp32 or None (one-hot greedy draft),
    draft_ids [S,k] int32, u_accept [S,k], u_sample [S]; inv_temp <= 0 = greedy.
    seen [V] fp32 (0/1) or None, presence_penalty, top_k (0..64), top_p: the
    target rows are filtered as Sampler.scores (engine/sampler.py:30-52).
    Returns (n_accept [S] int32, out_token [S] int32)."""
    target = np.ascontiguousarray(target, np.float32)
    S, k1, V = target.shape
    k = k1 - 1
    if draft is not None:
        draft = np.ascontiguousarray(draft, np.float32)
        assert draft.shape == (S, k, V)
    draft_ids = np.ascontiguousarray(draft_ids, np.int32).reshape(S, k)
    u_accept = np.ascontiguousarray(u_accept, np.float32).reshape(S, k)
    u_sample = np.ascontiguousarray(u_sample, np.float32).reshape(S)
    if seen is not None:
        seen = np.ascontiguousarray(seen, np.float32).reshape(V)
    n = np.empty(S, np.int32)
    tok = np.empty(S, np.int32)
    lib().orc_spec_accept_filtered(_p(target), _p(draft), _p(draft_ids), _p(u_accept), _p(u_sample),
                                   float(np.float32(inv_temp)), _p(seen), float(np.float32(presence_penalty)),
                                   int(top_k), float(np.float32(top_p)), _p(n), _p(tok), S, k, V, threads)
    return n, tok


# ---------------------------------------------------------------- uniforms

def philox4x32_10(ctr, key) -> np.ndarray:
    """One Philox4x32-10 block (Salmon et al. 2011) of 4 uint32 words."""
    c = np.ascontiguousarray(ctr, np.uint32).reshape(4)
    k = np.ascontiguousarray(key, np.uint32).reshape(2)
    out = np.empty(4, np.uint32)
    lib().orc_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def philox_uniforms(seed: int, event: int, n: int) -> np.ndarray:
    """The sampler's n uniforms of draw event `event` (oracle/rng.c)."""
    out = np.empty(n, np.float32)
    lib().orc_philox_uniforms(int(seed) & (2**64 - 1), int(event), int(n), _p(out))
    return out


def row_filter(row, inv_temp, seen=None, presence_penalty=0.0, top_k=0, top_p=1.0):
    """(c_0, S_p, cutoff) of one target row: the filter record of oracle/spec.c."""
    row = np.ascontiguousarray(row, np.float32).reshape(-1)
    if seen is not None:
        seen = np.ascontiguousarray(seen, np.float32).reshape(-1)
    out = np.empty(3, np.float32)
    lib().orc_row_filter(_p(row), row.size, float(np.float32(inv_temp)), _p(seen),
                         float(np.float32(presence_penalty)), int(top_k), float(np.float32(top_p)), _p(out))
    return out


def expf(x: float) -> float:
    return lib().orc_expf(float(x))
