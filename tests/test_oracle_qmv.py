"""Pins the qmv oracle against independent formulations (CPU only)."""

import numpy as np
import pytest

import oracle
from qvex import synth


def test_pack_matches_reference_bit_order():
    # quant/quantize.py:71-75: little-endian bit stream; code k at bits 4*(k%8) of word k/8
    q = np.arange(16, dtype=np.uint8)[None, :].repeat(2, 0)
    w = oracle.pack_w4(q)
    assert w.shape == (2, 2)
    assert w[0, 0] == 0x76543210 and w[0, 1] == 0xFEDCBA98


def test_pack_unpack_round_trip():
    g = np.random.default_rng(0)
    q = g.integers(0, 16, size=(7, 128), dtype=np.uint8)
    assert np.array_equal(oracle.unpack_w4(oracle.pack_w4(q), 128), q)


def test_unpack_matches_shift_mask_formula():
    # engine/kernels.py:164-166: (w >> 4*i) & 0xF
    g = np.random.default_rng(1)
    w = g.integers(0, 2**32, size=(3, 8), dtype=np.uint32)
    q = oracle.unpack_w4(w, 64)
    for n in range(3):
        for k in range(64):
            assert q[n, k] == (int(w[n, k // 8]) >> (4 * (k % 8))) & 0xF


@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (3, 33, 256), (5, 8, 512)])
def test_qmv_f64_matches_dense_dequant(M, N, K):
    w, s, b = synth.qmv_weights(N, K, seed=7, tag=M)
    x = synth.qmv_x(M, K, seed=7, tag=M)
    ref = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.dequant_w4_f64(w, s, b, K).T
    got = oracle.qmv_f64(x, w, s, b)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_qmv_closed_forms():
    N, K = 12, 128
    # q == 8 everywhere with b = -8 s -> exactly zero
    w = np.full((N, K // 8), 0x88888888, np.uint32)
    s = oracle.bf16_bits(np.full((N, K // 64), 0.0123, np.float32))
    b = oracle.bf16_bits(-8 * oracle.bf16_to_f32(s))
    x = synth.qmv_x(2, K, seed=3)
    assert np.all(oracle.qmv_f64(x, w, s, b) == 0.0)
    # x = e_k -> dequantized column k
    w, s, b = synth.qmv_weights(N, K, seed=4)
    xe = np.zeros((1, K), np.float32)
    xe[0, 77] = 1.0
    col = oracle.qmv_f64(oracle.bf16_bits(xe), w, s, b)[0]
    qcol = oracle.unpack_w4(w, K)[:, 77].astype(np.float64)
    sf = oracle.bf16_to_f32(s)[:, 77 // 64].astype(np.float64)
    bf = oracle.bf16_to_f32(b)[:, 77 // 64].astype(np.float64)
    np.testing.assert_array_equal(col, sf * qcol + bf)
    # s = 1, b = 0, small-integer x -> exact integer GEMV
    one = oracle.bf16_bits(np.ones((N, K // 64), np.float32))
    zero = oracle.bf16_bits(np.zeros((N, K // 64), np.float32))
    xi = np.random.default_rng(5).integers(-3, 4, size=(2, K)).astype(np.float32)
    got = oracle.qmv_f64(oracle.bf16_bits(xi), w, one, zero)
    want = xi.astype(np.int64) @ oracle.unpack_w4(w, K).astype(np.int64).T
    assert np.array_equal(got, want.astype(np.float64))


def test_qmv_rows_independent():
    N, K = 20, 192
    w, s, b = synth.qmv_weights(N, K, seed=9)
    x = synth.qmv_x(4, K, seed=9)
    full = oracle.qmv_f64(x, w, s, b)
    for m in range(4):
        np.testing.assert_array_equal(full[m], oracle.qmv_f64(x[m:m + 1], w, s, b)[0])


def test_qmv_f32_baseline_within_bf16():
    N, K = 64, 1024
    w, s, b = synth.qmv_weights(N, K, seed=11)
    x = synth.qmv_x(3, K, seed=11)
    ref = oracle.qmv_f64(x, w, s, b)
    got = oracle.bf16_to_f32(oracle.qmv_f32(x, w, s, b, threads=2)).astype(np.float64)
    tol = 2.0 ** -8 * np.abs(ref) + 1e-3 * np.abs(ref).max()
    assert np.all(np.abs(got - ref) <= tol)
