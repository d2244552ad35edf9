"""Pins the any-width MLX affine oracle (pack_bits, unpack_bits, dequant_f64,
qmv_affine_f64) against independent formulations (CPU only).

The layout is quant/quantize.py:71-75: each row one little-endian bit stream,
code k at stream bits [k*bits, (k+1)*bits), read as uint32 words."""

import numpy as np
import pytest

import oracle
from qvex import synth

WIDTHS = (2, 3, 4, 5, 6, 8)


def stream_words(q: np.ndarray, bits: int) -> np.ndarray:
    """The packing as Python integers: sum of q_k << (bits * k), cut into words."""
    N, K = q.shape
    out = np.empty((N, K * bits // 32), np.uint32)
    for n in range(N):
        acc = 0
        for k in range(K):
            acc |= int(q[n, k]) << (bits * k)
        for i in range(out.shape[1]):
            out[n, i] = (acc >> (32 * i)) & 0xFFFFFFFF
    return out


@pytest.mark.parametrize("bits", WIDTHS)
def test_pack_matches_integer_stream(bits):
    g = np.random.default_rng(bits)
    q = g.integers(0, 2 ** bits, size=(3, 96), dtype=np.uint8)
    assert np.array_equal(oracle.pack_bits(q, bits), stream_words(q, bits))


def test_pack_known_words():
    # 3 bits: codes 0..7 fill 24 bits 0b111_110_101_100_011_010_001_000 = 0xFAC688;
    # code 8 (= 1) starts at bit 24, code 10 (= 5 = 0b101) straddles bits 30..32
    q = np.array([[0, 1, 2, 3, 4, 5, 6, 7, 1, 0, 5] + [0] * 21], np.uint8)
    w = oracle.pack_bits(q, 3)
    assert w.shape == (1, 3)
    assert w[0, 0] == 0xFAC688 | (1 << 24) | (1 << 30)     # the low bits 01 of code 10
    assert w[0, 1] == 1                                      # its high bit
    # 2 bits: code j at bits 2j of the word; 8 bits: the little-endian bytes
    q2 = np.array([[1, 2, 3, 0] * 8], np.uint8)
    assert oracle.pack_bits(q2, 2)[0, 0] == sum(c << (2 * j) for j, c in enumerate([1, 2, 3, 0] * 4))
    q8 = np.arange(32, dtype=np.uint8)[None, :]
    assert np.array_equal(oracle.pack_bits(q8, 8)[0], q8[0].view("<u4"))


def test_pack_bits_equals_pack_w4():
    g = np.random.default_rng(4)
    q = g.integers(0, 16, size=(5, 256), dtype=np.uint8)
    assert np.array_equal(oracle.pack_bits(q, 4), oracle.pack_w4(q))
    assert np.array_equal(oracle.unpack_bits(oracle.pack_w4(q), 256, 4), q)


@pytest.mark.parametrize("bits", WIDTHS)
def test_unpack_round_trip(bits):
    g = np.random.default_rng(10 + bits)
    q = g.integers(0, 2 ** bits, size=(4, 128), dtype=np.uint8)
    assert np.array_equal(oracle.unpack_bits(oracle.pack_bits(q, bits), 128, bits), q)


@pytest.mark.parametrize("bits,gs", [(3, 64), (5, 32), (2, 128), (8, 32)])
def test_dequant_groups(bits, gs):
    g = np.random.default_rng(bits * gs)
    N, K = 3, 256
    q = g.integers(0, 2 ** bits, size=(N, K), dtype=np.uint8)
    s = oracle.bf16_bits(g.uniform(0.01, 0.1, size=(N, K // gs)).astype(np.float32))
    b = oracle.bf16_bits(g.uniform(-1, 1, size=(N, K // gs)).astype(np.float32))
    d = oracle.dequant_f64(oracle.pack_bits(q, bits), s, b, K, bits, gs)
    for n in range(N):
        for k in (0, gs - 1, gs, K - 1):
            sc, bi = float(oracle.bf16_to_f32(s[n, k // gs])), float(oracle.bf16_to_f32(b[n, k // gs]))
            want = sc * int(q[n, k]) + bi
            assert d[n, k] == want


def test_qmv_affine_equals_c_oracle_at_4bit():
    N, K = 40, 512
    w, s, b = synth.qmv_weights(N, K, seed=21)
    x = synth.qmv_x(3, K, seed=21)
    np.testing.assert_allclose(oracle.qmv_affine_f64(x, w, s, b, 4, 64), oracle.qmv_f64(x, w, s, b),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("bits", WIDTHS)
def test_qmv_affine_closed_forms(bits):
    N, K, gs = 6, 128, 32
    mid = 2 ** (bits - 1)
    # every code at the midpoint with b = -mid * s: exactly zero
    q = np.full((N, K), mid, np.uint8)
    s = oracle.bf16_bits(np.full((N, K // gs), 0.03125, np.float32))
    b = oracle.bf16_bits(-float(q[0, 0]) * oracle.bf16_to_f32(s))
    x = synth.qmv_x(2, K, seed=bits)
    assert np.all(oracle.qmv_affine_f64(x, oracle.pack_bits(q, bits), s, b, bits, gs) == 0.0)
    # s = 1, b = 0, small-integer x: the exact integer product of the codes
    g = np.random.default_rng(bits)
    q = g.integers(0, 2 ** bits, size=(N, K), dtype=np.uint8)
    one = oracle.bf16_bits(np.ones((N, K // gs), np.float32))
    zero = oracle.bf16_bits(np.zeros((N, K // gs), np.float32))
    xi = g.integers(-3, 4, size=(2, K)).astype(np.float32)
    got = oracle.qmv_affine_f64(oracle.bf16_bits(xi), oracle.pack_bits(q, bits), one, zero, bits, gs)
    assert np.array_equal(got, (xi.astype(np.int64) @ q.astype(np.int64).T).astype(np.float64))
