"""qmv HIP kernel vs the fp64 oracle (GPU).

Tolerance per output: |y - y64| <= 2^-8 |y64| + 2^-14 * sum_k |x_k w_nk|
(bf16 output rounding plus fp32 accumulation of the +128-offset dot products).
"""

import numpy as np
import pytest
import torch

import oracle
from qvex import kernels, synth

TILES = [(r, ks) for r in (1, 2, 4, 8) for ks in (1, 2, 4)]
MFMA_TILES = [("mfma", tn, ws) for tn in (1, 2, 4) for ws in (1, 2, 4, 8)]


def to_dev(a, dtype):
    a = np.ascontiguousarray(a)
    if dtype == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16)).to("cuda:0").view(torch.bfloat16)
    if dtype == torch.int32:
        return torch.from_numpy(a.view(np.int32)).to("cuda:0")
    return torch.from_numpy(a).to("cuda:0")


def run(x, w, s, b, tile=None):
    xd, wd = to_dev(x, torch.bfloat16), to_dev(w, torch.int32)
    sd, bd = to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16)
    y = kernels.quantized_matmul(xd, wd, sd, bd, tile=tile)
    torch.cuda.synchronize()
    return y.view(torch.int16).cpu().numpy().view(np.uint16)


def check(x, w, s, b, y_bits, rows=None):
    K = x.shape[1]
    if rows is None:
        rows = np.arange(w.shape[0])
    ref = oracle.qmv_f64(x, w[rows], s[rows], b[rows])
    dense = np.abs(oracle.dequant_w4_f64(w[rows], s[rows], b[rows], K))
    cond = np.abs(oracle.bf16_to_f32(x).astype(np.float64)) @ dense.T
    got = oracle.bf16_to_f32(y_bits[:, rows]).astype(np.float64)
    err = np.abs(got - ref)
    tol = 2.0 ** -8 * np.abs(ref) + 2.0 ** -14 * cond
    rel = float((err / np.maximum(np.abs(ref), 1e-30)).max())
    print(f"max_abs={err.max():.3e} max_rel={rel:.3e} worst_ratio={(err / tol).max():.3f}")
    assert np.all(err <= tol), f"max err/tol {(err / tol).max():.3f}"


@pytest.mark.gpu
def test_config0_gemv():
    N, K = 12288, 4096
    w, s, b = synth.qmv_weights(N, K)
    x = synth.qmv_x(1, K)
    y = run(x, w, s, b)
    check(x, w, s, b, y)


@pytest.mark.gpu
@pytest.mark.parametrize("M", range(1, 9))
def test_verify_rows(M):
    N, K = 4096, 4096
    w, s, b = synth.qmv_weights(N, K, tag=M)
    x = synth.qmv_x(M, K, tag=M)
    check(x, w, s, b, run(x, w, s, b))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["down", "qkvz", "gdn_in_proj", "attn_kv_proj", "mtp_fc"])
@pytest.mark.parametrize("M", [1, 4, 5])
def test_layer_shapes(name, M):
    K, N = {**synth.SKINNY_SHAPES, **synth.FUSED_SHAPES}[name]
    w, s, b = synth.qmv_weights(N, K, seed=synth.SEED_SKINNY, tag=N)
    x = synth.qmv_x(M, K, seed=synth.SEED_SKINNY, tag=M)
    rows = np.random.default_rng(N).choice(N, size=min(N, 1024), replace=False)
    check(x, w, s, b, run(x, w, s, b), rows=np.sort(rows))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4])
def test_lm_head_rows(M):
    K, N = synth.SKINNY_SHAPES["lm_head"]
    w, s, b = synth.qmv_weights(N, K, seed=synth.SEED_SKINNY, tag=N)
    x = synth.qmv_x(M, K, seed=synth.SEED_SKINNY, tag=M)
    y = run(x, w, s, b)
    rows = np.concatenate([np.arange(64), np.arange(N - 64, N),
                           np.random.default_rng(3).choice(N, 1024, replace=False)])
    check(x, w, s, b, y, rows=np.unique(rows))


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(1, 64), (7, 128), (33, 192), (5, 4160), (130, 960)])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_ragged_shapes(M, N, K):
    w, s, b = synth.qmv_weights(N, K, seed=5, tag=N * K)
    x = synth.qmv_x(M, K, seed=5, tag=M)
    check(x, w, s, b, run(x, w, s, b))


@pytest.mark.gpu
@pytest.mark.parametrize("tile", TILES)
def test_every_tile(tile):
    M, N, K = 3, 515, 2112
    w, s, b = synth.qmv_weights(N, K, seed=6)
    x = synth.qmv_x(M, K, seed=6)
    check(x, w, s, b, run(x, w, s, b, tile=tile))


@pytest.mark.gpu
def test_rows_bitwise_independent_of_m():
    N, K = 1000, 1024
    w, s, b = synth.qmv_weights(N, K, seed=8)
    x = synth.qmv_x(5, K, seed=8)
    full = run(x, w, s, b, tile=(2, 1))
    for m in range(5):
        one = run(x[m:m + 1], w, s, b, tile=(2, 1))
        assert np.array_equal(full[m], one[0])


@pytest.mark.gpu
def test_closed_forms():
    N, K = 256, 512
    w = np.full((N, K // 8), 0x88888888, np.uint32)
    s = oracle.bf16_bits(np.full((N, K // 64), 0.0123, np.float32))
    b = oracle.bf16_bits(-8 * oracle.bf16_to_f32(s))
    x = synth.qmv_x(2, K, seed=3)
    y = oracle.bf16_to_f32(run(x, w, s, b))
    assert np.abs(y).max() < 1e-4
    w, s, b = synth.qmv_weights(N, K, seed=4)
    one = oracle.bf16_bits(np.ones((N, K // 64), np.float32))
    zero = oracle.bf16_bits(np.zeros((N, K // 64), np.float32))
    xi = np.random.default_rng(5).integers(-3, 4, size=(2, K)).astype(np.float32)
    got = oracle.bf16_to_f32(run(oracle.bf16_bits(xi), w, one, zero)).astype(np.float64)
    want = (xi.astype(np.int64) @ oracle.unpack_w4(w, K).astype(np.int64).T).astype(np.float64)
    # integers up to ~2^14 round to bf16; compare after the same rounding
    assert np.array_equal(got, oracle.bf16_to_f32(oracle.bf16_bits(want.astype(np.float32))))


@pytest.mark.gpu
@pytest.mark.parametrize("tile", MFMA_TILES)
@pytest.mark.parametrize("M", [1, 3, 4, 5, 8])
def test_mfma_tiles(tile, M):
    N, K = 531, 2304
    w, s, b = synth.qmv_weights(N, K, seed=16, tag=M)
    x = synth.qmv_x(M, K, seed=16, tag=M)
    check(x, w, s, b, run(x, w, s, b, tile=tile))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4, 5])
@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288), (248320, 4096)])
def test_mfma_model_shapes(M, shape):
    N, K = shape
    w, s, b = synth.qmv_weights(N, K, seed=synth.SEED_SKINNY, tag=N)
    x = synth.qmv_x(M, K, seed=synth.SEED_SKINNY, tag=M)
    y = run(x, w, s, b, tile=("mfma", 2, 1))
    rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 32, N),
                                     np.random.default_rng(N).choice(N, 1024, replace=False)]))
    check(x, w, s, b, y, rows=rows)


# ---------------------------------------------------------------- dense (prefill) path

def _dequant_np(w, s, b):
    """bf16(s * q + b) with the product and sum in fp32 (one rounding), in numpy."""
    N, KW = w.shape
    K = KW * 8
    q = np.stack([(w >> (4 * j)) & 0xF for j in range(8)], axis=-1).reshape(N, K).astype(np.float32)
    sc = np.repeat(synth.bf16_to_f32(s), 64, axis=1).astype(np.float32)
    bi = np.repeat(synth.bf16_to_f32(b), 64, axis=1).astype(np.float32)
    prod = (sc.astype(np.float64) * q + bi).astype(np.float32)   # fma: exact product, one rounding
    return synth.bf16_bits(prod)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(256, 512), (12352, 4096), (64, 12288)])
def test_dequant_bit_exact(N, K):
    w, s, b = synth.qmv_weights(N, K, seed=5, tag=N)
    out = kernels.dequant_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    torch.cuda.synchronize()
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, _dequant_np(w, s, b))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [16, 100, 512])
def test_dense_prefill_product(M):
    """QLinear with M >= DENSE_MIN_ROWS: bf16(x W~^T) with W~ the bf16 dequantized
    weight and fp32 accumulation: within bf16 output rounding plus 2^-8 of
    sum |x||w| (weight rounding, accumulation) of the exact affine product."""
    from qvex.model import QLinear
    N, K = 1024, 4096
    w, s, b = synth.qmv_weights(N, K, seed=6, tag=M)
    lin = QLinear(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    assert M >= QLinear.DENSE_MIN_ROWS
    x = synth.qmv_x(M, K, seed=6, tag=M)
    y = lin(to_dev(x, torch.bfloat16))
    torch.cuda.synchronize()
    xf = synth.bf16_to_f32(x).astype(np.float64)
    q = np.stack([(w >> (4 * j)) & 0xF for j in range(8)], axis=-1).reshape(N, K).astype(np.float64)
    W = q * np.repeat(synth.bf16_to_f32(s), 64, axis=1) + np.repeat(synth.bf16_to_f32(b), 64, axis=1)
    ref = xf @ W.T
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -8 * (np.abs(xf) @ np.abs(W).T)
    err = np.abs(y.float().cpu().numpy().astype(np.float64) - ref)
    assert (err <= bound).all(), float((err - bound).max())
