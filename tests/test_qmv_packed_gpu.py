"""Tile-packed 4-bit qmv (qvex_w4g64_pack + qvex_qmv_w4g64_packed) vs the
float64 oracle of mx.quantized_matmul (engine/model.py:87-91), same tolerance
as the MLX-layout kernel: |err| <= 2^-8 |ref| + 2^-14 sum|x||w| (bf16 output
rounding plus fp32 accumulation)."""

import numpy as np
import pytest
import torch

from qvex import kernels, synth
from test_qmv_gpu import check, to_dev

PACKED_TILES = [(tn, ws) for tn in (1, 2, 4) for ws in (1, 2, 4, 8)] + [(1, 16)]


def run_packed(x, w, s, b, tile=None):
    wd, sd, bd = to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16)
    packed = kernels.pack_w4(wd, sd, bd)
    y = kernels.quantized_matmul_packed(to_dev(x, torch.bfloat16), packed, w.shape[0], tile=tile)
    torch.cuda.synchronize()
    return y.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.gpu
@pytest.mark.parametrize("tile", PACKED_TILES)
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_packed_tiles(tile, M):
    if M > 4 and tile[0] == 4:
        pytest.skip("5..8 rows run one or two tiles per wave (what the default tiles pick)")
    N, K = 531, 2304                       # ragged last tile, 9 sets
    w, s, b = synth.qmv_weights(N, K, seed=31, tag=M)
    x = synth.qmv_x(M, K, seed=31, tag=M)
    check(x, w, s, b, run_packed(x, w, s, b, tile=tile))


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(1, 256), (16, 256), (17, 512), (100, 4096), (4096, 256)])
def test_packed_edge_shapes(N, K):
    w, s, b = synth.qmv_weights(N, K, seed=32, tag=N)
    x = synth.qmv_x(4, K, seed=32, tag=K)
    check(x, w, s, b, run_packed(x, w, s, b))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("shape", [(24576, 4096), (4096, 12288), (12352, 4096), (248320, 4096), (4096, 8192)])
def test_packed_model_shapes(M, shape):
    N, K = shape
    w, s, b = synth.qmv_weights(N, K, seed=synth.SEED_SKINNY, tag=N)
    x = synth.qmv_x(M, K, seed=synth.SEED_SKINNY, tag=M)
    y = run_packed(x, w, s, b)
    rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 32, N),
                                     np.random.default_rng(N).choice(N, 1024, replace=False)]))
    check(x, w, s, b, y, rows=rows)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(12352, 4096), (4096, 12288), (248320, 4096)])
def test_packed_rows_bitwise_independent_of_m(N, K):
    """Verify (M = k + 1) and plain decode (M = 1) see the same bits for a row."""
    w, s, b = synth.qmv_weights(N, K, seed=33, tag=N)
    x4 = synth.qmv_x(4, K, seed=33, tag=K)
    y4 = run_packed(x4, w, s, b)
    for m in range(4):
        y1 = run_packed(x4[m:m + 1], w, s, b)
        assert np.array_equal(y1[0], y4[m]), f"row {m} differs between M=1 and M=4"
    y2 = run_packed(x4[1:3], w, s, b)
    assert np.array_equal(y2, y4[1:3])
    # 5..8 rows (two row halves in one launch): each row as in the 4-row calls
    x8 = np.concatenate([x4, synth.qmv_x(4, K, seed=34, tag=K)])
    y8 = run_packed(x8, w, s, b)
    assert np.array_equal(y8[:4], y4)
    assert np.array_equal(y8[4:], run_packed(x8[4:], w, s, b))
    assert np.array_equal(run_packed(x8[:5], w, s, b), y8[:5])


@pytest.mark.gpu
def test_packed_matches_mlx_layout_kernel_closely():
    """Same product as the MLX-layout kernel (different summation order)."""
    N, K = 2048, 4096
    w, s, b = synth.qmv_weights(N, K, seed=34)
    x = synth.qmv_x(4, K, seed=34)
    from test_qmv_gpu import run
    a = synth.bf16_to_f32(run_packed(x, w, s, b)).astype(np.float64)
    c = synth.bf16_to_f32(run(x, w, s, b)).astype(np.float64)
    assert np.abs(a - c).max() <= 2.0 ** -7 * np.abs(c).max()


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8])
@pytest.mark.parametrize("N,K", [(24576, 4096), (48, 512), (4096, 256)])
def test_packed_swiglu_equals_product_then_swiglu(M, N, K):
    """The fused SwiGLU epilogue matches the packed product followed by qvex_swiglu
    (_swiglu of engine/model.py:134-135 on the two bf16 halves). A row sits in a
    different block in the interleaved pack, so the per-set accumulation order,
    and with it the rounding of g and u, may differ: within two bf16 steps (a
    wrong interleave is off by far more)."""
    from qvex import _C
    from qvex.kernels import _ptr, _stream
    w, s, b = synth.qmv_weights(N, K, seed=35, tag=N)
    x = to_dev(synth.qmv_x(M, K, seed=35, tag=M), torch.bfloat16)
    wd, sd, bd = to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16)
    gu = kernels.quantized_matmul_packed(x, kernels.pack_w4(wd, sd, bd), N)
    ref = torch.empty((M, N // 2), dtype=torch.bfloat16, device="cuda:0")
    _C.call("qvex_swiglu", _ptr(gu), _ptr(ref), M, N // 2, _stream())
    got = kernels.quantized_matmul_packed(x, kernels.pack_w4(wd, sd, bd, swiglu=True), N, swiglu=True)
    torch.cuda.synchronize()
    d = (got.float() - ref.float()).abs()
    assert bool((d <= 2.0 ** -6 * ref.float().abs() + 2.0 ** -10).all()), float(d.max())


def default_tile(N, K):
    """The tile qvex_qmv_w4g64_packed picks (packed_default_tile)."""
    tiles, GS = (N + 15) // 16, K // 256
    tn = 2 if tiles >= 704 else 1
    limit, ws_max = (4096, 16) if tn == 1 else (3072, 8)
    ws = 2 if GS >= 8 else 1
    while ws < ws_max and (tiles // tn) * ws < limit and GS >= 2 * (ws * 2):
        ws *= 2
    if tiles // tn >= 4096 and GS >= 8 and ws < 4:
        ws = 4
    if GS >= 48 and ws > 8:
        ws = 8
    if tn == 2 and tiles < 1024 and GS >= 8:
        tn, ws = 1, 2
    return tn, ws


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("N,K", [(4096, 12288), (12352, 4096), (4096, 4096), (24576, 4096), (4096, 8192),
                                 (531, 2304), (17, 512), (4096, 256), (100, 1280), (131072, 2048)])
def test_prefetch_pipeline_equals_double_buffer(M, N, K):
    """The default entry (all of a wave's sets in flight when they fit) and the
    explicit-tile entry (two-deep pipeline) with the same tile give the same bits."""
    w, s, b = synth.qmv_weights(N, K, seed=36, tag=N)
    x = synth.qmv_x(M, K, seed=36, tag=K)
    auto = run_packed(x, w, s, b)
    two = run_packed(x, w, s, b, tile=(*default_tile(N, K), 0))
    assert np.array_equal(auto, two)


@pytest.mark.gpu
@pytest.mark.parametrize("tile", [(1, 16, 2), (1, 16, 4), (1, 16, 0), (1, 8, 8), (2, 4, 4), (1, 2, 8)])
def test_prefetch_explicit_tiles(tile):
    N, K = 531, 2304 * 2                   # ragged last tile, 18 sets
    GS = K // 256
    if tile[2] and -(-GS // tile[1]) > tile[2]:
        pytest.skip("the wave's sets do not fit the prefetch depth")
    w, s, b = synth.qmv_weights(N, K, seed=37, tag=tile[1])
    x = synth.qmv_x(4, K, seed=37, tag=tile[2])
    y = run_packed(x, w, s, b, tile=tile)
    check(x, w, s, b, y)
    assert np.array_equal(y, run_packed(x, w, s, b, tile=(*tile[:2], 0)))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3, 4, 7])
@pytest.mark.parametrize("N,K,ties", [(248320, 4096, False), (4096, 512, True), (531, 2304, True), (50000, 1024, False)])
def test_argmax_epilogue_equals_argmax_of_product(M, N, K, ties):
    """qvex_qmv_w4g64_packed_argmax == the first index of the maximum of the bf16
    product (the greedy pick over the lm_head's output), also with exact ties
    (duplicated weight rows) and with the folded-norm row scale."""
    from qvex.model import NormedRows
    w, s, b = synth.qmv_weights(N, K, seed=38, tag=N)
    if ties:
        g = np.random.default_rng(N)
        src = g.integers(0, N, 64)
        dst = g.integers(0, N, 64)
        w[dst], s[dst], b[dst] = w[src], s[src], b[src]
    packed = kernels.pack_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    x = to_dev(synth.qmv_x(M, K, seed=38, tag=M), torch.bfloat16)
    out = torch.empty(M, dtype=torch.int32, device="cuda:0")
    kernels.qmv_packed_argmax(x, packed, N, out)
    y = kernels.quantized_matmul_packed(x, packed, N).float()
    want = torch.tensor([int(torch.nonzero(y[r] == y[r].max())[0]) for r in range(M)], dtype=torch.int32)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)
    g = torch.Generator().manual_seed(M)
    h = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16).to("cuda:0")
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).to("cuda:0")
    st = NormedRows.of(h, nw, 1e-6)
    kernels.qmv_packed_argmax(st.u, packed, N, out, st.parts, 1e-6)
    y2 = kernels.qmv_packed_rstd(st.u, packed, N, st.parts, 1e-6).float()
    want2 = torch.tensor([int(torch.nonzero(y2[r] == y2[r].max())[0]) for r in range(M)], dtype=torch.int32)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want2)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [5, 7, 8, 13])
@pytest.mark.parametrize("swiglu", [False, True])
def test_qlinear_rows_5_to_15_equal_single_row_calls(M, swiglu):
    """QLinear runs 5..15 rows through the packed kernel (5..8 in one launch, more
    in chunks of 8): every row has the bits of the same row computed alone (as
    decode computes it)."""
    from qvex.model import QLinear
    N, K = 1024, 2048
    w, s, b = synth.qmv_weights(N, K, seed=41, tag=M)
    lin = QLinear(torch.from_numpy(w.view(np.int32)).to("cuda:0"),
                  torch.from_numpy(s.view(np.int16)).to("cuda:0").view(torch.bfloat16),
                  torch.from_numpy(b.view(np.int16)).to("cuda:0").view(torch.bfloat16), swiglu=swiglu)
    assert lin.packed is not None and M < QLinear.DENSE_MIN_ROWS
    x = torch.from_numpy(synth.qmv_x(M, K, seed=41, tag=M).view(np.int16)).to("cuda:0").view(torch.bfloat16)
    f = lin.swiglu if swiglu else lin
    wide = f(x)
    rows = torch.cat([f(x[r:r + 1]) for r in range(M)])
    torch.cuda.synchronize()
    assert torch.equal(wide, rows)
    # and the values are the product's (plain: against the MLX-layout kernel)
    if not swiglu:
        ref = torch.cat([kernels.quantized_matmul(x[m0:m0 + 8], lin.w, lin.scales, lin.biases)
                         for m0 in range(0, M, 8)]).float()
        d = (wide.float() - ref).abs()
        assert float((d / (ref.abs() + 1.0)).max()) < 2e-2
