"""Prefill GEMM on the packed copy (qvex_w4g64_packed_gemm[_swiglu]) (GPU).

Reference: x @ W~^T in float64 with W~ the bf16-dequantized weight
bf16(s * q + b) (what the kernel feeds the matrix cores; restated in numpy,
tests/test_qmv_gpu.py:_dequant_np). The kernel accumulates in fp32 and rounds
the output to bf16: |y - ref| <= 2^-8 |ref| + 2^-16 sum |x| |W~|. Ragged M and
N (rows past the block and tiles past the end), K up to 12288, and the
vocabulary-wide shape (checked on a subset of its rows). The fused SwiGLU form
equals the plain GEMM followed by qvex_swiglu bit for bit."""

import numpy as np
import pytest
import torch

from qvex import _C, kernels, synth
from qvex.kernels import _ptr, _stream
from test_qmv_gpu import _dequant_np, to_dev

DEV = "cuda:0"


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(16, 1024, 4096), (37, 12352, 4096), (100, 4096, 12288), (512, 1040, 8192),
                                   (513, 24576, 4096), (1, 272, 256), (64, 248320, 4096)])
def test_packed_gemm_matches_bf16_weight_product(M, N, K):
    w, s, b = synth.qmv_weights(N, K, seed=11, tag=N + M)
    x = synth.qmv_x(M, K, seed=11, tag=M)
    packed = kernels.pack_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    y = kernels.packed_gemm(to_dev(x, torch.bfloat16), packed, N)
    torch.cuda.synchronize()
    rows = np.arange(N) if N <= 25000 else np.concatenate([np.arange(512), np.arange(N - 512, N),
                                                           np.random.default_rng(N).choice(N, 1024, replace=False)])
    Wd = synth.bf16_to_f32(_dequant_np(w[rows], s[rows], b[rows])).astype(np.float64)
    xf = synth.bf16_to_f32(x).astype(np.float64)
    ref = xf @ Wd.T
    got = y.float().cpu().numpy()[:, rows].astype(np.float64)
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -16 * (np.abs(xf) @ np.abs(Wd).T)
    err = np.abs(got - ref)
    print(f"M={M} N={N} K={K}: max err / bound {float((err / bound).max()):.3f}")
    assert (err <= bound).all()


@pytest.mark.gpu
@pytest.mark.parametrize("M,I", [(16, 1024), (77, 12288), (512, 512)])
def test_packed_gemm_swiglu_equals_gemm_then_swiglu(M, I):
    K = 4096
    w, s, b = synth.qmv_weights(2 * I, K, seed=12, tag=M)
    x = to_dev(synth.qmv_x(M, K, seed=12, tag=M), torch.bfloat16)
    wt, st, bt = to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16)
    fused = kernels.packed_gemm(x, kernels.pack_w4(wt, st, bt, swiglu=True), 2 * I, swiglu=True)
    gu = kernels.packed_gemm(x, kernels.pack_w4(wt, st, bt), 2 * I)
    h = torch.empty((M, I), dtype=torch.bfloat16, device=DEV)
    _C.call("qvex_swiglu", _ptr(gu), _ptr(h), M, I, _stream())
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), h.view(torch.int16))


@pytest.mark.gpu
def test_packed_gemm_rows_do_not_depend_on_m():
    """A row's output is the same whatever the other rows of the call (the
    products of a 64-row block do not mix rows)."""
    N, K = 2048, 4096
    w, s, b = synth.qmv_weights(N, K, seed=13)
    packed = kernels.pack_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    x = to_dev(synth.qmv_x(200, K, seed=13), torch.bfloat16)
    full = kernels.packed_gemm(x, packed, N)
    part = kernels.packed_gemm(x[130:150].contiguous(), packed, N)
    torch.cuda.synchronize()
    assert torch.equal(full[130:150].view(torch.int16), part.view(torch.int16))
