"""Torch-tensor front end of the HIP kernels (mirror of engine/kernels.py).

Each function checks device, dtype, contiguity and shape on the host, then
enqueues the kernel on torch's current HIP stream through the C ABI. There is
no CPU or PyTorch fallback: a missing library or a non-GPU tensor raises.
"""

from __future__ import annotations

import torch

from . import _C

GROUP = 64
BITS = 4


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _check(t: torch.Tensor, name: str, dtype: torch.dtype, ndim: int | None = None):
    if not t.is_cuda:
        raise _C.QvexError(f"{name} must be a GPU tensor (got {t.device})")
    if t.dtype != dtype:
        raise _C.QvexError(f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise _C.QvexError(f"{name} must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise _C.QvexError(f"{name} must have {ndim} dims (got {tuple(t.shape)})")


# ---------------------------------------------------------------- quantized matmul

def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     out: torch.Tensor | None = None, group_size: int = GROUP, bits: int = BITS,
                     tile: tuple[int, int] | None = None) -> torch.Tensor:
    """y = x @ dequant(w)^T for MLX 4-bit group-64 weights
    (mx.quantized_matmul(transpose=True), engine/model.py:87-91).

    x: bf16 [..., K] with at most 8 rows in total; w: uint32 viewed as int32
    [N, K/8]; scales, biases: bf16 [N, K/64]. Returns bf16 [..., N]."""
    if group_size != GROUP or bits != BITS:
        raise _C.QvexError(f"only group_size={GROUP}, bits={BITS} is implemented")
    K = x.shape[-1]
    N = w.shape[0]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    _check(x2, "x", torch.bfloat16, 2)
    _check(w, "w", torch.int32, 2)
    _check(scales, "scales", torch.bfloat16, 2)
    _check(biases, "biases", torch.bfloat16, 2)
    if w.shape[1] * 8 != K or scales.shape != (N, K // GROUP) or biases.shape != (N, K // GROUP):
        raise _C.QvexError(f"shape mismatch: x {tuple(x.shape)} w {tuple(w.shape)} "
                           f"scales {tuple(scales.shape)} biases {tuple(biases.shape)}")
    if out is None:
        out = torch.empty((*x.shape[:-1], N), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != M * N:
        raise _C.QvexError("out has the wrong size")
    if tile is None:
        _C.call("qvex_qmv_w4g64", _ptr(x2), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                M, N, K, _stream())
    else:
        _C.call("qvex_qmv_w4g64_tiled", _ptr(x2), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                M, N, K, int(tile[0]), int(tile[1]), _stream())
    return out


def qmv_multi(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> torch.Tensor:
    """x [M, K] (M small), w [N, K/8] 4-bit/group-64 -> y [M, N]
    (engine/kernels.py:197-211; the K % 512 restriction of the Metal kernel does
    not apply here: K % 64 == 0 suffices)."""
    return quantized_matmul(x, w, scales, biases)


def read_roof(buf: torch.Tensor, sink: torch.Tensor, blocks: int = 4096) -> None:
    """Stream-read every byte of buf (HBM roof probe, experiments/native/qmv_spike.mm:21-32)."""
    nbytes = buf.numel() * buf.element_size()
    _C.call("qvex_read_roof", _ptr(buf), nbytes, _ptr(sink), int(blocks), _stream())
