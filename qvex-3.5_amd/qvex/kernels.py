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
    """y = x @ dequant(w)^T for MLX affine weights
    (mx.quantized_matmul(transpose=True), engine/model.py:87-91).

    x: bf16 [..., K] with at most 8 rows in total; w: uint32 viewed as int32
    [N, K*bits/32]; scales, biases: bf16 [N, K/group_size]. Returns bf16 [..., N].
    4-bit group-64 runs qvex_qmv_w4g64 (tile optional); the other widths
    (bits 2, 3, 5, 6, 8, groups 32 / 128) run qvex_qmv_affine."""
    if (group_size, bits) != (GROUP, BITS):
        if tile is not None:
            raise _C.QvexError("explicit tiles exist for 4-bit group-64 weights only")
        return quantized_matmul_affine(x, w, scales, biases, group_size, bits, out)
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
    if tile is not None and tile[0] == "mfma":
        _C.call("qvex_qmv_w4g64_mfma", _ptr(x2), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                M, N, K, int(tile[1]), int(tile[2]), _stream())
    elif tile is None:
        _C.call("qvex_qmv_w4g64", _ptr(x2), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                M, N, K, _stream())
    else:
        _C.call("qvex_qmv_w4g64_tiled", _ptr(x2), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                M, N, K, int(tile[0]), int(tile[1]), _stream())
    return out


def _check_affine(w, scales, biases, K: int, group_size: int, bits: int):
    _check(w, "w", torch.int32, 2)
    _check(scales, "scales", torch.bfloat16, 2)
    _check(biases, "biases", torch.bfloat16, 2)
    if group_size not in (32, 64, 128) or bits not in (2, 3, 4, 5, 6, 8):
        raise _C.QvexError(f"unsupported quantization bits={bits} group_size={group_size} "
                           "(bits 2, 3, 4, 5, 6, 8; groups 32, 64, 128)")
    N = w.shape[0]
    if K % group_size or w.shape[1] * 32 != K * bits or scales.shape != (N, K // group_size) \
            or biases.shape != (N, K // group_size):
        raise _C.QvexError(f"shape mismatch for {bits}-bit group-{group_size} weights of K={K}: "
                           f"w {tuple(w.shape)} scales {tuple(scales.shape)} biases {tuple(biases.shape)}")


def quantized_matmul_affine(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                            group_size: int, bits: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ dequant(w)^T for any supported width (qvex_qmv_affine); x at most
    8 rows, w int32 [N, K*bits/32], scales/biases bf16 [N, K/group_size]."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    _check(x2, "x", torch.bfloat16, 2)
    _check_affine(w, scales, biases, K, group_size, bits)
    N = w.shape[0]
    if out is None:
        out = torch.empty((*x.shape[:-1], N), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != M * N:
        raise _C.QvexError("out has the wrong size")
    _C.call("qvex_qmv_affine", _ptr(x2), _ptr(w), _ptr(scales), _ptr(biases), _ptr(out), M, N, K, bits,
            group_size, _stream())
    return out


def embed_affine(ids: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, H: int,
                 group_size: int, bits: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(s * q + b) of the rows ids (clamped to [0, V)) of an affine-quantized
    table of any supported width (qvex_embed_affine)."""
    ids1 = ids.reshape(-1).to(torch.int32).contiguous()
    _check(ids1, "ids", torch.int32, 1)
    _check_affine(w, scales, biases, H, group_size, bits)
    L = ids1.numel()
    if out is None:
        out = torch.empty((L, H), dtype=torch.bfloat16, device=ids1.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != L * H:
        raise _C.QvexError("out has the wrong size")
    _C.call("qvex_embed_affine", _ptr(ids1), L, _ptr(w), _ptr(scales), _ptr(biases), w.shape[0], H, bits,
            group_size, _ptr(out), _stream())
    return out


def widen_w4g64(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, K: int, group_size: int,
                bits: int):
    """The same weight in the 4-bit group-64 layout (qvex_affine_widen_w4g64):
    bits <= 4 and group 64 or 128 re-encode losslessly. Returns (w4 int32
    [N, K/8], scales4, biases4 bf16 [N, K/64])."""
    _check_affine(w, scales, biases, K, group_size, bits)
    if bits > 4 or group_size % 64:
        raise _C.QvexError(f"{bits}-bit group-{group_size} weights do not fit the 4-bit group-64 layout")
    N = w.shape[0]
    w4 = torch.empty((N, K // 8), dtype=torch.int32, device=w.device)
    s4 = torch.empty((N, K // 64), dtype=torch.bfloat16, device=w.device)
    b4 = torch.empty_like(s4)
    _C.call("qvex_affine_widen_w4g64", _ptr(w), _ptr(scales), _ptr(biases), N, K, bits, group_size, _ptr(w4),
            _ptr(s4), _ptr(b4), _stream())
    return w4, s4, b4


def qmv_multi(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor) -> torch.Tensor:
    """x [M, K] (M small), w [N, K/8] 4-bit/group-64 -> y [M, N]
    (engine/kernels.py:197-211; the K % 512 restriction of the Metal kernel does
    not apply here: K % 64 == 0 suffices)."""
    return quantized_matmul(x, w, scales, biases)


def pack_w4(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, swiglu: bool = False) -> torch.Tensor:
    """Tile-packed copy of a QLinear triplet (engine/model.py:83-85) for
    quantized_matmul_packed: uint8 [ceil(N/16) * K/256 * 2304]. K % 256 == 0.
    swiglu=True packs a fused gate/up weight (gate rows first) with the gate/up
    interleave that quantized_matmul_packed(..., swiglu=True) expects."""
    _check(w, "w", torch.int32, 2)
    _check(scales, "scales", torch.bfloat16, 2)
    _check(biases, "biases", torch.bfloat16, 2)
    N, K = w.shape[0], w.shape[1] * 8
    if scales.shape != (N, K // GROUP) or biases.shape != (N, K // GROUP):
        raise _C.QvexError("pack_w4: scales/biases shape mismatch")
    nbytes = int(_C.lib().qvex_w4g64_packed_bytes(N, K))
    if nbytes == 0:
        raise _C.QvexError(f"pack_w4: K={K} is not a positive multiple of 256")
    packed = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _C.call("qvex_w4g64_pack_swiglu" if swiglu else "qvex_w4g64_pack", _ptr(w), _ptr(scales), _ptr(biases),
            N, K, _ptr(packed), nbytes, _stream())
    return packed


def dequant_w4(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, out: torch.Tensor | None = None):
    """bf16 [N, K] copy of an MLX 4-bit group-64 weight, bf16(s * q + b) computed
    in fp32: the operand of the dense GEMM that long (prefill) calls use."""
    _check(w, "w", torch.int32, 2)
    _check(scales, "scales", torch.bfloat16, 2)
    _check(biases, "biases", torch.bfloat16, 2)
    N, K = w.shape[0], w.shape[1] * 8
    if scales.shape != (N, K // 64) or biases.shape != (N, K // 64):
        raise _C.QvexError(f"scales/biases must be [N, K/64] = ({N}, {K // 64})")
    if out is None:
        out = torch.empty((N, K), dtype=torch.bfloat16, device=w.device)
    _check(out, "out", torch.bfloat16, 2)
    if out.shape != (N, K):
        raise _C.QvexError(f"out must be [N, K] = ({N}, {K})")
    _C.call("qvex_w4g64_dequant", _ptr(w), _ptr(scales), _ptr(biases), N, K, _ptr(out), _stream())
    return out


def packed_gemm(x: torch.Tensor, packed: torch.Tensor, N: int, out: torch.Tensor | None = None,
                swiglu: bool = False) -> torch.Tensor:
    """Prefill product y = x @ dequant(W)^T of any number of rows from pack_w4's
    copy (qvex_w4g64_packed_gemm): weights dequantized in registers to bf16,
    fp32 accumulation on MFMA. swiglu=True (a swiglu-packed [gate; up] weight):
    y [M, N/2] = silu(gate) * up."""
    _check(x, "x", torch.bfloat16)
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    if packed.dtype != torch.uint8 or not packed.is_contiguous() or packed.device != x.device:
        raise _C.QvexError("packed must be a contiguous uint8 tensor on the device of x")
    if packed.numel() != int(_C.lib().qvex_w4g64_packed_bytes(N, K)):
        raise _C.QvexError(f"packed has {packed.numel()} bytes, not the size of an N={N} K={K} pack")
    No = N // 2 if swiglu else N
    if out is None:
        out = torch.empty((M, No), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != M * No:
        raise _C.QvexError(f"out must hold M x {No} = {M * No} values")
    _C.call("qvex_w4g64_packed_gemm_swiglu" if swiglu else "qvex_w4g64_packed_gemm", _ptr(x2), _ptr(packed),
            _ptr(out), M, N, K, _stream())
    return out


def quantized_matmul_packed(x: torch.Tensor, packed: torch.Tensor, N: int, out: torch.Tensor | None = None,
                            tile: tuple[int, ...] | None = None, swiglu: bool = False) -> torch.Tensor:
    """y = x @ dequant(W)^T from pack_w4's copy, x bf16 [..., K] with 1..8 rows
    (the product of mx.quantized_matmul in QLinear.__call__, engine/model.py:87-91).
    tile = (tiles_per_wave, wave_ksplit[, prefetch_sets]) forces a tile and load
    pipeline (prefetch_sets 0 = two-deep, default -1 = automatic).
    swiglu=True (weight packed with swiglu=True): y [..., N/2] = silu(gate) * up
    (_swiglu, engine/model.py:134-135)."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    _check(x2, "x", torch.bfloat16, 2)
    if packed.dtype != torch.uint8 or not packed.is_contiguous() or packed.device != x.device:
        raise _C.QvexError("packed must be a contiguous uint8 tensor on the device of x")
    if packed.numel() != int(_C.lib().qvex_w4g64_packed_bytes(N, K)):
        raise _C.QvexError(f"packed has {packed.numel()} bytes, not the size of an N={N} K={K} pack")
    NO = N // 2 if swiglu else N
    if out is None:
        out = torch.empty((*x.shape[:-1], NO), dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != M * NO:
        raise _C.QvexError("out has the wrong size")
    if swiglu:
        if tile is not None:
            raise _C.QvexError("the SwiGLU form picks its own tile")
        _C.call("qvex_qmv_w4g64_packed_swiglu", _ptr(x2), _ptr(packed), _ptr(out), M, N, K, _stream())
    elif tile is None:
        _C.call("qvex_qmv_w4g64_packed", _ptr(x2), _ptr(packed), _ptr(out), M, N, K, _stream())
    else:
        _C.call("qvex_qmv_w4g64_packed_tiled", _ptr(x2), _ptr(packed), _ptr(out), M, N, K,
                int(tile[0]), int(tile[1]), int(tile[2]) if len(tile) > 2 else -1, _stream())
    return out


def qmv_packed_resid(x: torch.Tensor, packed: torch.Tensor, N: int, resid: torch.Tensor, norm_w: torch.Tensor,
                     h_out: torch.Tensor | None = None, u_out: torch.Tensor | None = None,
                     parts: torch.Tensor | None = None):
    """Product that ends a sub-block, with the residual add and the next norm's
    inputs in its epilogue: h = bf16(resid + bf16(x W^T)), u = bf16(h * norm_w),
    parts [M, ceil(N/16)] fp32 sums of h^2 per 16 columns. Returns (h, u, parts)."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    _check(x2, "x", torch.bfloat16, 2)
    _check(resid, "resid", torch.bfloat16)
    _check(norm_w, "norm_w", torch.bfloat16)
    if resid.numel() != M * N or norm_w.numel() != N:
        raise _C.QvexError(f"resid must hold M*N = {M * N} and norm_w N = {N} values")
    if packed.numel() != int(_C.lib().qvex_w4g64_packed_bytes(N, K)):
        raise _C.QvexError(f"packed has {packed.numel()} bytes, not the size of an N={N} K={K} pack")
    tiles = (N + 15) // 16
    h_out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if h_out is None else h_out
    u_out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if u_out is None else u_out
    parts = torch.empty((M, tiles), dtype=torch.float32, device=x.device) if parts is None else parts
    if h_out.numel() != M * N or u_out.numel() != M * N or parts.numel() != M * tiles:
        raise _C.QvexError("h_out/u_out/parts have the wrong size")
    _C.call("qvex_qmv_w4g64_packed_resid", _ptr(x2), _ptr(packed), M, N, K, _ptr(resid), _ptr(norm_w),
            _ptr(h_out), _ptr(u_out), _ptr(parts), _stream())
    return h_out, u_out, parts


def qmv_packed_gnorm_resid(u: torch.Tensor, ss_parts: torch.Tensor, packed: torch.Tensor, N: int, eps: float,
                           resid: torch.Tensor, norm_w: torch.Tensor, h_out: torch.Tensor | None = None):
    """out_proj over the gated norm's unscaled input u = bf16(silu(z) * w * y)
    [M, K] (heads of 128 columns), each head's share of the product scaled by
    rsqrt(sum(ss_parts[r, head, :]) / 128 + eps) (ss_parts [M, K/128, nb] fp32,
    nb in 1, 2, 4, 8), then the residual epilogue of qmv_packed_resid.
    Returns (h, u_next, parts)."""
    K = u.shape[-1]
    u2 = u.reshape(-1, K)
    M = u2.shape[0]
    _check(u2, "u", torch.bfloat16, 2)
    _check(ss_parts, "ss_parts", torch.float32)
    _check(resid, "resid", torch.bfloat16)
    _check(norm_w, "norm_w", torch.bfloat16)
    nb = ss_parts.shape[-1]
    if ss_parts.numel() != M * (K // 128) * nb or K % 128:
        raise _C.QvexError(f"ss_parts must hold M * K/128 * nb = {M * (K // 128) * nb} values")
    if resid.numel() != M * N or norm_w.numel() != N:
        raise _C.QvexError(f"resid must hold M*N = {M * N} and norm_w N = {N} values")
    if packed.numel() != int(_C.lib().qvex_w4g64_packed_bytes(N, K)):
        raise _C.QvexError(f"packed has {packed.numel()} bytes, not the size of an N={N} K={K} pack")
    tiles = (N + 15) // 16
    h_out = torch.empty((M, N), dtype=torch.bfloat16, device=u.device) if h_out is None else h_out
    u_out = torch.empty((M, N), dtype=torch.bfloat16, device=u.device)
    parts = torch.empty((M, tiles), dtype=torch.float32, device=u.device)
    if h_out.numel() != M * N:
        raise _C.QvexError("h_out has the wrong size")
    _C.call("qvex_qmv_w4g64_packed_gnorm_resid", _ptr(u2), _ptr(packed), M, N, K, _ptr(ss_parts), nb, float(eps),
            _ptr(resid), _ptr(norm_w), _ptr(h_out), _ptr(u_out), _ptr(parts), _stream())
    return h_out, u_out, parts


def qmv_packed_rstd(u: torch.Tensor, packed: torch.Tensor, N: int, parts: torch.Tensor, eps: float,
                    out: torch.Tensor | None = None, swiglu: bool = False,
                    tile_max: torch.Tensor | None = None) -> torch.Tensor:
    """quantized_matmul_packed of rms_norm(h) given as u = bf16(h * w) and the
    per-16-column sums of h^2 (qmv_packed_resid / rms_parts); swiglu as there.
    tile_max (bf16 [M, ceil(N/16)], not with swiglu): also each 16-column tile's
    largest output, for spec_accept's one-kernel list form."""
    K = u.shape[-1]
    u2 = u.reshape(-1, K)
    M = u2.shape[0]
    _check(u2, "u", torch.bfloat16, 2)
    _check(parts, "parts", torch.float32)
    nparts = (K + 15) // 16
    if parts.numel() != M * nparts:
        raise _C.QvexError(f"parts must hold M * ceil(K/16) = {M * nparts} values")
    if packed.numel() != int(_C.lib().qvex_w4g64_packed_bytes(N, K)):
        raise _C.QvexError(f"packed has {packed.numel()} bytes, not the size of an N={N} K={K} pack")
    NO = N // 2 if swiglu else N
    out = torch.empty((M, NO), dtype=torch.bfloat16, device=u.device) if out is None else out
    _check(out, "out", torch.bfloat16)
    if tile_max is not None:
        if swiglu:
            raise _C.QvexError("tile maxima are written by the plain product only")
        _check(tile_max, "tile_max", torch.bfloat16)
        if tile_max.numel() != M * ((N + 15) // 16):
            raise _C.QvexError(f"tile_max must hold M * ceil(N/16) = {M * ((N + 15) // 16)} values")
        _C.call("qvex_qmv_w4g64_packed_rstd_tilemax", _ptr(u2), _ptr(packed), _ptr(out), M, N, K, _ptr(parts),
                nparts, K, float(eps), _ptr(tile_max), _stream())
        return out
    _C.call("qvex_qmv_w4g64_packed_rstd", _ptr(u2), _ptr(packed), _ptr(out), M, N, K, _ptr(parts), nparts, K,
            float(eps), int(bool(swiglu)), _stream())
    return out


def qmv_packed_argmax(x: torch.Tensor, packed: torch.Tensor, N: int, out: torch.Tensor | None,
                      parts: torch.Tensor | None = None, eps: float = 0.0,
                      workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy token of each row of x W^T (first index of the largest bf16-rounded
    output, as an argmax over the product's bf16 result) without writing the
    product: out int32 [M]. With parts, x is NormedRows' u (the rows are scaled
    by rsqrt(mean(h^2) + eps) as qmv_packed_rstd does). out=None defers the
    reduction: returns the per-tile (max, first index) pairs [M, ceil(N/16), 2]
    (a view of the workspace) for mtp_input / embed_rms_parts to reduce."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    _check(x2, "x", torch.bfloat16, 2)
    if out is not None:
        _check(out, "out", torch.int32)
        if out.numel() != M:
            raise _C.QvexError(f"out must hold M = {M} values")
    if packed.numel() != int(_C.lib().qvex_w4g64_packed_bytes(N, K)):
        raise _C.QvexError(f"packed has {packed.numel()} bytes, not the size of an N={N} K={K} pack")
    need = int(_C.lib().qvex_qmv_w4g64_argmax_workspace_bytes(M, N))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty((need + 3) // 4, dtype=torch.float32, device=x.device)
    nparts = (K + 15) // 16
    if parts is not None:
        _check(parts, "parts", torch.float32)
        if parts.numel() != M * nparts:
            raise _C.QvexError(f"parts must hold M * ceil(K/16) = {M * nparts} values")
    _C.call("qvex_qmv_w4g64_packed_argmax", _ptr(x2), _ptr(packed), M, N, K,
            _ptr(parts) if parts is not None else None, nparts, K, float(eps),
            _ptr(out) if out is not None else None, _ptr(workspace),
            workspace.numel() * workspace.element_size(), _stream())
    if out is None:
        tiles = (N + 15) // 16
        return workspace.view(-1)[:M * tiles * 2].view(M, tiles, 2)
    return out


def _argmax_src(am, am_row):
    """(pointer, tiles, row pointer) of a deferred argmax input (qmv_packed_argmax with out=None)."""
    if am is None:
        return None, 0, None
    _check(am, "am", torch.float32)
    if am.dim() != 3 or am.shape[2] != 2 or not am.is_contiguous():
        raise _C.QvexError("am must be the [M, tiles, 2] pairs of qmv_packed_argmax(out=None)")
    if am_row is not None:
        _check(am_row, "am_row", torch.int32)
    return _ptr(am), am.shape[1], _ptr(am_row) if am_row is not None else None


def mtp_input(emb, ids, T: int, w_emb, hid, w_hid, eps: float, x_in: torch.Tensor, hid_sel=None, am=None,
              am_row=None, ids_out=None, counters=None, n_accept=None, extra: int = 0) -> torch.Tensor:
    """x_in [T, 2H] = [rms_norm(embed(ids)) * w_emb | rms_norm(hid[sel]) * w_hid] in one
    launch (engine/mtp.py:61-63); emb is a QEmbedding with a 4-bit group-64 copy. With am
    (T = 1) the token is the argmax of row am_row (device int32, None: 0) of the
    deferred pairs, also stored to ids_out; hid_sel: device row index of hid; with
    counters, *n_accept + extra is added to every counter in the same launch."""
    H = emb.H
    e4 = emb.w4g64()
    if e4 is None:
        raise _C.QvexError("mtp_input needs an embedding in (or widened to) the 4-bit group-64 layout")
    hid2 = hid.reshape(-1, hid.shape[-1])
    _check(hid2, "hid", torch.bfloat16, 2)
    _check(x_in, "x_in", torch.bfloat16, 2)
    if x_in.shape[0] < T or x_in.shape[1] < 2 * H:
        raise _C.QvexError(f"x_in must hold [{T}, {2 * H}]")
    amp, tiles, rowp = _argmax_src(am, am_row)
    if am is None:
        _check(ids, "ids", torch.int32)
        if not ids.is_contiguous() or ids.numel() != T:
            raise _C.QvexError("ids must be a contiguous int32 tensor of T values")
    elif ids_out is None:
        raise _C.QvexError("ids_out is needed with am")
    if hid_sel is not None:
        _check(hid_sel, "hid_sel", torch.int32)
    if n_accept is not None:
        _check(n_accept, "n_accept", torch.int32)
    if counters is not None:
        _check(counters, "counters", torch.int32)
    _C.call("qvex_mtp_input", _ptr(ids) if am is None else None, T, amp, tiles, rowp,
            _ptr(ids_out) if ids_out is not None else None, _ptr(e4[0]), _ptr(e4[1]), _ptr(e4[2]),
            emb.V, H, _ptr(w_emb), _ptr(hid2), hid2.stride(0), _ptr(hid_sel) if hid_sel is not None else None,
            _ptr(w_hid), _ptr(x_in), x_in.stride(0), float(eps),
            _ptr(counters) if counters is not None else None, counters.numel() if counters is not None else 0,
            _ptr(n_accept) if n_accept is not None else None, int(extra), _stream())
    return x_in


def embed_rms_parts(emb, ids: torch.Tensor, norm_w: torch.Tensor, am=None, am_row=None, am_slot: int = -1,
                    h_out=None, u_out=None, parts=None):
    """h = embed(ids) [L, H] and the first norm's folded inputs (u, parts as
    rms_parts(h, norm_w)) in one launch; with am, ids[am_slot] is first set to the
    argmax of row am_row of the deferred pairs (the last draft). Returns (h, u, parts)."""
    H = emb.H
    e4 = emb.w4g64()
    if e4 is None:
        raise _C.QvexError("embed_rms_parts needs an embedding in (or widened to) the 4-bit group-64 layout")
    _check(ids, "ids", torch.int32)
    if not ids.is_contiguous():
        raise _C.QvexError("ids must be contiguous")
    L = ids.numel()
    dev = ids.device
    h_out = torch.empty((L, H), dtype=torch.bfloat16, device=dev) if h_out is None else h_out
    u_out = torch.empty((L, H), dtype=torch.bfloat16, device=dev) if u_out is None else u_out
    parts = torch.empty((L, (H + 15) // 16), dtype=torch.float32, device=dev) if parts is None else parts
    amp, tiles, rowp = _argmax_src(am, am_row)
    _C.call("qvex_embed_rms_parts", _ptr(ids), L, amp, tiles, rowp, int(am_slot), _ptr(e4[0]), _ptr(e4[1]),
            _ptr(e4[2]), emb.V, H, _ptr(norm_w), _ptr(h_out), _ptr(u_out), _ptr(parts), _stream())
    return h_out, u_out, parts


def rms_parts(x: torch.Tensor, w: torch.Tensor, u_out: torch.Tensor | None = None,
              parts: torch.Tensor | None = None):
    """u = bf16(x * w) and the per-16-column sums of x^2 of rows x [M, D]."""
    D = x.shape[-1]
    x2 = x.reshape(-1, D)
    M = x2.shape[0]
    _check(x2, "x", torch.bfloat16, 2)
    u_out = torch.empty((M, D), dtype=torch.bfloat16, device=x.device) if u_out is None else u_out
    parts = torch.empty((M, (D + 15) // 16), dtype=torch.float32, device=x.device) if parts is None else parts
    _C.call("qvex_rms_parts", _ptr(x2), _ptr(w), _ptr(u_out), _ptr(parts), M, D, _stream())
    return u_out, parts


def read_roof(buf: torch.Tensor, sink: torch.Tensor, blocks: int = 4096) -> None:
    """Stream-read every byte of buf (HBM roof probe, experiments/native/qmv_spike.mm:21-32)."""
    nbytes = buf.numel() * buf.element_size()
    _C.call("qvex_read_roof", _ptr(buf), nbytes, _ptr(sink), int(blocks), _stream())


def read_probe(buf: torch.Tensor, sink: torch.Tensor, iters: int, lds: bool, waves_per_block: int = 4) -> None:
    """Read every byte of buf with qvex_read_probe (VGPR or direct-to-LDS loads)."""
    nbytes = buf.numel() * buf.element_size()
    _C.call("qvex_read_probe", _ptr(buf), nbytes, _ptr(sink), int(iters), int(bool(lds)), int(waves_per_block),
            _stream())


# ---------------------------------------------------------------- Gated DeltaNet

def _gdn_check(q, k, v, a, b, A_log, dt_bias):
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (a, "a"), (b, "b"), (dt_bias, "dt_bias")):
        _check(t, n, torch.bfloat16)
    _check(A_log, "A_log", torch.float32, 1)
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2:]
    if q.shape != k.shape or v.shape[:2] != (B, T) or a.shape != (B, T, Hv) or b.shape != (B, T, Hv):
        raise _C.QvexError(f"gated_delta shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} "
                           f"v {tuple(v.shape)} a {tuple(a.shape)} b {tuple(b.shape)}")
    if A_log.shape != (Hv,) or dt_bias.shape != (Hv,):
        raise _C.QvexError("A_log and dt_bias must have shape [Hv]")
    return B, T, Hk, Hv, Dk, Dv


def gated_delta_snapshots(q, k, v, a, b, A_log, dt_bias, state, snapshots=None, y=None):
    """Recurrent Gated DeltaNet over T tokens, keeping the state after every token.

    q, k [B,T,Hk,Dk], v [B,T,Hv,Dv], a, b [B,T,Hv] bf16; A_log fp32 [Hv];
    dt_bias bf16 [Hv]; state fp32 [B,Hv,Dv,Dk] (may be a slot of `snapshots`).
    Returns (y [B,T,Hv,Dv] bf16, snapshots fp32 [T,B,Hv,Dv,Dk]); snapshots[t] is
    the state after token t, so rolling back to L kept tokens is snapshots[L-1]."""
    B, T, Hk, Hv, Dk, Dv = _gdn_check(q, k, v, a, b, A_log, dt_bias)
    _check(state, "state", torch.float32)
    if state.shape != (B, Hv, Dv, Dk):
        raise _C.QvexError(f"state must be [B,Hv,Dv,Dk]=({B},{Hv},{Dv},{Dk})")
    if snapshots is None:
        snapshots = torch.empty((T, B, Hv, Dv, Dk), dtype=torch.float32, device=q.device)
    if y is None:
        y = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=q.device)
    _C.call("qvex_gdn_recurrent", _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(A_log),
            _ptr(dt_bias), _ptr(state), _ptr(snapshots), 1, _ptr(y), B, T, Hk, Hv, Dk, Dv, _stream())
    return y, snapshots


def gated_delta(q, k, v, a, b, A_log, dt_bias, state, keep_mid=False):
    """Mirror of engine/kernels.py:92-116: returns y, the new state and, with
    keep_mid, the state before the last token."""
    B, T, Hk, Hv, Dk, Dv = _gdn_check(q, k, v, a, b, A_log, dt_bias)
    if keep_mid:
        y, snaps = gated_delta_snapshots(q, k, v, a, b, A_log, dt_bias, state)
        mid = snaps[T - 2] if T >= 2 else state.clone()
        return y, snaps[T - 1], mid
    _check(state, "state", torch.float32)
    out = torch.empty((1, B, Hv, Dv, Dk), dtype=torch.float32, device=q.device)
    y = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=q.device)
    _C.call("qvex_gdn_recurrent", _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(A_log),
            _ptr(dt_bias), _ptr(state), _ptr(out), 0, _ptr(y), B, T, Hk, Hv, Dk, Dv, _stream())
    return y, out[0]


def gated_delta_ring(q, k, v, a, b, A_log, dt_bias, ring, cur_slot, y=None, snap_every=True):
    """Ring-buffer form: with c = cur_slot mod n_slots (cur_slot a device int32),
    the state is read from ring[c] and the state after token t is written to
    ring[(c + 1 + t) % n_slots] (only the last token's unless snap_every)."""
    B, T, Hk, Hv, Dk, Dv = _gdn_check(q, k, v, a, b, A_log, dt_bias)
    _check(ring, "ring", torch.float32)
    _check(cur_slot, "cur_slot", torch.int32)
    if y is None:
        y = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=q.device)
    _C.call("qvex_gdn_recurrent_ring", _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(A_log),
            _ptr(dt_bias), _ptr(ring), ring.shape[0], _ptr(cur_slot), int(bool(snap_every)), _ptr(y),
            B, T, Hk, Hv, Dk, Dv, _stream())
    return y


# ---------------------------------------------------------------- speculative acceptance

def gated_delta_chunked(q, k, v, a, b, A_log, dt_bias, state, state_out=None, y=None, workspace=None):
    """Chunked (64-token, MFMA) Gated DeltaNet over a long prefill: the same
    recurrence as gated_delta (engine/kernels.py:92-116) without per-token
    snapshots. Shapes as gated_delta_snapshots; returns (y, final state)."""
    B, T, Hk, Hv, Dk, Dv = _gdn_check(q, k, v, a, b, A_log, dt_bias)
    _check(state, "state", torch.float32)
    if state.shape != (B, Hv, Dv, Dk):
        raise _C.QvexError(f"state must be [B,Hv,Dv,Dk]=({B},{Hv},{Dv},{Dk})")
    if state_out is None:
        state_out = torch.empty_like(state)
    if y is None:
        y = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=q.device)
    need = int(_C.lib().qvex_gdn_chunked_workspace_bytes(B, T, Hv, Dk, Dv, 64))
    if need == 0:
        raise _C.QvexError(f"gated_delta_chunked: needs Dk = Dv = 128 (got {Dk}, {Dv})")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _C.call("qvex_gdn_chunked", _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(A_log), _ptr(dt_bias),
            _ptr(state), _ptr(state_out), _ptr(y), B, T, Hk, Hv, Dk, Dv, 64, _ptr(workspace),
            workspace.numel() * workspace.element_size(), _stream())
    return y, state_out


def spec_workspace(S: int, k: int, V: int, has_draft: bool, device, top_k: int = 0,
                   zeroed: bool = True) -> torch.Tensor:
    """Sampler workspace. zeroed: filled with zeros, as the one-kernel list form
    (spec_accept with tile maxima) needs it: it counts each step's finished rows
    there and relies on the count starting at zero (every call leaves it at
    zero); the other forms need no fill. A zero-filled workspace is refused
    while a graph is being captured on the current stream: the fill would only
    be recorded, so a graph captured later on the same workspace would start
    from whatever the memory held."""
    if zeroed and torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise _C.QvexError("spec_workspace: make the sampler workspace before the graph capture "
                           "(Sampler.prepare_accept), not inside it")
    n = int(_C.lib().qvex_spec_accept_filtered_workspace_bytes(S, k, V, int(has_draft), int(top_k)))
    return (torch.zeros if zeroed else torch.empty)((max(n, 4) + 3) // 4, dtype=torch.float32, device=device)


def tile_max(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Each 16-column tile's largest value of bf16 logits [..., V] -> bf16
    [rows, ceil(V/16)] (what the lm_head's tile-maxima epilogue writes)."""
    _check(logits, "logits", torch.bfloat16)
    V = logits.shape[-1]
    rows = logits.numel() // V
    tiles = (V + 15) // 16
    if out is None:
        out = torch.empty((rows, tiles), dtype=torch.bfloat16, device=logits.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != rows * tiles:
        raise _C.QvexError(f"out must hold rows * ceil(V/16) = {rows * tiles} values")
    _C.call("qvex_tile_max_bf16", _ptr(logits), rows, V, _ptr(out), _stream())
    return out


def spec_accept(target: torch.Tensor, draft: torch.Tensor | None, draft_ids: torch.Tensor,
                u_accept: torch.Tensor, u_sample: torch.Tensor, temperature: float,
                n_accept: torch.Tensor | None = None, out_token: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, seen: torch.Tensor | None = None,
                presence_penalty: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                tile_max: torch.Tensor | None = None):
    """Fused accept / residual-resample / bonus sampling for S verify steps.

    target fp32 or bf16 [S,k+1,V]; draft [S,k,V] of the same dtype or None (greedy
    one-hot drafts, the reference's rule, engine/speculative.py:79-80); bf16
    logits are read as they are (exact widening, same results as their fp32
    copies); draft_ids int32 [S,k];
    u_accept fp32 [S,k]; u_sample fp32 [S]; temperature <= 0 means greedy.
    The target rows are scored as Sampler.scores (engine/sampler.py:30-52):
    presence penalty over `seen` (fp32 [V], 0/1) plus the drafts before each row,
    then top-k (0..64, 0 = off) and top-p (needs top-k) when sampling.
    tile_max: bf16 [S*(k+1), ceil(V/16)], each target row's 16-column tile maxima
    (qmv_packed_rstd's epilogue or tile_max()); with bf16 logits, no draft
    logits and no presence penalty the list form (1 <= top_k <= 64) then runs as
    one kernel that reads only the tiles that can hold the top-k (the same
    results as without it).
    Returns (n_accept int32 [S], out_token int32 [S]) on the device."""
    bf = target.dtype == torch.bfloat16
    ldt = torch.bfloat16 if bf else torch.float32
    _check(target, "target", ldt, 3)
    S, k1, V = target.shape
    k = k1 - 1
    if draft is not None:
        _check(draft, "draft", ldt, 3)
        if draft.shape != (S, k, V):
            raise _C.QvexError(f"draft must be [S,k,V]=({S},{k},{V})")
    _check(draft_ids, "draft_ids", torch.int32)
    _check(u_accept, "u_accept", torch.float32)
    _check(u_sample, "u_sample", torch.float32)
    if draft_ids.numel() != S * k or u_accept.numel() != S * k or u_sample.numel() != S:
        raise _C.QvexError("draft_ids/u_accept must hold S*k values and u_sample S values")
    import numpy as np
    inv_temp = float(np.float32(1.0) / np.float32(temperature)) if temperature > 0 else 0.0
    dev = target.device
    if n_accept is None:
        n_accept = torch.empty(S, dtype=torch.int32, device=dev)
    if out_token is None:
        out_token = torch.empty(S, dtype=torch.int32, device=dev)
    if seen is not None:
        _check(seen, "seen", torch.float32)
        if seen.numel() != V:
            raise _C.QvexError(f"seen must hold V={V} values")
    if workspace is None:   # zero-filled only for the one-kernel form's step counters
        workspace = spec_workspace(S, k, V, draft is not None, dev, top_k, zeroed=tile_max is not None)
    if tile_max is not None:
        if not bf or draft is not None:
            raise _C.QvexError("tile maxima go with bf16 target logits and no draft logits")
        _check(tile_max, "tile_max", torch.bfloat16)
        if tile_max.numel() != S * k1 * ((V + 15) // 16):
            raise _C.QvexError(f"tile_max must hold S*(k+1)*ceil(V/16) = {S * k1 * ((V + 15) // 16)} values")
        _C.call("qvex_spec_accept_tiles_bf16", _ptr(target), _ptr(tile_max), _ptr(draft_ids), _ptr(u_accept),
                _ptr(u_sample), inv_temp, _ptr(seen) if seen is not None else None,
                float(np.float32(presence_penalty)), int(top_k), float(np.float32(top_p)), _ptr(n_accept),
                _ptr(out_token), S, k, V, _ptr(workspace), workspace.numel() * 4, _stream())
        return n_accept, out_token
    _C.call("qvex_spec_accept_filtered_bf16" if bf else "qvex_spec_accept_filtered", _ptr(target),
            _ptr(draft) if draft is not None else None,
            _ptr(draft_ids), _ptr(u_accept), _ptr(u_sample), inv_temp,
            _ptr(seen) if seen is not None else None, float(np.float32(presence_penalty)), int(top_k),
            float(np.float32(top_p)), _ptr(n_accept), _ptr(out_token), S, k, V, _ptr(workspace),
            workspace.numel() * 4, _stream())
    return n_accept, out_token


def _inv_temp(temperature: float) -> float:
    import numpy as np
    return float(np.float32(1.0) / np.float32(temperature)) if temperature > 0 else 0.0


def tiles_rows_apply(S: int, k: int, V: int, temperature: float, top_k: int, presence_penalty: float) -> bool:
    """Whether spec_accept_rows (the one-kernel form from tile maxima) serves a
    call with these arguments: bf16 logits, no draft logits, sampling with
    1 <= top_k <= 64, no presence penalty, V a multiple of 128 that fits."""
    import numpy as np
    return bool(_C.lib().qvex_spec_accept_tiles_applies(S, k, V, _inv_temp(temperature), int(top_k),
                                                        float(np.float32(presence_penalty))))


def spec_accept_rows(target: torch.Tensor, draft_ids: torch.Tensor, u_accept: torch.Tensor, u_sample: torch.Tensor,
                     temperature: float, tile_max: torch.Tensor, rows: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None, seen: torch.Tensor | None = None,
                     presence_penalty: float = 0.0, top_k: int = 0, top_p: float = 1.0) -> torch.Tensor:
    """spec_accept's one-kernel form without the step decision: each target row
    leaves (accept flag, draw) in rows int32 [S*(k+1), 2] (the flag of row k, the
    bonus row, is 0 and unused); a step's (n, token) is its first row with flag
    0 among rows 0..k-1 (else row k) and that row's draw, which the decode
    cycle's finishing kernel takes (cycle_finish_ex with rows). Only where
    tiles_rows_apply holds; bf16 target [S,k+1,V] with its tile maxima."""
    import numpy as np
    _check(target, "target", torch.bfloat16, 3)
    S, k1, V = target.shape
    k = k1 - 1
    _check(draft_ids, "draft_ids", torch.int32)
    _check(u_accept, "u_accept", torch.float32)
    _check(u_sample, "u_sample", torch.float32)
    if draft_ids.numel() != S * k or u_accept.numel() != S * k or u_sample.numel() != S:
        raise _C.QvexError("draft_ids/u_accept must hold S*k values and u_sample S values")
    _check(tile_max, "tile_max", torch.bfloat16)
    if tile_max.numel() != S * k1 * ((V + 15) // 16):
        raise _C.QvexError(f"tile_max must hold S*(k+1)*ceil(V/16) = {S * k1 * ((V + 15) // 16)} values")
    if not tiles_rows_apply(S, k, V, temperature, top_k, presence_penalty):
        raise _C.QvexError("spec_accept_rows: the one-kernel form does not apply to this call")
    if rows is None:
        rows = torch.empty((S * k1, 2), dtype=torch.int32, device=target.device)
    _check(rows, "rows", torch.int32)
    if rows.numel() != 2 * S * k1:
        raise _C.QvexError(f"rows must hold 2*S*(k+1) = {2 * S * k1} values")
    if workspace is None:   # no counter in this form: no fill needed
        workspace = spec_workspace(S, k, V, False, target.device, top_k, zeroed=False)
    _C.call("qvex_spec_accept_tiles_rows_bf16", _ptr(target), _ptr(tile_max), _ptr(draft_ids), _ptr(u_accept),
            _ptr(u_sample), _inv_temp(temperature), _ptr(seen) if seen is not None else None,
            float(np.float32(presence_penalty)), int(top_k), float(np.float32(top_p)), _ptr(rows), S, k, V,
            _ptr(workspace), workspace.numel() * 4, _stream())
    return rows


# ---------------------------------------------------------------- KV cache layouts

def kv_tile_k(k: torch.Tensor) -> torch.Tensor:
    """[Hkv, cap, D] keys -> the tiled K cache layout [Hkv, cap/16, D/32, 64, 8]
    (key p, dim d at lane 16 ((d % 32) / 8) + p % 16 of block p / 16, step d / 32)."""
    h, cap, D = k.shape
    return k.reshape(h, cap // 16, 16, D // 32, 4, 8).permute(0, 1, 3, 4, 2, 5).contiguous()


def kv_tile_v(v: torch.Tensor) -> torch.Tensor:
    """[Hkv, cap, D] values -> the tiled V cache layout [Hkv, cap/32, D, 32]."""
    h, cap, D = v.shape
    return v.reshape(h, cap // 32, 32, D).permute(0, 1, 3, 2).contiguous()


def kv_untile_k(kt: torch.Tensor) -> torch.Tensor:
    """The tiled K cache [Hkv, cap/16, D/32, 64, 8] as [Hkv, cap, D] (a copy)."""
    h, nb, ns = kt.shape[:3]
    return kt.reshape(h, nb, ns, 4, 16, 8).permute(0, 1, 4, 2, 3, 5).reshape(h, nb * 16, ns * 32)


def kv_untile_v(vt: torch.Tensor) -> torch.Tensor:
    """The tiled V cache [Hkv, cap/32, D, 32] as [Hkv, cap, D] (a copy)."""
    h, nb, d = vt.shape[:3]
    return vt.permute(0, 1, 3, 2).reshape(h, nb * 32, d)
