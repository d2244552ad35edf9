"""Qwen3.5 hybrid stack (dense, text-only) on the qvex HIP kernels.

Mirror of engine/model.py: Config, QLinear, QEmbedding, KVCache,
RecurrentCache, Attention, GatedDeltaNet, MLP, Layer, Qwen35 keep the
reference's names, call signatures and cache API (make_cache, rollback(n),
state(), offset). Every op runs in libqvex.so; torch only holds device memory.

MI355X-specific state layout (what makes rollback free):
  * every cache of a model shares one device int32 table ``CacheCounters``:
    entry i is layer i's token count, which all position-dependent kernels read
    on the device (RoPE position / KV append slot, conv-ring row, DeltaNet
    ring slot);
  * KVCache: bf16 [Hkv, cap, D] preallocated to the context capacity;
  * RecurrentCache: conv history ring [R, conv_dim] bf16 (R >= max verify
    width + K - 1) and a DeltaNet state ring [S, Hv, Dv, Dk] fp32 with a state
    snapshot per verify token;
  so rollback(n) is ``offset -= n`` for every cache kind, any n <= the last
  call's width (the reference allows n = 1 for recurrent caches only,
  engine/model.py:189-193).
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import _C, kernels
from .kernels import _ptr, _stream

QMV_MAX_ROWS = 8


# ---------------------------------------------------------------- config

@dataclass
class Config:
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    linear_num_key_heads: int
    linear_num_value_heads: int
    linear_key_head_dim: int
    linear_value_head_dim: int
    linear_conv_kernel_dim: int
    full_attention_interval: int
    rms_norm_eps: float
    vocab_size: int
    rope_theta: float
    rotary_dim: int
    group_size: int
    bits: int
    quant: dict = field(default_factory=dict)

    @classmethod
    def from_file(cls, path: Path) -> "Config":
        """Same parsing as engine/model.py:39-66 (text_config, rope_parameters,
        quantization overrides with the language_model. prefix stripped)."""
        raw = json.loads(Path(path).read_text())
        t = raw.get("text_config", raw)
        rope = t.get("rope_parameters") or {}
        q = raw.get("quantization") or raw.get("quantization_config") or {}
        head_dim = t.get("head_dim") or t["hidden_size"] // t["num_attention_heads"]
        return cls(
            hidden_size=t["hidden_size"], intermediate_size=t["intermediate_size"],
            num_hidden_layers=t["num_hidden_layers"], num_attention_heads=t["num_attention_heads"],
            num_key_value_heads=t["num_key_value_heads"], head_dim=head_dim,
            linear_num_key_heads=t["linear_num_key_heads"], linear_num_value_heads=t["linear_num_value_heads"],
            linear_key_head_dim=t["linear_key_head_dim"], linear_value_head_dim=t["linear_value_head_dim"],
            linear_conv_kernel_dim=t["linear_conv_kernel_dim"],
            full_attention_interval=t.get("full_attention_interval", 4),
            rms_norm_eps=t["rms_norm_eps"], vocab_size=t["vocab_size"],
            rope_theta=rope.get("rope_theta", t.get("rope_theta", 10_000_000)),
            rotary_dim=int(head_dim * rope.get("partial_rotary_factor", 0.25)),
            group_size=q.get("group_size", 64), bits=q.get("bits", 4),
            quant={k.removeprefix("language_model."): v for k, v in q.items() if isinstance(v, dict)},
        )

    @classmethod
    def qwen35_9b(cls) -> "Config":
        """Qwen3.5-9B text shape: 32 layers (every 4th full attention), hidden 4096,
        MLP 12288, vocab 248320, GDN 16 key / 32 value heads of 128, attention 16 q /
        4 kv heads of 256, conv kernel 4, partial rotary 64 of 256."""
        return cls(hidden_size=4096, intermediate_size=12288, num_hidden_layers=32,
                   num_attention_heads=16, num_key_value_heads=4, head_dim=256,
                   linear_num_key_heads=16, linear_num_value_heads=32, linear_key_head_dim=128,
                   linear_value_head_dim=128, linear_conv_kernel_dim=4, full_attention_interval=4,
                   rms_norm_eps=1e-6, vocab_size=248320, rope_theta=10_000_000.0, rotary_dim=64,
                   group_size=64, bits=4)

    @classmethod
    def tiny(cls, layers: int = 4, vocab: int = 4096) -> "Config":
        """Small shape with the same head geometry rules, for parity tests."""
        return cls(hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                   num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                   linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=128,
                   linear_value_head_dim=128, linear_conv_kernel_dim=4, full_attention_interval=4,
                   rms_norm_eps=1e-6, vocab_size=vocab, rope_theta=10_000_000.0, rotary_dim=32,
                   group_size=64, bits=4)

    def qparams(self, module: str) -> tuple[int, int]:
        o = self.quant.get(module, {})
        return o.get("group_size", self.group_size), o.get("bits", self.bits)

    def is_linear(self, i: int) -> bool:
        return (i + 1) % self.full_attention_interval != 0


# ---------------------------------------------------------------- building blocks

WIDTHS = (2, 3, 4, 5, 6, 8)      # bits of the MLX affine layouts the kernels read
GROUPS = (32, 64, 128)


def widens_to_w4g64(bits: int, group_size: int) -> bool:
    """A weight of this width re-encodes losslessly as 4-bit group-64 (codes
    fit a nibble; a 128-code group's scale and bias serve both 64-code halves)."""
    return bits <= 4 and group_size % 64 == 0


def _check_quant(what: str, bits: int, group_size: int):
    if bits not in WIDTHS or group_size not in GROUPS:
        raise _C.QvexError(f"{what}: {bits}-bit group-{group_size} quantization is not supported "
                           f"(bits {WIDTHS}, groups {GROUPS})")


class QLinear:
    """Affine-quantized linear layer, y = x @ dequant(W)^T (engine/model.py:80-104).

    w: int32 [N, K*bits/32] (uint32 words of each row's little-endian code
    stream), scales, biases: bf16 [N, K/group_size]; bits 2, 3, 4, 5, 6, 8 and
    groups 32, 64, 128 (Config.qparams overrides). A width that re-encodes
    losslessly as 4-bit group-64 (bits <= 4, group 64 or 128: every 3-bit layer
    of a mixed 4/3-bit model) is widened once, at construction, and then takes
    every path below exactly as a 4-bit layer does; the other widths run the
    any-width VALU product (qvex_qmv_affine) in chunks of 8 rows, without the
    fused epilogues. For the 4-bit group-64 layout: when K is
    a multiple of 256 the layer also keeps the tile-packed copy (pack_w4), built
    once here, and runs every call of 1..8 rows - decode, MTP drafts, verify of
    up to 7 drafts - through the MFMA kernel on it (5..8 rows as two halves over
    one read of the weights); the row bits of that kernel do not depend on the
    number of rows. Calls of 9..DENSE_MIN_ROWS-1 rows (short prefill tails) run
    it on chunks of 8 rows, so their rows have the same bits too; longer calls (prefill) run the packed
    MFMA GEMM (weights dequantized to bf16 in registers). Without a packed copy
    (K not a multiple of 256) the MLX-layout kernel takes chunks of 8 rows."""

    PACKED_MAX_ROWS = 8
    # calls of at least this many rows (prefill) run the packed GEMM; 0 disables it
    DENSE_MIN_ROWS = 16

    def __init__(self, w, scales, biases, group_size=64, bits=4, pack: bool = True, swiglu: bool = False):
        _check_quant("QLinear", bits, group_size)
        self.w, self.scales, self.biases = w, scales, biases
        self.group_size, self.bits = group_size, bits
        self.N = w.shape[0]
        self.K = w.shape[1] * 32 // bits
        if w.shape[1] * 32 != self.K * bits or self.K % group_size:
            raise _C.QvexError(f"QLinear: w {tuple(w.shape)} is not a {bits}-bit row of whole {group_size}-code groups")
        # swiglu: a fused [gate; up] weight whose packed copy carries the gate/up
        # interleave; its 1..8-row calls go through swiglu() (SwiGLU fused in)
        self.swiglu_packed = swiglu and self.N % 16 == 0
        self.packed = None
        if pack and self.K % 256 == 0 and widens_to_w4g64(bits, group_size):
            self.packed = kernels.pack_w4(*self._w4g64(w, scales, biases), swiglu=self.swiglu_packed)

    def _w4g64(self, w, s, b):
        """The triplet in the 4-bit group-64 layout (widened when stored narrower)."""
        if (self.bits, self.group_size) == (4, 64):
            return w, s, b
        return kernels.widen_w4g64(w, s, b, self.K, self.group_size, self.bits)

    def repack(self) -> None:
        """Rebuild the packed copy after the MLX-layout tensors were edited in place."""
        if self.packed is not None:
            w, s, b = self._mlx_on(self.packed.device)
            self.packed = kernels.pack_w4(*self._w4g64(w, s, b), swiglu=self.swiglu_packed)

    def offload_mlx(self) -> None:
        """Keep the MLX-layout triplet in host memory once the packed copy exists:
        every device path of a packed layer reads the packed copy, so the
        weight is resident on the GPU once (the host copy serves repack() and
        the plain product of a gate/up-interleaved weight)."""
        if self.packed is not None and self.w.is_cuda:
            self.w, self.scales, self.biases = self.w.cpu(), self.scales.cpu(), self.biases.cpu()

    def _mlx_on(self, device):
        """The MLX-layout triplet on `device` (a transient copy when offloaded)."""
        if self.w.device == torch.device(device):
            return self.w, self.scales, self.biases
        return self.w.to(device), self.scales.to(device), self.biases.to(device)

    def _takes_normed(self, x, M: int) -> bool:
        return self.packed is not None and M <= self.PACKED_MAX_ROWS and NormedRows.supported(self.K)

    def _packed_chunks(self, M: int) -> bool:
        """Rows for the packed kernel in chunks of PACKED_MAX_ROWS (below the dense GEMM)."""
        return self.packed is not None and M < max(self.DENSE_MIN_ROWS, self.PACKED_MAX_ROWS + 1)

    def swiglu(self, x) -> torch.Tensor:
        """silu(x W_gate^T) * (x W_up^T) for a fused [gate; up] layer
        (_swiglu over the split halves, engine/model.py:134-135, 302)."""
        if isinstance(x, NormedRows):
            M = x.u.reshape(-1, self.K).shape[0]
            if self.swiglu_packed and self._takes_normed(x, M):
                return kernels.qmv_packed_rstd(x.u, self.packed, self.N, x.parts, x.eps, swiglu=True)
            x = x.materialize()
        x2 = x.reshape(-1, self.K)
        M, I = x2.shape[0], self.N // 2
        if self.swiglu_packed and self.packed is not None and M <= self.PACKED_MAX_ROWS:
            return kernels.quantized_matmul_packed(x2, self.packed, self.N, swiglu=True)
        if self.swiglu_packed and self.packed is not None and self.DENSE_MIN_ROWS and M >= self.DENSE_MIN_ROWS:
            return kernels.packed_gemm(x2.contiguous(), self.packed, self.N, swiglu=True)
        if self.swiglu_packed and self._packed_chunks(M):
            h = torch.empty((M, I), dtype=torch.bfloat16, device=x.device)
            for m0 in range(0, M, self.PACKED_MAX_ROWS):
                m1 = min(M, m0 + self.PACKED_MAX_ROWS)
                kernels.quantized_matmul_packed(x2[m0:m1], self.packed, self.N, out=h[m0:m1], swiglu=True)
            return h
        gu = self(x2)
        h = torch.empty((M, I), dtype=torch.bfloat16, device=x.device)
        _C.call("qvex_swiglu", _ptr(gu), _ptr(h), M, I, _stream())
        return h

    def __call__(self, x, out: torch.Tensor | None = None) -> torch.Tensor:
        if isinstance(x, NormedRows):
            M = x.u.reshape(-1, self.K).shape[0]
            if not self.swiglu_packed and self._takes_normed(x, M):
                o = kernels.qmv_packed_rstd(x.u, self.packed, self.N, x.parts, x.eps,
                                            out=None if out is None else out.view(M, self.N))
                return o.view(*x.u.shape[:-1], self.N)
            x = x.materialize()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.K)
        M = x2.shape[0]
        if out is None:
            out = torch.empty((M, self.N), dtype=torch.bfloat16, device=x.device)
        o2 = out.view(M, self.N)
        if self.packed is not None and not self.swiglu_packed and M <= self.PACKED_MAX_ROWS:
            kernels.quantized_matmul_packed(x2, self.packed, self.N, out=o2)
            return out.view(*lead, self.N)
        if not self.swiglu_packed and self._packed_chunks(M):
            for m0 in range(0, M, self.PACKED_MAX_ROWS):
                m1 = min(M, m0 + self.PACKED_MAX_ROWS)
                kernels.quantized_matmul_packed(x2[m0:m1], self.packed, self.N, out=o2[m0:m1])
            return out.view(*lead, self.N)
        if self.packed is not None and not self.swiglu_packed and self.DENSE_MIN_ROWS and \
                M >= self.DENSE_MIN_ROWS:
            # long (prefill) call: the packed MFMA GEMM
            kernels.packed_gemm(x2.contiguous(), self.packed, self.N, out=o2)
            return out.view(*lead, self.N)
        w, sc, bi = self._mlx_on(x.device)
        for m0 in range(0, M, QMV_MAX_ROWS):
            m1 = min(M, m0 + QMV_MAX_ROWS)
            kernels.quantized_matmul(x2[m0:m1], w, sc, bi, out=o2[m0:m1], group_size=self.group_size,
                                     bits=self.bits)
        return out.view(*lead, self.N)

    def with_tile_max(self, x, tile_max: torch.Tensor) -> torch.Tensor:
        """self(x) that also writes each output row's 16-column tile maxima into
        tile_max (bf16 [M, ceil(N/16)]) for Sampler.accept_device: in the
        product's epilogue for NormedRows input on packed weights (1..8 rows),
        else by a pass over the result."""
        if isinstance(x, NormedRows):
            M = x.u.reshape(-1, self.K).shape[0]
            if not self.swiglu_packed and self._takes_normed(x, M):
                o = kernels.qmv_packed_rstd(x.u, self.packed, self.N, x.parts, x.eps, tile_max=tile_max)
                return o.view(*x.u.shape[:-1], self.N)
        y = self(x)
        kernels.tile_max(y.reshape(-1, self.N), out=tile_max)
        return y

    def argmax(self, x, out: torch.Tensor | None) -> torch.Tensor:
        """Greedy token per row of the product (first index of the largest bf16
        output) into out int32 [M]; x a tensor or NormedRows of 1..8 rows. out=None
        (NormedRows input, packed weights): the reduction is left to the next
        launch, which takes the returned per-tile pairs [M, ceil(N/16), 2]
        (kernels.mtp_input / embed_rms_parts); the buffer is reused by the next
        call with the same M."""
        if isinstance(x, NormedRows):
            M = x.u.reshape(-1, self.K).shape[0]
            if self._takes_normed(x, M) and not self.swiglu_packed:
                if not hasattr(self, "_am_ws"):
                    self._am_ws = {}
                ws = self._am_ws.get(M)
                if ws is None:
                    need = int(_C.lib().qvex_qmv_w4g64_argmax_workspace_bytes(M, self.N))
                    ws = self._am_ws[M] = torch.empty((need + 3) // 4, dtype=torch.float32, device=x.device)
                return kernels.qmv_packed_argmax(x.u, self.packed, self.N, out, x.parts, x.eps, workspace=ws)
        if out is None:
            raise _C.QvexError("a deferred argmax needs NormedRows input and a packed QLinear")
        from .speculative import _argmax
        logits = self(x).reshape(-1, self.N)
        for r in range(logits.shape[0]):
            _argmax(logits[r], out=out.reshape(-1)[r:r + 1])
        return out

    def residual(self, x: torch.Tensor, resid: torch.Tensor, norm_w: torch.Tensor, eps: float,
                 h_out: torch.Tensor | None = None):
        """h = resid + x W^T and the next norm of h: returns (h, NormedRows) with
        the add and the norm's inputs in the product's epilogue (1..8 rows), or
        (h, normalised tensor) through add_rms_norm otherwise. h_out: where h goes."""
        x2 = x.reshape(-1, self.K)
        M = x2.shape[0]
        ho = None if h_out is None else h_out.view(M, self.N)
        if (self.packed is not None and not self.swiglu_packed and M <= self.PACKED_MAX_ROWS
                and NormedRows.supported(self.N)):
            h, u, parts = kernels.qmv_packed_resid(x2, self.packed, self.N, resid.reshape(M, self.N), norm_w,
                                                   h_out=ho)
            return h, NormedRows(u, parts, eps)
        return add_rms_norm(resid.reshape(M, self.N), self(x2), norm_w, eps, h_out=ho)

    @staticmethod
    def fuse(layers: list["QLinear"], swiglu: bool = False) -> "QLinear":
        """Stack output rows of layers sharing the input (lossless, engine/model.py:93-104)."""
        l0 = layers[0]
        assert all((l.group_size, l.bits) == (l0.group_size, l0.bits) for l in layers), \
            "fused layers must share the quantization (bits, group size)"
        return QLinear(torch.cat([l.w for l in layers]), torch.cat([l.scales for l in layers]),
                       torch.cat([l.biases for l in layers]), l0.group_size, l0.bits, swiglu=swiglu)


class QEmbedding:
    """Quantized embedding rows, dequantized on gather (engine/model.py:121-130).

    Any width of QLinear's layouts. A table that widens losslessly to 4-bit
    group-64 (bits <= 4, group 64 or 128) keeps only the widened copy on the
    device (the stored triplet moves to host memory), so the fused decode-cycle
    inputs (qvex_mtp_input, qvex_embed_rms_parts) read it as they read a 4-bit
    table; the other widths gather with qvex_embed_affine."""

    def __init__(self, w, scales, biases, group_size=64, bits=4):
        _check_quant("QEmbedding", bits, group_size)
        self.w, self.scales, self.biases = w, scales, biases
        self.group_size, self.bits = group_size, bits
        self.V, self.H = w.shape[0], w.shape[1] * 32 // bits
        if w.shape[1] * 32 != self.H * bits or self.H % group_size:
            raise _C.QvexError(f"QEmbedding: w {tuple(w.shape)} is not a {bits}-bit row of whole "
                               f"{group_size}-code groups")
        self._w4 = None
        if (bits, group_size) == (4, 64):
            self._w4 = (w, scales, biases)
        elif widens_to_w4g64(bits, group_size) and w.is_cuda:
            self._w4 = kernels.widen_w4g64(w, scales, biases, self.H, group_size, bits)
            self.w, self.scales, self.biases = w.cpu(), scales.cpu(), biases.cpu()

    def w4g64(self):
        """(w, scales, biases) in the 4-bit group-64 layout on the device, or None."""
        return self._w4

    def __call__(self, ids: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        ids1 = ids.reshape(-1).to(torch.int32).contiguous()
        L = ids1.numel()
        if out is None:
            out = torch.empty((L, self.H), dtype=torch.bfloat16, device=ids.device)
        if self._w4 is None:
            return kernels.embed_affine(ids1, self.w, self.scales, self.biases, self.H, self.group_size, self.bits,
                                        out=out)
        w, sc, bi = self._w4
        _C.call("qvex_embed_w4g64", _ptr(ids1), L, _ptr(w), _ptr(sc), _ptr(bi), self.V, self.H, _ptr(out),
                _stream())
        return out


def rms_norm(x: torch.Tensor, w: torch.Tensor | None, eps: float, out=None, scale: float = 1.0):
    """mx.fast.rms_norm over the last dim (weight optional)."""
    D = x.shape[-1]
    x2 = x.reshape(-1, D)
    if out is None:
        out = torch.empty_like(x2)
    o2 = out.reshape(-1, out.shape[-1]) if out.dim() > 1 else out
    _C.call("qvex_rmsnorm", _ptr(x2), x2.stride(0), _ptr(w) if w is not None else None, _ptr(o2),
            o2.stride(0), x2.shape[0], D, float(eps), float(scale), _stream())
    return out


def add_rms_norm(x, delta, w, eps, h_out=None, out=None):
    """h = x + delta (bf16), n = rms_norm(h) * w; returns (h, n)."""
    R, D = x.reshape(-1, x.shape[-1]).shape
    h_out = torch.empty_like(x) if h_out is None else h_out
    out = torch.empty_like(x) if out is None else out
    _C.call("qvex_add_rmsnorm", _ptr(x), _ptr(delta), _ptr(h_out), _ptr(w), _ptr(out), R, D, float(eps), _stream())
    return h_out, out


class NormedRows:
    """rms_norm(h) * w for 1..8 rows kept unnormalised: u = bf16(h * w) and the
    fp32 sums of h^2 per 16 columns (written by the product that made h, or by
    rms_parts). A packed QLinear takes it as input and applies the per-row
    rsqrt(mean(h^2) + eps) to its outputs, so the norm costs no launch."""

    def __init__(self, u: torch.Tensor, parts: torch.Tensor, eps: float):
        self.u, self.parts, self.eps = u, parts, eps

    @classmethod
    def of(cls, x: torch.Tensor, w: torch.Tensor, eps: float) -> "NormedRows":
        u, parts = kernels.rms_parts(x, w)
        return cls(u, parts, eps)

    @staticmethod
    def supported(D: int) -> bool:
        n = (D + 15) // 16
        return n % 4 == 0 and n <= 256

    @property
    def shape(self):
        return self.u.shape

    @property
    def device(self):
        return self.u.device

    def __getitem__(self, rows) -> "NormedRows":
        return NormedRows(self.u[rows], self.parts[rows], self.eps)

    def materialize(self) -> torch.Tensor:
        """The normalised rows as a tensor (for a consumer without the packed path)."""
        D = self.u.shape[-1]
        ms = self.parts.sum(dim=-1, keepdim=True) / D
        return (self.u.float() * torch.rsqrt(ms + self.eps)).to(torch.bfloat16)


# ---------------------------------------------------------------- caches

class CacheCounters:
    """Device int32 table of per-cache token counts (one entry per cache), with a
    host mirror. Kernels read the device copy; ``sync()`` uploads host edits."""

    def __init__(self, n: int, device):
        self.host = np.zeros(n, np.int32)
        self.dev = torch.zeros(n, dtype=torch.int32, device=device)
        self.dirty = False
        # in graph mode the device table is authoritative (advanced by captured
        # commit kernels) and the host mirror is kept by the replaying code;
        # host edits are then refused except while a graph is being captured
        self.graph_mode = False
        self.capturing = False

    def _check_host_edit(self) -> None:
        if self.graph_mode and not self.capturing:
            raise _C.QvexError("these caches are driven by a captured cycle (GraphedMTPCycle); release() it "
                               "before eager calls, rollbacks or offset edits")

    def get(self, i: int) -> int:
        return int(self.host[i])

    def set(self, i: int, v: int) -> None:
        self._check_host_edit()
        self.host[i] = v
        self.dirty = True

    def sync(self) -> None:
        self._check_host_edit()
        if self.graph_mode:
            return
        if self.dirty:
            # from pageable memory: the runtime stages the bytes before returning,
            # so later host edits cannot race the copy
            self.dev.copy_(torch.from_numpy(self.host.copy()))
            self.dirty = False

    def ptr(self, i: int) -> int:
        return self.dev.data_ptr() + 4 * i

    def clone(self) -> "CacheCounters":
        self._check_host_edit()
        c = CacheCounters(len(self.host), self.dev.device)
        c.host[:] = self.host
        c.dev.copy_(self.dev)
        c.dirty = self.dirty
        return c


_ROPE_TABLES: dict = {}


def rope_table(rot: int, theta: float, rows: int, device, capturing: bool = False) -> torch.Tensor | None:
    """The (cos, sin) table [rows', rot/2, 2] of qvex_rope_table with rows' >=
    rows, shared by every attention layer with the same rot and theta on a
    device; grown (never inside a graph capture) when a larger cache appears."""
    if rot == 0:
        return None
    key = (int(rot), float(theta), str(torch.device(device)))
    t = _ROPE_TABLES.get(key)
    if t is None or t.shape[0] < rows:
        if capturing:
            raise _C.QvexError(f"rope table for {rows} positions missing while a graph is captured "
                               "(run one eager step with the cache first)")
        t = torch.empty((int(rows), rot // 2, 2), dtype=torch.float32, device=device)
        _C.call("qvex_rope_table", int(rot), float(theta), int(rows), _ptr(t), _stream())
        _ROPE_TABLES[key] = t
    return t


class KVCache:
    """bf16 K and V of Hkv heads x cap keys x D dims in the tiled layouts the
    attention kernels read 1 KiB at a time (K [Hkv, cap/16, D/32, 64, 8], V
    [Hkv, cap/32, D, 32]; ``keys()`` / ``values()`` give [Hkv, cap, D] copies),
    preallocated (engine/model.py:149-176 grows [B, H, cap, D] arrays in 256-token
    steps instead). rollback(n) is offset -= n."""

    step = 256

    def __init__(self, counters: CacheCounters | None = None, index: int = 0, *, n_kv: int = 0,
                 head_dim: int = 0, capacity: int = 0, device=None):
        if counters is None:
            counters = CacheCounters(1, device)
            index = 0
        self.counters, self.index = counters, index
        self.capacity = int(math.ceil(max(capacity, 1) / self.step) * self.step)
        if head_dim % 32:
            raise ValueError(f"KVCache: head_dim={head_dim} must be a multiple of 32")
        cap = self.capacity
        self.k = torch.zeros((n_kv, cap // 16, head_dim // 32, 64, 8), dtype=torch.bfloat16, device=device)
        self.v = torch.zeros((n_kv, cap // 32, head_dim, 32), dtype=torch.bfloat16, device=device)

    def keys(self) -> torch.Tensor:
        """K as [Hkv, cap, D] (a copy)."""
        return kernels.kv_untile_k(self.k)

    def values(self) -> torch.Tensor:
        """V as [Hkv, cap, D] (a copy)."""
        return kernels.kv_untile_v(self.v)

    @property
    def offset(self) -> int:
        return self.counters.get(self.index)

    @offset.setter
    def offset(self, v: int) -> None:
        self.counters.set(self.index, v)

    def state(self):
        return [self.k, self.v]

    def rollback(self, n=1):
        self.offset -= n  # entries past offset are overwritten by the next append

    def grow(self, min_capacity: int) -> bool:
        """Enlarge the cache to hold at least min_capacity keys, rounded up to a
        whole step (engine/model.py:156-170 grows by the same 256-token steps
        when an update would pass the end). The keys kept so far move to the new
        tiles; a HIP graph captured on the old buffers must be captured again.
        Returns whether the buffers changed."""
        self.counters._check_host_edit()
        if min_capacity <= self.capacity:
            return False
        cap = int(math.ceil(min_capacity / self.step) * self.step)
        k = torch.zeros((self.k.shape[0], cap // 16) + tuple(self.k.shape[2:]), dtype=self.k.dtype,
                        device=self.k.device)
        v = torch.zeros((self.v.shape[0], cap // 32) + tuple(self.v.shape[2:]), dtype=self.v.dtype,
                        device=self.v.device)
        # a head's tiles are consecutive and key-major: the old tiles are the new head's first ones
        k[:, : self.k.shape[1]].copy_(self.k)
        v[:, : self.v.shape[1]].copy_(self.v)
        self.k, self.v, self.capacity = k, v, cap
        return True

    def clone(self, counters: CacheCounters | None = None) -> "KVCache":
        """A copy of the cache (device tensors copied); counters: the cloned table
        it indexes (a new one-entry table for a standalone cache)."""
        c = KVCache.__new__(KVCache)
        c.counters = counters if counters is not None else self.counters.clone()
        c.index, c.capacity = self.index, self.capacity
        c.k, c.v = self.k.clone(), self.v.clone()
        return c


class RecurrentCache:
    """GDN caches: conv history ring and DeltaNet state ring, both indexed by
    the layer's token count, so ``rollback(n)`` (n <= last call width) only
    moves the counter. ``conv``/``ssm`` give the current state like the
    reference's fields (engine/model.py:179-193)."""

    def __init__(self, counters: CacheCounters, index: int, *, conv_dim: int, kernel: int, hv: int,
                 dv: int, dk: int, max_width: int, device, prefill_width: int = 64):
        self.counters, self.index = counters, index
        self.kernel = kernel
        self.ring_rows = max(max_width, prefill_width) + kernel - 1
        self.conv_ring = torch.zeros((self.ring_rows, conv_dim), dtype=torch.bfloat16, device=device)
        self.n_slots = max_width + 1
        self.ssm_ring = torch.zeros((self.n_slots, 1, hv, dv, dk), dtype=torch.float32, device=device)
        self.last_width = 0

    @property
    def offset(self) -> int:
        return self.counters.get(self.index)

    @offset.setter
    def offset(self, v: int) -> None:
        self.counters.set(self.index, v)

    @property
    def ssm(self) -> torch.Tensor:
        return self.ssm_ring[self.offset % self.n_slots]

    @property
    def conv(self) -> torch.Tensor:
        p, W, R = self.offset, self.kernel - 1, self.ring_rows
        rows = [(p - W + j) % R for j in range(W)]
        return self.conv_ring[rows]

    def state(self):
        return [self.conv_ring, self.ssm_ring]

    def rollback(self, n=1):
        self.counters._check_host_edit()
        if n > self.last_width:
            raise _C.QvexError(f"RecurrentCache.rollback({n}): only the last {self.last_width} tokens are kept")
        self.offset -= n
        self.last_width -= n

    def clone(self, counters: CacheCounters) -> "RecurrentCache":
        c = RecurrentCache.__new__(RecurrentCache)
        c.__dict__.update(self.__dict__)
        c.counters = counters
        c.conv_ring, c.ssm_ring = self.conv_ring.clone(), self.ssm_ring.clone()
        return c


class LayerCaches(list):
    """The list returned by make_cache(): one cache per layer, sharing counters."""

    def __init__(self, items, counters):
        super().__init__(items)
        self.counters = counters

    def clone(self) -> "LayerCaches":
        """A deep copy (device tensors and counters): a prefix to branch from."""
        counters = self.counters.clone()
        return LayerCaches([c.clone(counters) for c in self], counters)


# ---------------------------------------------------------------- layers

class Attention:
    """Gated full attention (engine/model.py:199-232) with q/k/v projections fused
    into one quantized matmul (lossless, like the reference's in_proj fusion)."""

    # keys per split of the decode / verify attention (a multiple of 128)
    decode_kps = 128
    fused_decode = False    # qvex_attention_decode for 1..8 new tokens (slower per cycle: see its header)
    late_splits = True      # captured: splits past the position at capture read it before loading

    def __init__(self, cfg: Config, p: dict):
        self.cfg = cfg
        self.n_heads, self.n_kv = cfg.num_attention_heads, cfg.num_key_value_heads
        self.head_dim = cfg.head_dim
        self.qkv_proj = QLinear.fuse([p["q_proj"], p["k_proj"], p["v_proj"]])
        self.o_proj = p["o_proj"]
        self.q_norm, self.k_norm = p["q_norm"], p["k_norm"]
        self._ws = None

    def _workspace(self, L, cap, kps, device):
        need = int(_C.lib().qvex_attn_workspace_bytes(L, self.n_heads, self.n_kv, self.head_dim, cap, kps))
        if self._ws is None or self._ws.numel() * 4 < need:
            self._ws = torch.empty((need + 3) // 4, dtype=torch.float32, device=device)
        return self._ws

    def __call__(self, x, cache: KVCache, resid=None, norm_w=None, eps=None):
        """x [L, H] (or NormedRows); with resid the o_proj also adds the residual
        and prepares the next norm (QLinear.residual)."""
        L = x.shape[0]
        cfg = self.cfg
        H, Hkv, D = self.n_heads, self.n_kv, self.head_dim
        if not cache.counters.graph_mode and cache.offset + L > cache.capacity:
            # grown in 256-token steps as engine/model.py:156-170 does; a captured
            # call cannot move its buffers (GraphedMTPCycle checks room before each
            # replay, and decode() grows the caches and captures again)
            cache.grow(cache.offset + L)
        proj = self.qkv_proj(x)                                   # [L, H*2D + 2*Hkv*D]
        pos = cache.counters.ptr(cache.index)
        # a captured call must work for every later context length: bound by capacity
        max_keys = cache.capacity if cache.counters.graph_mode else min(cache.capacity, cache.offset + L)
        kps = self.decode_kps if L <= 8 else 512   # keys per 4-wave block: verify spreads ~ctx/32 waves per kv head
        ws = self._workspace(L, max_keys, kps, x.device)
        o = torch.empty((L, H * D), dtype=torch.bfloat16, device=x.device)
        rot = cfg.rotary_dim
        if self.fused_decode and L <= 8 and (rot == 0 or ((rot // 2) % (D // 16) == 0 and L * (rot // 2) <= 256)):
            # norms, RoPE and the cache append inside the split kernel
            tab = rope_table(rot, cfg.rope_theta, cache.capacity, x.device, cache.counters.graph_mode)
            _C.call("qvex_attention_decode", _ptr(proj), proj.stride(0), _ptr(self.q_norm), _ptr(self.k_norm), pos,
                    L, H, Hkv, D, rot, float(cfg.rms_norm_eps), _ptr(tab) if tab is not None else 0,
                    tab.shape[0] if tab is not None else 0, _ptr(cache.k), _ptr(cache.v), cache.capacity, max_keys,
                    kps, _ptr(o), _ptr(ws), ws.numel() * 4, _stream())
        else:
            q = torch.empty((L, H, D), dtype=torch.bfloat16, device=x.device)
            # the rotation's (cos, sin) from the shared table covering the cache; a
            # call under graph capture never makes one (decode() makes it before
            # capturing) and without it the kernel evaluates the same angles
            tab = None
            if rot:
                key = (int(rot), float(cfg.rope_theta), str(torch.device(x.device)))
                have = _ROPE_TABLES.get(key)
                if torch.cuda.is_current_stream_capturing():
                    tab = have if have is not None and have.shape[0] >= cache.capacity else None
                else:
                    tab = rope_table(rot, cfg.rope_theta, cache.capacity, x.device)
            _C.call("qvex_attn_qk_rope", _ptr(proj), proj.stride(0), _ptr(self.q_norm), _ptr(self.k_norm), pos,
                    L, H, Hkv, D, rot, float(cfg.rope_theta), float(cfg.rms_norm_eps), _ptr(q),
                    _ptr(cache.k), _ptr(cache.v), cache.capacity, _ptr(tab) if tab is not None else 0,
                    tab.shape[0] if tab is not None else 0, _stream())
            # keys below the position at capture stay visible on every replay
            known = min(cache.offset, max_keys) if cache.counters.graph_mode and self.late_splits else max_keys
            _C.call("qvex_attention", _ptr(q), _ptr(cache.k), _ptr(cache.v), pos, L, H, Hkv, D, cache.capacity,
                    max_keys, known, kps, _ptr(proj), proj.stride(0), _ptr(o), _ptr(ws), ws.numel() * 4, _stream())
        cache.offset += L
        if resid is not None:
            return self.o_proj.residual(o, resid, norm_w, eps)
        return self.o_proj(o)


class GatedDeltaNet:
    """Gated DeltaNet block (engine/model.py:235-291)."""

    def __init__(self, cfg: Config, p: dict):
        self.cfg = cfg
        self.hk, self.hv = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        self.dk, self.dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        self.key_dim, self.value_dim = self.hk * self.dk, self.hv * self.dv
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.K = cfg.linear_conv_kernel_dim
        self.in_proj = QLinear.fuse([p["in_proj_qkv"], p["in_proj_z"], p["in_proj_b"], p["in_proj_a"]])
        self.conv_w = p["conv1d"]          # bf16 [conv_dim, K]
        self.A_log, self.dt_bias = p["A_log"], p["dt_bias"]
        self.norm_w = p["norm"]
        self.out_proj = p["out_proj"]

    # 1..8 tokens (decode / verify) run the conv, recurrence and gated norm as
    # one kernel (qvex_gdn_decode_fused, bitwise the three-kernel path)
    FUSED_MAX_T = 8
    fused_decode = True
    # calls of at least this many tokens without snapshots (prefill) use the
    # chunked recurrence (qvex_gdn_chunked); larger than any ring-snapshot width
    CHUNKED_MIN_T = 64
    # with the norms folded (resid given, <= 8 rows) each head is split over this
    # many workgroups (qvex_gdn_decode_split) and the gated norm's scale moves
    # into the out_proj; 0 keeps one workgroup per head. 8: 16 state rows per
    # workgroup on one wave per SIMD, its other 4 waves on conv tasks (-4.5 us
    # per decode cycle against 4 at the 9B shape)
    split_blocks = 8

    def _out(self, g, resid, norm_w, eps):
        if resid is not None:
            return self.out_proj.residual(g, resid, norm_w, eps)
        return self.out_proj(g)

    def __call__(self, x, cache: RecurrentCache, keep_prev=False, resid=None, norm_w=None, eps=None):
        """x [S, H] (or NormedRows); with resid the out_proj also adds the residual
        and prepares the next norm (QLinear.residual)."""
        S = x.shape[0]
        dev = x.device
        proj = self.in_proj(x)                                    # [S, conv | z | b | a]
        if self.fused_decode and S <= self.FUSED_MAX_T and self.dk == 128 and self.dv == 128 and self.K == 4:
            if (self.split_blocks and resid is not None and S <= QLinear.PACKED_MAX_ROWS
                    and self.out_proj.packed is not None and NormedRows.supported(self.out_proj.N)):
                u, ss = self.mix_split(proj, cache)
                h, un, parts = kernels.qmv_packed_gnorm_resid(u, ss, self.out_proj.packed, self.out_proj.N,
                                                              float(self.cfg.rms_norm_eps), resid.reshape(S, -1),
                                                              norm_w)
                return h, NormedRows(un, parts, eps)
            return self._out(self.mix_fused(proj, cache), resid, norm_w, eps)
        q = torch.empty((1, S, self.hk, self.dk), dtype=torch.bfloat16, device=dev)
        k = torch.empty_like(q)
        v = torch.empty((1, S, self.hv, self.dv), dtype=torch.bfloat16, device=dev)
        a = torch.empty((1, S, self.hv), dtype=torch.bfloat16, device=dev)
        b = torch.empty_like(a)
        inv = self.dk ** -0.5
        pos = cache.counters.ptr(cache.index)
        ab_off = self.conv_dim + self.value_dim
        _C.call("qvex_gdn_conv_qk", _ptr(proj), proj.stride(0), _ptr(cache.conv_ring), cache.ring_rows, pos,
                _ptr(self.conv_w), self.K, _ptr(q), _ptr(k), _ptr(v), _ptr(a), _ptr(b), S, self.conv_dim,
                self.key_dim, self.hv, ab_off, float(inv * inv), float(inv), 1e-6, _stream())
        snap = S <= cache.n_slots - 1
        if not snap and S >= self.CHUNKED_MIN_T and self.dk == 128 and self.dv == 128:
            # long prefill chunk: the 64-token MFMA form, state read from the
            # current slot and the final state written to slot (p + S) mod n
            cur = cache.offset % cache.n_slots
            nxt = (cache.offset + S) % cache.n_slots
            y, _ = kernels.gated_delta_chunked(q, k, v, a, b, self.A_log, self.dt_bias, cache.ssm_ring[cur],
                                               state_out=cache.ssm_ring[nxt])
        else:
            y = kernels.gated_delta_ring(q, k, v, a, b, self.A_log, self.dt_bias, cache.ssm_ring,
                                         cache.counters.dev[cache.index:cache.index + 1], snap_every=snap)
        cache.offset += S
        cache.last_width = S if snap else 0
        z = proj[:, self.conv_dim:self.conv_dim + self.value_dim]
        g = torch.empty((S, self.value_dim), dtype=torch.bfloat16, device=dev)
        _C.call("qvex_gated_rmsnorm", _ptr(y), _ptr(proj) + 2 * self.conv_dim, proj.stride(0), self.hv,
                _ptr(self.norm_w), _ptr(g), S * self.hv, self.dv, float(self.cfg.rms_norm_eps), _stream())
        return self._out(g, resid, norm_w, eps)

    def mix_fused(self, proj, cache: RecurrentCache):
        """conv + recurrence + gated norm of S <= 8 rows of in_proj output in one
        launch; returns the out_proj input [S, value_dim] and advances the cache."""
        S = proj.shape[0]
        g = torch.empty((S, self.value_dim), dtype=torch.bfloat16, device=proj.device)
        inv = self.dk ** -0.5
        snap = S <= cache.n_slots - 1
        _C.call("qvex_gdn_decode_fused", _ptr(proj), proj.stride(0), _ptr(cache.conv_ring), cache.ring_rows,
                cache.counters.ptr(cache.index), _ptr(self.conv_w), self.K, self.conv_dim, self.key_dim,
                float(inv * inv), float(inv), 1e-6, _ptr(self.A_log), _ptr(self.dt_bias), self.conv_dim,
                self.conv_dim + self.value_dim, _ptr(cache.ssm_ring), cache.n_slots, int(snap), _ptr(self.norm_w),
                float(self.cfg.rms_norm_eps), _ptr(g), S, self.hk, self.hv, self.dk, self.dv, _stream())
        cache.offset += S
        cache.last_width = S if snap else 0
        return g

    def mix_split(self, proj, cache: RecurrentCache):
        """mix_fused over split_blocks workgroups per head: returns the unscaled
        gated-norm input u [S, value_dim] and the per-workgroup sums of y^2
        [S, hv, split_blocks] (the out_proj applies the scale)."""
        S = proj.shape[0]
        nb = self.split_blocks
        u = torch.empty((S, self.value_dim), dtype=torch.bfloat16, device=proj.device)
        ss = torch.empty((S, self.hv, nb), dtype=torch.float32, device=proj.device)
        inv = self.dk ** -0.5
        snap = S <= cache.n_slots - 1
        _C.call("qvex_gdn_decode_split", _ptr(proj), proj.stride(0), _ptr(cache.conv_ring), cache.ring_rows,
                cache.counters.ptr(cache.index), _ptr(self.conv_w), self.K, self.conv_dim, self.key_dim,
                float(inv * inv), float(inv), 1e-6, _ptr(self.A_log), _ptr(self.dt_bias), self.conv_dim,
                self.conv_dim + self.value_dim, _ptr(cache.ssm_ring), cache.n_slots, int(snap), _ptr(self.norm_w),
                _ptr(u), _ptr(ss), S, self.hk, self.hv, self.dk, self.dv, nb, _stream())
        cache.offset += S
        cache.last_width = S if snap else 0
        return u, ss


class MLP:
    """down(silu(gate(x)) * up(x)) (engine/model.py:294-302); for 1..8 rows the
    SwiGLU is fused into the gate/up product."""

    def __init__(self, p: dict):
        self.gate_up = QLinear.fuse([p["gate_proj"], p["up_proj"]], swiglu=True)
        self.down = p["down_proj"]
        self.hidden = p["gate_proj"].N

    def __call__(self, x):
        return self.down(self.gate_up.swiglu(x))


class Layer:
    def __init__(self, cfg: Config, i: int, p: dict):
        self.linear = cfg.is_linear(i)
        self.mixer = GatedDeltaNet(cfg, p["linear_attn"]) if self.linear else Attention(cfg, p["self_attn"])
        self.mlp = MLP(p["mlp"])
        self.ln1, self.ln2 = p["input_layernorm"], p["post_attention_layernorm"]
        self.eps = cfg.rms_norm_eps

    def fused(self, h, st, cache, keep_prev, next_w, h_out=None):
        """1..8 rows with the norms folded into the products: h the residual stream,
        st its ln1 norm as NormedRows; returns the new stream (into h_out when
        given) and its norm by next_w."""
        kw = dict(resid=h, norm_w=self.ln2, eps=self.eps)
        h2, st2 = self.mixer(st, cache, keep_prev, **kw) if self.linear else self.mixer(st, cache, **kw)
        return self.mlp.down.residual(self.mlp.gate_up.swiglu(st2), h2, next_w, self.eps, h_out=h_out)

    def __call__(self, x, cache, keep_prev=False, normed=None):
        """x [L, H] residual stream. Returns the new residual stream."""
        n = normed if normed is not None else rms_norm(x, self.ln1, self.eps)
        d = self.mixer(n, cache, keep_prev) if self.linear else self.mixer(n, cache)
        h, n2 = add_rms_norm(x, d, self.ln2, self.eps)
        m = self.mlp(n2)
        return h, m


class Qwen35:
    """Forward of the hybrid stack (engine/model.py:319-336) for batch 1."""

    # 1..8-row calls fold every residual RMSNorm into the neighbouring products
    # (QLinear.residual / NormedRows); False keeps the separate norm kernels
    fuse_norms = True
    # prompt tokens per forward call of a prefill (engine/engine.py:232-248 runs
    # 512-token chunks); the conv rings are sized for it
    prefill_chunk = 512

    def __init__(self, cfg: Config, embed: QEmbedding, layers: list[Layer], norm, lm_head: QLinear,
                 max_context: int = 8192, max_width: int = 8):
        self.cfg = cfg
        self.embed, self.layers, self.norm, self.lm_head = embed, layers, norm, lm_head
        self.max_context, self.max_width = max_context, max_width

    def make_cache(self, max_context: int | None = None, max_width: int | None = None):
        cfg = self.cfg
        dev = self.norm.device
        cap = max_context or self.max_context
        width = max_width or self.max_width
        counters = CacheCounters(len(self.layers), dev)
        caches = []
        for i, l in enumerate(self.layers):
            if l.linear:
                caches.append(RecurrentCache(counters, i, conv_dim=l.mixer.conv_dim, kernel=l.mixer.K,
                                             hv=l.mixer.hv, dv=l.mixer.dv, dk=l.mixer.dk,
                                             max_width=width, device=dev, prefill_width=self.prefill_chunk))
            else:
                caches.append(KVCache(counters, i, n_kv=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                                      capacity=cap, device=dev))
        return LayerCaches(caches, counters)

    def qlinears(self):
        """Every QLinear of the stack (the shared lm_head included)."""
        for l in self.layers:
            m = l.mixer
            if l.linear:
                yield from (m.in_proj, m.out_proj)
            else:
                yield from (m.qkv_proj, m.o_proj)
            yield from (l.mlp.gate_up, l.mlp.down)
        yield self.lm_head

    def offload_mlx(self) -> None:
        """QLinear.offload_mlx for every layer: one device copy of each weight."""
        for q in self.qlinears():
            q.offload_mlx()

    def all_packed(self) -> bool:
        """Every product has the packed copy (4-bit group-64, or widened to it):
        the condition for folding the norms into the products' epilogues; a
        model with any other width runs the separate norm kernels."""
        return all(q.packed is not None for q in self.qlinears())

    def _deferred_argmax(self) -> bool:
        """The decode cycle may leave each draft's argmax to the next launch."""
        return self.fuse_norms and self.all_packed() and self._fused_inputs()

    def _fused_inputs(self) -> bool:
        e = self.embed
        return isinstance(e, QEmbedding) and e.w4g64() is not None and e.H % 64 == 0 and e.H <= 8192

    def __call__(self, ids, cache, last_only=True, return_hidden=False, keep_prev=False, hidden_out=None,
                 in_argmax=None, tile_max_out=None):
        """ids: [1, L] int -> logits [1, L or 1, V] bf16 (and pre-norm hidden [1, L, H],
        written into hidden_out when given). in_argmax = (pairs, row, slot): ids[slot]
        is first set, on the device, to the token of the deferred lm_head argmax
        `pairs` (QLinear.argmax with out=None), row `row` (device int32 or None).
        tile_max_out: bf16 [rows, ceil(V/16)] for the logits rows' 16-column tile
        maxima (QLinear.with_tile_max), which Sampler.accept_device takes."""
        ids = torch.as_tensor(ids, device=self.norm.device).reshape(-1)
        L = ids.numel()
        counters = cache.counters
        # chunk long inputs so every call fits the conv rings (prefill)
        step = L
        for c in cache:
            if isinstance(c, RecurrentCache):
                step = min(step, c.ring_rows - c.kernel + 1)
        if L > step:
            outs, hs = [], []
            for s0 in range(0, L, step):
                ho = None if hidden_out is None else hidden_out.view(L, -1)[s0:s0 + step]
                r = self(ids[s0:s0 + step].reshape(1, -1), cache, last_only=last_only and s0 + step >= L,
                         return_hidden=return_hidden, keep_prev=keep_prev, hidden_out=ho)
                if return_hidden:
                    outs.append(r[0]); hs.append(r[1])
                else:
                    outs.append(r)
            logits = outs[-1] if last_only else torch.cat(outs, dim=1)
            return (logits, torch.cat(hs, dim=1)) if return_hidden else logits
        counters.sync()
        eps = self.cfg.rms_norm_eps
        fused = (self.fuse_norms and L <= QLinear.PACKED_MAX_ROWS and NormedRows.supported(self.cfg.hidden_size)
                 and self.all_packed())
        if in_argmax is not None and not (fused and self._fused_inputs()):
            raise _C.QvexError("in_argmax needs the fused decode path (1..8 rows, 4-bit group-64 embedding)")
        if fused and self._fused_inputs():
            # embedding + the first norm's inputs in one launch (and the last
            # draft's argmax, when the caller left it to this launch)
            am, am_row, am_slot = in_argmax if in_argmax is not None else (None, None, -1)
            ids32 = ids if ids.dtype == torch.int32 and ids.is_contiguous() else ids.to(torch.int32).contiguous()
            if am is not None and ids32 is not ids:
                raise _C.QvexError("in_argmax needs ids as a contiguous int32 device tensor (the slot is written)")
            x, u, parts = kernels.embed_rms_parts(self.embed, ids32, self.layers[0].ln1, am, am_row, am_slot)
            st = NormedRows(u, parts, eps)
        else:
            x = self.embed(ids)
            if fused:
                st = NormedRows.of(x, self.layers[0].ln1, eps)
        if fused:
            # decode / verify: residual adds and norms ride on the products' epilogues
            h = x
            for i, (layer, c) in enumerate(zip(self.layers, cache)):
                last = i + 1 == len(self.layers)
                nxt = self.norm if last else self.layers[i + 1].ln1
                h, st = layer.fused(h, st, c, keep_prev, nxt, h_out=hidden_out if last else None)
            xs = st[-1:] if last_only else st
            logits = (self.lm_head(xs) if tile_max_out is None else self.lm_head.with_tile_max(xs, tile_max_out))
            logits = logits.view(1, -1, self.cfg.vocab_size)
            return (logits, h.view(1, L, -1)) if return_hidden else logits
        n = rms_norm(x, self.layers[0].ln1, eps)
        for i, (layer, c) in enumerate(zip(self.layers, cache)):
            h, m = layer(x, c, keep_prev, normed=n)
            nxt = self.layers[i + 1].ln1 if i + 1 < len(self.layers) else self.norm
            x, n = add_rms_norm(h, m, nxt, eps)
        hidden = x
        if hidden_out is not None:
            hidden_out.view(L, -1).copy_(hidden.view(L, -1))
            hidden = hidden_out
        if last_only:
            n = n[-1:]
        logits = self.lm_head(n) if tile_max_out is None else self.lm_head.with_tile_max(n, tile_max_out)
        logits = logits.view(1, -1, self.cfg.vocab_size)
        return (logits, hidden.view(1, L, -1)) if return_hidden else logits


# ---------------------------------------------------------------- random init in the MLX layout

def _rand_qlinear(N, K, gen, scale, device, pack: bool = True, group_size: int = 64, bits: int = 4) -> QLinear:
    """Random affine weights: codes uniform on 0..2^bits-1 (uniform random stream
    words), scales ~ U(0.5, 1.5) * scale, biases = -2^(bits-1) * scale (zero-mean
    dequantized weights). `scale` is given for 4 bits (code variance 21.25);
    other widths rescale it so the dequantized variance is the same."""
    _check_quant("random weights", bits, group_size)
    w = torch.randint(-2**31, 2**31, (N, K * bits // 32), generator=gen, device=device, dtype=torch.int64)
    w = w.to(torch.int32)
    if bits != 4:
        scale = scale * math.sqrt(21.25 / ((4 ** bits - 1) / 12))
    s = (torch.rand((N, K // group_size), generator=gen, device=device) + 0.5) * scale
    s = s.to(torch.bfloat16)
    b = (-float(2 ** (bits - 1)) * s.float()).to(torch.bfloat16)
    return QLinear(w, s, b, group_size, bits, pack=pack)


def random_model(cfg: Config, seed: int = 1004, device="cuda", max_context: int = 8192,
                 max_width: int = 8, lm_head_scale: float = 2.0, keep_mlx: bool = False) -> Qwen35:
    """Random-init model of the given shape with weights generated directly in the
    MLX affine layout on the device (no checkpoint): 4-bit group-64 unless the
    config's quantization overrides (Config.qparams) name another width for a
    module (model.layers.{i}.mlp.gate_proj, ..., model.embed_tokens, lm_head).
    Linear scales are chosen so a
    unit-RMS input gives a unit-RMS output (dequantized w has variance 21.25 s^2).
    Unless keep_mlx, each packed layer's MLX-layout triplet then moves to host
    memory (QLinear.offload_mlx)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    H, I = cfg.hidden_size, cfg.intermediate_size

    def lin(N, K, gain=1.0, name=""):
        gs, bits = cfg.qparams(name)
        return _rand_qlinear(N, K, gen, gain / math.sqrt(21.25 * K), device, group_size=gs, bits=bits)

    def ones(n):
        return (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)

    layers = []
    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}"
        mlp = f"{pre}.mlp"
        p = {"input_layernorm": ones(H), "post_attention_layernorm": ones(H),
             "mlp": {"gate_proj": lin(I, H, name=f"{mlp}.gate_proj"), "up_proj": lin(I, H, name=f"{mlp}.up_proj"),
                     "down_proj": lin(H, I, 0.5, f"{mlp}.down_proj")}}
        if cfg.is_linear(i):
            kd = cfg.linear_num_key_heads * cfg.linear_key_head_dim
            vd = cfg.linear_num_value_heads * cfg.linear_value_head_dim
            conv_dim = 2 * kd + vd
            hv = cfg.linear_num_value_heads
            la = f"{pre}.linear_attn"
            p["linear_attn"] = {
                "in_proj_qkv": lin(conv_dim, H, name=f"{la}.in_proj_qkv"),
                "in_proj_z": lin(vd, H, name=f"{la}.in_proj_z"),
                "in_proj_b": lin(hv, H, name=f"{la}.in_proj_b"), "in_proj_a": lin(hv, H, name=f"{la}.in_proj_a"),
                "out_proj": lin(H, vd, 0.5, f"{la}.out_proj"),
                "conv1d": (0.5 * torch.randn((conv_dim, cfg.linear_conv_kernel_dim), generator=gen,
                                             device=device)).to(torch.bfloat16),
                "A_log": (0.5 * torch.randn(hv, generator=gen, device=device)).float(),
                "dt_bias": (0.5 * torch.randn(hv, generator=gen, device=device)).to(torch.bfloat16),
                "norm": ones(cfg.linear_value_head_dim),
            }
        else:
            D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
            sa = f"{pre}.self_attn"
            p["self_attn"] = {"q_proj": lin(Hq * 2 * D, H, name=f"{sa}.q_proj"),
                              "k_proj": lin(Hkv * D, H, name=f"{sa}.k_proj"),
                              "v_proj": lin(Hkv * D, H, name=f"{sa}.v_proj"),
                              "o_proj": lin(H, Hq * D, 0.5, f"{sa}.o_proj"),
                              "q_norm": ones(D), "k_norm": ones(D)}
        layers.append(Layer(cfg, i, p))
    V = cfg.vocab_size
    egs, ebits = cfg.qparams("model.embed_tokens")
    e = _rand_qlinear(V, H, gen, 1.0 / math.sqrt(21.25), device, pack=False, group_size=egs, bits=ebits)
    embed = QEmbedding(e.w, e.scales, e.biases, egs, ebits)
    lm_head = lin(V, H, lm_head_scale, "lm_head")
    model = Qwen35(cfg, embed, layers, ones(H), lm_head, max_context=max_context, max_width=max_width)
    if not keep_mlx:
        model.offload_mlx()
    return model
