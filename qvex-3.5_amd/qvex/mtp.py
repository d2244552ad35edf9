"""Multi-token prediction (MTP) head of Qwen3.5 as the draft model
(mirror of engine/mtp.py).

    x = fc([rms(embed(tok_{i+1})), rms(h_i)]) -> attention + MLP block -> norm -> lm_head

It shares embed_tokens and lm_head with the main model; its attention layer keeps
its own KV cache. For k > 1 drafts the head is chained on its own output: draft
step j + 1 takes (hidden after the MTP block at step j, draft token j), a
convention of this implementation (the reference drafts one token).
"""

from __future__ import annotations

import math

import torch

from . import _C, kernels
from .kernels import _ptr, _stream
from .model import (Attention, KVCache, Layer, MLP, NormedRows, QLinear, Qwen35, _rand_qlinear, add_rms_norm,
                    rms_norm)


class MTPHead:
    # the first norm of the block from the fc product's epilogue (False: its own launch)
    fc_epilogue = True

    def __init__(self, model: Qwen35, w: dict, group_size: int = 64, bits: int = 4, hidden_mode: str = "pre"):
        cfg = model.cfg
        self.model = model
        self.eps = cfg.rms_norm_eps
        self.hidden_mode = hidden_mode  # "pre": raw last-layer output, "post": after the final norm
        self.fc = w["fc"]
        self.norm_emb, self.norm_hid, self.norm_out = w["norm_emb"], w["norm_hid"], w["norm_out"]
        layer = Layer.__new__(Layer)
        layer.linear = False
        layer.eps = cfg.rms_norm_eps
        layer.ln1, layer.ln2 = w["ln1"], w["ln2"]
        layer.mixer = Attention(cfg, w["attn"])
        layer.mlp = MLP(w["mlp"])
        self.layer = layer
        # zero residual for the fc product, whose epilogue then leaves the block
        # input x = bf16(0 + fc(.)) and the first norm's inputs (allocated here,
        # never inside a graph capture)
        self._zero = torch.zeros((QLinear.PACKED_MAX_ROWS, cfg.hidden_size), dtype=torch.bfloat16,
                                 device=model.norm.device)

    def qlinears(self):
        m = self.layer.mixer
        return [self.fc, m.qkv_proj, m.o_proj, self.layer.mlp.gate_up, self.layer.mlp.down]

    def all_packed(self) -> bool:
        """The head's products and the shared lm_head all have packed copies
        (the norms then ride on their epilogues, as in Qwen35.all_packed)."""
        return self.model.lm_head.packed is not None and all(q.packed is not None for q in self.qlinears())

    def offload_mlx(self) -> None:
        """QLinear.offload_mlx for the head's own layers (the lm_head is the model's)."""
        for q in self.qlinears():
            q.offload_mlx()

    def make_cache(self, max_context: int | None = None) -> KVCache:
        cfg = self.model.cfg
        return KVCache(None, 0, n_kv=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                       capacity=max_context or self.model.max_context, device=self.model.norm.device)

    def __call__(self, hidden, next_ids, cache: KVCache, last_only=True, return_hidden=False, select=None,
                 argmax_out=None, defer_argmax=False, in_argmax=None, hid_sel=None, commit=None):
        """hidden [1, T, H] (main model, pre-norm) and next_ids [1, T] -> logits
        [1, 1 or T, V] (engine/mtp.py:58-68); with return_hidden also the block
        output [1, T, H] before the final norm (what a chained draft step takes).
        select: optional device int32 [1] row index; only that row goes through
        the lm_head (and is returned as the hidden), chosen on the device.
        argmax_out: optional int32 [1]; the greedy draft of the (selected or last)
        row is written there by the lm_head's argmax epilogue and no logits are
        made (logits returned as None).
        Launch-saving forms of the decode cycle (4-bit group-64 embedding, "pre"
        hidden): defer_argmax returns the lm_head's per-tile argmax pairs of the
        last (or, with last_only False, every) row in place of logits, for the next
        launch to reduce; in_argmax = (pairs, row, ids_out) takes the step's token
        (T = 1) from such pairs, row `row` (device int32 or None), storing it to
        ids_out; hid_sel: device row index of `hidden`; commit = (counters, n,
        extra) adds *n (None: 0) + extra to the cache counters in the same launch
        (the previous step's advance)."""
        H = self.model.cfg.hidden_size
        h = hidden.reshape(-1, H)
        if in_argmax is not None:
            ids, T = None, 1
        else:
            ids = torch.as_tensor(next_ids, device=h.device).reshape(-1)
            T = ids.numel()
        if self.hidden_mode == "post":
            h = rms_norm(h, self.model.norm, self.eps)
        cache.counters.sync()
        x_in = torch.empty((T, 2 * H), dtype=torch.bfloat16, device=h.device)
        if self.model._fused_inputs():
            # embedding + both input norms (+ the previous draft's argmax and the
            # previous step's counter advance) in one launch
            am, am_row, ids_out = in_argmax if in_argmax is not None else (None, None, None)
            cnt, n_ptr, extra = commit if commit is not None else (None, None, 0)
            ids32 = None
            if ids is not None:
                ids32 = ids if ids.dtype == torch.int32 and ids.is_contiguous() else ids.to(torch.int32).contiguous()
            kernels.mtp_input(self.model.embed, ids32, T, self.norm_emb, h, self.norm_hid, self.eps, x_in,
                              hid_sel=hid_sel, am=am, am_row=am_row, ids_out=ids_out,
                              counters=cnt.dev if cnt is not None else None, n_accept=n_ptr, extra=extra)
        else:
            if in_argmax is not None or hid_sel is not None or commit is not None:
                raise _C.QvexError("in_argmax / hid_sel / commit need a 4-bit group-64 embedding")
            e = self.model.embed(ids)
            # [rms(embed) | rms(hidden)] in one launch
            _C.call("qvex_rmsnorm_pair", _ptr(e), e.stride(0), _ptr(self.norm_emb), _ptr(x_in), _ptr(h), h.stride(0),
                    _ptr(self.norm_hid), _ptr(x_in) + 2 * H, x_in.stride(0), T, H, float(self.eps), _stream())
        V = self.model.cfg.vocab_size
        if (self.model.fuse_norms and T <= QLinear.PACKED_MAX_ROWS and NormedRows.supported(H)
                and self.all_packed()):
            # the block's residual norms ride on its products (Layer.fused); the
            # first one on the fc product, as a residual add onto zero
            if self.fc_epilogue:
                x, n1 = self.fc.residual(x_in, self._zero[:T], self.layer.ln1, self.eps)
            else:
                x, n1 = self.fc(x_in), None
            if not isinstance(n1, NormedRows):
                n1 = NormedRows.of(x, self.layer.ln1, self.eps)
            out, st = self.layer.fused(x, n1, cache, False, self.norm_out)
            if defer_argmax:
                am = self.model.lm_head.argmax(st[-1:] if last_only else st, None)
                return (am, out.view(1, T, H)) if return_hidden else am
            if select is not None:
                o_sel = torch.empty((1, H), dtype=torch.bfloat16, device=h.device)
                _C.call("qvex_gather_row", _ptr(out), H, _ptr(select), T, _ptr(o_sel), H, _stream())
                st_sel = NormedRows.of(o_sel, self.norm_out, self.eps)
                if argmax_out is not None:
                    self.model.lm_head.argmax(st_sel, argmax_out)
                    return (None, o_sel.view(1, 1, H)) if return_hidden else None
                logits = self.model.lm_head(st_sel).view(1, 1, V)
                return (logits, o_sel.view(1, 1, H)) if return_hidden else logits
            if argmax_out is not None and last_only:
                self.model.lm_head.argmax(st[-1:], argmax_out)
                return (None, out.view(1, T, H)) if return_hidden else None
            logits = self.model.lm_head(st[-1:] if last_only else st).view(1, -1, V)
            if argmax_out is not None:
                from .speculative import _argmax
                _argmax(logits[0, -1], out=argmax_out)
            return (logits, out.view(1, T, H)) if return_hidden else logits
        if defer_argmax:
            raise _C.QvexError("defer_argmax needs the fused path (1..8 rows)")
        x = self.fc(x_in)
        n = rms_norm(x, self.layer.ln1, self.eps)
        hh, m = self.layer(x, cache, normed=n)
        out, n_out = add_rms_norm(hh, m, self.norm_out, self.eps)
        if select is not None:
            n_sel = torch.empty((1, H), dtype=torch.bfloat16, device=h.device)
            o_sel = torch.empty((1, H), dtype=torch.bfloat16, device=h.device)
            _C.call("qvex_gather_row", _ptr(n_out), H, _ptr(select), T, _ptr(n_sel), H, _stream())
            _C.call("qvex_gather_row", _ptr(out), H, _ptr(select), T, _ptr(o_sel), H, _stream())
            logits = self.model.lm_head(n_sel).view(1, 1, self.model.cfg.vocab_size)
            if argmax_out is not None:
                from .speculative import _argmax
                _argmax(logits[0, -1], out=argmax_out)
            return (logits, o_sel.view(1, 1, H)) if return_hidden else logits
        if last_only:
            n_out = n_out[-1:]
        logits = self.model.lm_head(n_out).view(1, -1, self.model.cfg.vocab_size)
        if argmax_out is not None:
            from .speculative import _argmax
            _argmax(logits[0, -1], out=argmax_out)
        return (logits, out.view(1, T, H)) if return_hidden else logits


def random_mtp(model: Qwen35, seed: int = 2004, keep_mlx: bool = False, group_size: int = 64,
               bits: int = 4) -> MTPHead:
    """Random-init MTP head (fc 2H -> H plus one full-attention layer) in the MLX
    affine layout of the given width (the head file's one group_size / bits;
    the MLX triplets moved to host memory unless keep_mlx)."""
    cfg = model.cfg
    dev = model.norm.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    Hq, Hkv = cfg.num_attention_heads, cfg.num_key_value_heads

    def lin(N, K, gain=1.0):
        return _rand_qlinear(N, K, gen, gain / math.sqrt(21.25 * K), dev, group_size=group_size, bits=bits)

    def ones(n):
        return (1.0 + 0.1 * torch.randn(n, generator=gen, device=dev)).to(torch.bfloat16)

    w = {"fc": lin(H, 2 * H), "norm_emb": ones(H), "norm_hid": ones(H), "norm_out": ones(H),
         "ln1": ones(H), "ln2": ones(H),
         "attn": {"q_proj": lin(Hq * 2 * D, H), "k_proj": lin(Hkv * D, H), "v_proj": lin(Hkv * D, H),
                  "o_proj": lin(H, Hq * D, 0.5), "q_norm": ones(D), "k_norm": ones(D)},
         "mlp": {"gate_proj": lin(I, H), "up_proj": lin(I, H), "down_proj": lin(H, I, 0.5)}}
    head = MTPHead(model, w, group_size, bits)
    if not keep_mlx:
        head.offload_mlx()
    return head
