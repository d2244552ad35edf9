"""Token sampling on the device (mirror of engine/sampler.py).

The fused kernel (qvex_spec_accept_filtered) scores the target rows as
Sampler.scores does (presence penalty, temperature, top-k, top-p over the top-k
candidates or, with top_k = 0 or >= V, over the whole vocabulary), then runs
the speculative accept test, residual resampling and plain sampling in one
place.

Uniforms come from a counter-based Philox4x32-10 stream on the device
(qvex_philox_uniforms): the sampler's seed (SamplingParams.seed, or fresh
entropy when None, as the reference seeds MLX's generator only when given one,
engine/sampler.py:25-26) and one device draw counter, advanced once per draw.
The reference draws from MLX's generator (engine/speculative.py:79-81). Draws
need no host work, so a captured cycle draws the same stream as eager calls,
for any number of cycles. The presence mask lives on the device and is
updated by observe().

API as engine/sampler.py: scores(logits, extra_seen) -> full-vocabulary scores,
pick(scores) -> argmax (greedy) or a categorical draw from the scores. The
decode path uses pick_logits(logits), which applies the same filtering inside
the sampling kernel (no score vector is made).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _C, kernels


@dataclass
class SamplingParams:
    temperature: float = 0.6
    top_p: float = 0.95
    top_k: int = 20
    presence_penalty: float = 0.0
    max_tokens: int = 2048
    seed: int | None = None


class Sampler:
    def __init__(self, params: SamplingParams, vocab_size: int):
        self.p = params
        self.V = vocab_size
        # engine/sampler.py:44-50: top-k when 0 < top_k < V, top-p when 0 < top_p < 1
        tk = params.top_k if 0 < params.top_k < vocab_size else 0
        tp = params.top_p if 0 < params.top_p < 1 else 1.0
        self.top_k = tk if params.temperature > 0 else 0
        self.top_p = tp
        self.seen = None            # device fp32 [V] presence mask, made on first use
        seed = params.seed if params.seed is not None else np.random.SeedSequence().entropy
        self.seed = int(seed) & (2**64 - 1)
        self.u_counter = None       # device uint64 draw counter (int64 storage), made on first use
        self._ws = {}

    @property
    def greedy(self) -> bool:
        return self.p.temperature <= 0

    def _filter(self, device) -> dict:
        if self.p.presence_penalty and self.seen is None:
            if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
                # a mask made inside a capture would be cleared on every replay
                raise _C.QvexError("Sampler: the presence mask must exist before a graph capture "
                                   "(Sampler.prepare_accept)")
            self.seen = torch.zeros(self.V, dtype=torch.float32, device=device)
        return dict(seen=self.seen if self.p.presence_penalty else None,
                    presence_penalty=float(self.p.presence_penalty), top_k=self.top_k, top_p=self.top_p)

    def prepare_accept(self, k: int, device) -> None:
        """Make the device buffers that accept_device() uses for k drafts (the
        presence mask, the workspace, the draw counter) now, zero-filled: inside
        a graph capture their fill would only be recorded (each replay of that
        graph would clear them, and other graphs captured on them would start
        from whatever the memory held)."""
        self._filter(device)
        self._workspace(1, k, False, device)
        self.counter(device)

    def _workspace(self, S, k, has_draft, device, top_k=None):
        tk = self.top_k if top_k is None else top_k
        key = (S, k, has_draft, tk)
        if key not in self._ws:
            self._ws[key] = kernels.spec_workspace(S, k, self.V, has_draft, device, tk)
        return self._ws[key]

    def scores(self, logits: torch.Tensor, extra_seen=None) -> torch.Tensor:
        """Full-vocabulary fp32 scores as engine/sampler.py:30-52 (qvex_sampler_scores):
        penalised logits when greedy, else filtered log-probabilities (-inf outside
        the top-k / top-p set). logits: [V] or [R, V] bf16 / fp32 on the device;
        extra_seen: ids that count as seen for this call only. The decode path
        does the same filtering inside its sampling kernel instead."""
        t = as_logits(logits)
        R = t.numel() // self.V
        seen = None
        if self.p.presence_penalty:
            seen = self._filter(t.device)["seen"]
            if extra_seen is not None:
                seen = seen.clone()
                ids = torch.as_tensor(extra_seen, device=t.device).reshape(-1).to(torch.int32)
                _C.call("qvex_mark_seen", seen.data_ptr(), self.V, ids.data_ptr(), ids.numel(), None, ids.numel(),
                        kernels._stream())
        key = ("scores", R)
        if key not in self._ws:
            n = int(_C.lib().qvex_sampler_scores_workspace_bytes(R, self.V, self.top_k))
            self._ws[key] = torch.empty((max(n, 4) + 3) // 4, dtype=torch.float32, device=t.device)
        ws = self._ws[key]
        out = torch.empty(t.shape, dtype=torch.float32, device=t.device)
        inv = float(np.float32(1.0) / np.float32(self.p.temperature)) if not self.greedy else 0.0
        _C.call("qvex_sampler_scores", t.data_ptr(), int(t.dtype == torch.bfloat16), R, self.V,
                seen.data_ptr() if seen is not None else None, float(self.p.presence_penalty), inv, self.top_k,
                float(self.top_p), out.data_ptr(), ws.data_ptr(), ws.numel() * 4, kernels._stream())
        return out

    def counter(self, device) -> torch.Tensor:
        """The device draw counter (one uint64 in an int64 tensor)."""
        if self.u_counter is None:
            if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
                # a counter made inside a capture would restart on every replay
                raise _C.QvexError("Sampler: the draw counter must exist before a graph capture")
            self.u_counter = torch.zeros(1, dtype=torch.int64, device=device)
        return self.u_counter

    def draw_into(self, out: torch.Tensor) -> torch.Tensor:
        """One draw event: out (device fp32, 1..256 values) = the next uniforms."""
        if out.dtype != torch.float32 or not out.is_contiguous() or not 1 <= out.numel() <= 256:
            raise _C.QvexError("draw_into: out must be a contiguous fp32 tensor of 1..256 values")
        _C.call("qvex_philox_uniforms", self.seed, self.counter(out.device).data_ptr(), out.numel(),
                out.data_ptr(), kernels._stream())
        return out

    def _uniforms(self, n: int, device) -> torch.Tensor:
        u = torch.empty(n, dtype=torch.float32, device=device)
        for i in range(0, n, 256):
            self.draw_into(u[i:i + 256])
        return u

    def accept(self, target: torch.Tensor, draft_ids: torch.Tensor, draft_logits: torch.Tensor | None = None):
        """target [k+1, V] logits of the verify rows, draft_ids [k] -> device int32
        (n_accept [1], token [1]); token is the residual sample at the first
        rejection or the bonus sample from row k."""
        t = to_f32(target).reshape(1, -1, self.V)
        k = t.shape[1] - 1
        d = None if draft_logits is None else to_f32(draft_logits).reshape(1, k, self.V)
        u = self._uniforms(k + 1, t.device)
        return kernels.spec_accept(t, d, draft_ids.reshape(1, k).to(torch.int32), u[:k].reshape(1, k).contiguous(),
                                   u[k:].contiguous(), self.p.temperature,
                                   workspace=self._workspace(1, k, d is not None, t.device), **self._filter(t.device))

    def accept_device(self, target: torch.Tensor, draft_ids: torch.Tensor, u: torch.Tensor,
                      tile_max: torch.Tensor | None = None):
        """accept() with the k + 1 uniforms given as a device fp32 [k+1] tensor
        (no host RNG, so the call can be captured in a graph). bf16 logits are
        read in place. tile_max: the rows' 16-column tile maxima (the lm_head's
        epilogue, Qwen35(..., tile_max_out=...)), which lets the filtered accept
        run as one kernel over the few tiles that hold the top-k (same results)."""
        t = as_logits(target).reshape(1, -1, self.V)
        k = t.shape[1] - 1
        use_tm = tile_max is not None and t.dtype == torch.bfloat16
        return kernels.spec_accept(t, None, draft_ids.reshape(1, k), u[:k].reshape(1, k), u[k:],
                                   self.p.temperature, workspace=self._workspace(1, k, False, t.device),
                                   tile_max=tile_max if use_tm else None, **self._filter(t.device))

    def accept_rows_device(self, target: torch.Tensor, draft_ids: torch.Tensor, u: torch.Tensor,
                           tile_max: torch.Tensor, rows: torch.Tensor | None = None):
        """accept_device() without the step decision, when its one-kernel form
        applies (bf16 logits, top-k 1..64, no penalty): each of the k + 1 rows
        leaves (accept flag, draw) in rows [k+1, 2] for the decode cycle's
        finishing kernel to decide; returns rows, or None when the form does not
        apply (then use accept_device)."""
        t = as_logits(target).reshape(1, -1, self.V)
        k = t.shape[1] - 1
        f = self._filter(t.device)
        if t.dtype != torch.bfloat16 or not kernels.tiles_rows_apply(1, k, self.V, self.p.temperature,
                                                                     f["top_k"], f["presence_penalty"]):
            return None
        return kernels.spec_accept_rows(t, draft_ids.reshape(1, k), u[:k].reshape(1, k), u[k:],
                                        self.p.temperature, tile_max, rows=rows,
                                        workspace=self._workspace(1, k, False, t.device), **f)

    def pick(self, scores: torch.Tensor) -> torch.Tensor:
        """One token per row of scores [R, V] as made by scores() (engine/sampler.py:
        57-58): argmax when greedy, else a categorical draw with probabilities
        proportional to exp(scores) -> int32 [R] on the device."""
        t = to_f32(scores).reshape(-1, 1, self.V)
        R = t.shape[0]
        empty_i = torch.empty((R, 0), dtype=torch.int32, device=t.device)
        empty_f = torch.empty((R, 0), dtype=torch.float32, device=t.device)
        _, tok = kernels.spec_accept(t, None, empty_i, empty_f, self._uniforms(R, t.device),
                                     0.0 if self.greedy else 1.0, workspace=self._workspace(R, 0, False, t.device,
                                                                                            top_k=0))
        return tok

    def pick_logits(self, logits: torch.Tensor) -> torch.Tensor:
        """pick(scores(logits)) in one kernel pass: one token per row of logits
        [R, V] (penalty, temperature and filters applied inside) -> int32 [R]."""
        t = as_logits(logits).reshape(-1, 1, self.V)
        R = t.shape[0]
        empty_i = torch.empty((R, 0), dtype=torch.int32, device=t.device)
        empty_f = torch.empty((R, 0), dtype=torch.float32, device=t.device)
        _, tok = kernels.spec_accept(t, None, empty_i, empty_f, self._uniforms(R, t.device), self.p.temperature,
                                     workspace=self._workspace(R, 0, False, t.device), **self._filter(t.device))
        return tok

    def observe(self, tok) -> None:
        """Mark emitted tokens as seen (engine/sampler.py:60-62): an int, a list of
        ints or a device int32 tensor."""
        if not self.p.presence_penalty:
            return
        if isinstance(tok, torch.Tensor):
            ids = tok.reshape(-1).to(torch.int32)
            dev = ids.device
        else:
            vals = [int(tok)] if not isinstance(tok, (list, tuple)) else [int(v) for v in tok]
            dev = self.seen.device if self.seen is not None else torch.device("cuda")
            ids = torch.tensor(vals, dtype=torch.int32, device=dev)
        seen = self._filter(dev)["seen"]
        _C.call("qvex_mark_seen", seen.data_ptr(), self.V, ids.data_ptr(), ids.numel(), None, ids.numel(),
                kernels._stream())

    def observe_result(self, result: torch.Tensor) -> None:
        """observe() for a device cycle result [n, token, d_0, ...]: the token and the
        n accepted drafts (graph-capturable)."""
        if not self.p.presence_penalty:
            return
        seen = self._filter(result.device)["seen"]
        _C.call("qvex_mark_seen", seen.data_ptr(), self.V, result[1:].data_ptr(), result.numel() - 1,
                result.data_ptr(), 1, kernels._stream())


def as_logits(x: torch.Tensor) -> torch.Tensor:
    """Logits as the accept kernels take them: bf16 or fp32 as they are (contiguous)."""
    if x.dtype in (torch.bfloat16, torch.float32):
        return x.contiguous()
    raise _C.QvexError(f"logits must be bf16 or fp32 (got {x.dtype})")


def to_f32(x: torch.Tensor) -> torch.Tensor:
    """fp32 copy of a bf16 device tensor (qvex_bf16_to_f32); fp32 passes through."""
    if x.dtype == torch.float32:
        return x.contiguous()
    if x.dtype != torch.bfloat16:
        raise _C.QvexError(f"logits must be bf16 or fp32 (got {x.dtype})")
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    _C.call("qvex_bf16_to_f32", x.data_ptr(), out.data_ptr(), x.numel(), kernels._stream())
    return out
