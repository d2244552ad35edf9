"""Token sampling on the device (mirror of engine/sampler.py).

The fused kernel (qvex_spec_accept) does temperature softmax, the speculative
accept test, residual resampling and plain sampling in one place. The reference's
top-k / top-p candidate filtering and presence penalty (engine/sampler.py:30-55)
are not implemented by it: a Sampler refuses parameters that would need them.
Uniforms come from a host PCG64 stream seeded by SamplingParams.seed (the
reference draws them from MLX's generator, engine/speculative.py:79-80), so a
run is reproducible given the seed.
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
        if 0 < params.top_k < vocab_size or 0 < params.top_p < 1 or params.presence_penalty:
            raise NotImplementedError(
                "the fused sampler implements temperature sampling only: use top_k=0, top_p=1.0, "
                "presence_penalty=0 (got top_k=%d top_p=%g presence_penalty=%g)"
                % (params.top_k, params.top_p, params.presence_penalty))
        self.rng = np.random.Generator(np.random.PCG64(params.seed if params.seed is not None else 0))
        self._ws = {}

    @property
    def greedy(self) -> bool:
        return self.p.temperature <= 0

    def scores(self, logits: torch.Tensor, extra_seen=None) -> torch.Tensor:
        """Full-vocab fp32 scores: raw logits (greedy) or logits / temperature."""
        z = to_f32(logits.reshape(-1))
        return z if self.greedy else z / self.p.temperature

    def _uniforms(self, n: int, device) -> torch.Tensor:
        return torch.from_numpy(self.rng.random(n, dtype=np.float32)).to(device)

    def accept(self, target: torch.Tensor, draft_ids: torch.Tensor, draft_logits: torch.Tensor | None = None):
        """target [k+1, V] logits of the verify rows, draft_ids [k] -> device int32
        (n_accept [1], token [1]); token is the residual sample at the first
        rejection or the bonus sample from row k."""
        t = to_f32(target).reshape(1, -1, self.V)
        k = t.shape[1] - 1
        d = None if draft_logits is None else to_f32(draft_logits).reshape(1, k, self.V)
        u = self._uniforms(k + 1, t.device)
        key = (k, d is not None)
        if key not in self._ws:
            self._ws[key] = kernels.spec_workspace(1, k, self.V, d is not None, t.device)
        return kernels.spec_accept(t, d, draft_ids.reshape(1, k).to(torch.int32), u[:k].reshape(1, k).contiguous(),
                                   u[k:].contiguous(), self.p.temperature, workspace=self._ws[key])

    def accept_device(self, target: torch.Tensor, draft_ids: torch.Tensor, u: torch.Tensor):
        """accept() with the k + 1 uniforms given as a device fp32 [k+1] tensor
        (no host RNG, so the call can be captured in a graph)."""
        t = to_f32(target).reshape(1, -1, self.V)
        k = t.shape[1] - 1
        key = (k, False)
        if key not in self._ws:
            self._ws[key] = kernels.spec_workspace(1, k, self.V, False, t.device)
        return kernels.spec_accept(t, None, draft_ids.reshape(1, k), u[:k].reshape(1, k), u[k:],
                                   self.p.temperature, workspace=self._ws[key])

    def pick(self, logits: torch.Tensor) -> torch.Tensor:
        """One token per row of logits [R, V] (argmax when greedy) -> int32 [R]."""
        t = to_f32(logits).reshape(-1, 1, self.V)
        R = t.shape[0]
        empty_i = torch.empty((R, 0), dtype=torch.int32, device=t.device)
        empty_f = torch.empty((R, 0), dtype=torch.float32, device=t.device)
        _, tok = kernels.spec_accept(t, None, empty_i, empty_f, self._uniforms(R, t.device),
                                     self.p.temperature)
        return tok

    def observe(self, tok):
        """Presence tracking is not needed without a presence penalty."""
        return None


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
