"""Decoding loop with speculative steps from the model's own MTP head
(mirror of engine/speculative.py, generalised from 1 to k drafted tokens).

An MTP cycle drafts k tokens with the MTP head (greedy, chained on its own
hidden state), verifies [feed, d_0 .. d_{k-1}] in one (k+1)-token pass of the
main model, and emits n accepted drafts plus one sampled token (residual at the
first rejection, bonus after k acceptances). Acceptance is the standard rule
with a one-hot draft distribution, so the output follows the main model:
accept d_i with probability p_i(d_i). Caches keep n + 1 of the k + 1 verify
tokens: rollback(k - n) on every cache (a counter change here, any n).
There is one host synchronisation per cycle (reading n and the token).
"""

from __future__ import annotations

from typing import Callable

import torch

from .model import Qwen35
from .mtp import MTPHead
from .sampler import Sampler

MAX_PENDING = 1024


def mtp_prefill(mtp: MTPHead, mtp_cache, hidden, ids, prev_hidden):
    """Feed the MTP head the (h_i, tok_{i+1}) pairs of a prefill chunk
    (engine/speculative.py:26-41). Returns the chunk's last hidden."""
    if prev_hidden is not None:
        h_in = torch.cat([prev_hidden, hidden[:, :-1]], dim=1)
        next_ids = ids
    else:
        h_in, next_ids = hidden[:, :-1], ids[:, 1:]
    if next_ids.shape[1] > 0:
        mtp(h_in, next_ids, mtp_cache)
    return hidden[:, -1:]


def draft_tokens(mtp: MTPHead, mtp_cache, h_in, id_in, k: int):
    """k greedy drafts, chained: step 0 consumes the pending confirmed pairs,
    step j > 0 consumes (its own block output, draft j-1). The k - 1 speculative
    MTP cache entries are rolled back afterwards. Returns int32 [k] on the device."""
    drafts = []
    h, ids = h_in, id_in
    for j in range(k):
        logits, hid = mtp(h, ids, mtp_cache, last_only=True, return_hidden=True)
        d = _argmax(logits[0, -1])
        drafts.append(d)
        h, ids = hid[:, -1:], d.reshape(1, 1)
    if k > 1:
        mtp_cache.rollback(k - 1)
    return torch.cat(drafts)


def _argmax(logits_row):
    from .sampler import to_f32
    from . import kernels
    t = to_f32(logits_row).reshape(1, 1, -1)
    e_i = torch.empty((1, 0), dtype=torch.int32, device=t.device)
    e_f = torch.empty((1, 0), dtype=torch.float32, device=t.device)
    _, tok = kernels.spec_accept(t, None, e_i, e_f, torch.zeros(1, dtype=torch.float32, device=t.device), 0.0)
    return tok


class MTPDecoder:
    """One object per generation: holds the pending (hidden, token) pairs and
    runs whole MTP cycles (draft k, verify k + 1, accept, rollback) or plain
    steps. decode() wraps it in the reference's generator API; benchmarks call
    cycle() directly."""

    def __init__(self, model: Qwen35, sampler: Sampler, cache, first_logits, last_hidden=None,
                 mtp: MTPHead | None = None, mtp_cache=None, k: int = 1, stats: dict | None = None):
        self.model, self.sampler, self.cache = model, sampler, cache
        self.mtp, self.mtp_cache, self.k = mtp, mtp_cache, k
        self.stats = stats if stats is not None else {}
        for key in ("cycles", "accepted", "plain", "emitted"):
            self.stats.setdefault(key, 0)
        self.feed = sampler.pick(first_logits.reshape(1, -1))        # int32 [1] on the device
        self.pend_h = [last_hidden] if mtp is not None else []
        self.pend_ids = [self.feed.reshape(1, 1)] if mtp is not None else []
        self.first = int(self.feed.item())
        self.stats["emitted"] += 1

    def can_speculate(self) -> bool:
        return self.mtp is not None and bool(self.pend_h)

    def cycle(self) -> list[int]:
        """One MTP cycle; returns the emitted tokens (n accepted drafts + 1)."""
        k, model, sampler, cache = self.k, self.model, self.sampler, self.cache
        h_in = self.pend_h[0] if len(self.pend_h) == 1 else torch.cat(self.pend_h, dim=1)
        id_in = self.pend_ids[0] if len(self.pend_ids) == 1 else torch.cat(self.pend_ids, dim=1)
        drafts = draft_tokens(self.mtp, self.mtp_cache, h_in, id_in, k)
        ids = torch.cat([self.feed.reshape(1), drafts]).reshape(1, k + 1)
        logits, hidden = model(ids, cache, last_only=False, return_hidden=True, keep_prev=True)
        n_t, tok_t = sampler.accept(logits[0], drafts)
        vals = torch.cat([n_t, tok_t, drafts]).tolist()                 # the one host sync
        n, tok = int(vals[0]), int(vals[1])
        self.stats["cycles"] += 1
        self.stats["accepted"] += n
        if n < k:
            for c in cache:
                c.rollback(k - n)
        emitted = [int(t) for t in vals[2:2 + n]] + [tok]
        tok_dev = tok_t.reshape(1, 1)
        self.pend_h = [hidden[:, : n + 1]]
        self.pend_ids = [torch.cat([drafts[:n].reshape(1, n), tok_dev], dim=1) if n else tok_dev]
        self.feed = tok_t
        self.stats["emitted"] += len(emitted)
        return emitted

    def plain(self, forced_token: int | None = None) -> int:
        """One non-speculative step (engine/speculative.py:103-118)."""
        model, dev = self.model, self.model.norm.device
        if self.mtp is not None:
            logits, hidden = model(self.feed.reshape(1, 1), self.cache, return_hidden=True)
        else:
            logits, hidden = model(self.feed.reshape(1, 1), self.cache), None
        if forced_token is not None:
            t = torch.tensor([forced_token], dtype=torch.int32, device=dev)
        else:
            t = self.sampler.pick(logits[0, -1:])
        self.stats["plain"] += 1
        if self.mtp is not None:
            self.pend_h.append(hidden)
            self.pend_ids.append(t.reshape(1, 1))
            if len(self.pend_h) > MAX_PENDING:
                self.pend_h, self.pend_ids = self.pend_h[-MAX_PENDING:], self.pend_ids[-MAX_PENDING:]
        self.feed = t
        self.stats["emitted"] += 1
        return int(t.item())


def decode(model: Qwen35, sampler: Sampler, cache, first_logits, last_hidden=None,
           mtp: MTPHead | None = None, mtp_cache=None,
           use_mtp: Callable[[], bool] = lambda: True, stats: dict | None = None,
           forced: list[int] | None = None, k: int = 1):
    """Generator of token ids (engine/speculative.py:44-118). stats gets 'cycles',
    'accepted' (accepted drafts), 'plain' and 'emitted'. forced: tokens emitted
    next, in order, instead of sampled ones (plain steps only)."""
    forced = forced if forced is not None else []
    dec = MTPDecoder(model, sampler, cache, first_logits, last_hidden, mtp, mtp_cache, k, stats)
    yield dec.first
    while True:
        if dec.can_speculate() and not forced and use_mtp():
            for t in dec.cycle():
                yield t
        else:
            yield dec.plain(forced.pop(0) if forced else None)
