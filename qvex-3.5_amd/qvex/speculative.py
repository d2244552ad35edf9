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

import time
from typing import Callable

import torch

from . import _C
from .kernels import _ptr, _stream
from .model import Qwen35, rope_table
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


_ZERO_U = {}


def _argmax(logits_row, out=None):
    """Greedy token of one logits row (first index of the maximum) -> int32 [1]
    on the device, written into `out` (an int32 [1] view) when given."""
    from .sampler import as_logits
    from . import kernels
    t = as_logits(logits_row).reshape(1, 1, -1)
    dev = t.device
    if dev not in _ZERO_U:
        _ZERO_U[dev] = torch.zeros(1, dtype=torch.float32, device=dev)
    e_i = torch.empty((1, 0), dtype=torch.int32, device=dev)
    e_f = torch.empty((1, 0), dtype=torch.float32, device=dev)
    _, tok = kernels.spec_accept(t, None, e_i, e_f, _ZERO_U[dev], 0.0, out_token=out)
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
        self.feed = sampler.pick_logits(first_logits.reshape(1, -1))  # int32 [1] on the device
        sampler.observe(self.feed)
        self.pend_h = [last_hidden] if mtp is not None else []
        self.pend_ids = [self.feed.reshape(1, 1)] if mtp is not None else []
        self.first = int(self.feed.item())
        self.stats["emitted"] += 1

    def can_speculate(self) -> bool:
        return self.mtp is not None and bool(self.pend_h)

    def pending(self) -> int:
        """(hidden, token) pairs not yet given to the MTP head."""
        return sum(int(h.shape[1]) for h in self.pend_h)

    def _eager(self) -> None:
        if self.cache.counters.graph_mode or (self.mtp_cache is not None and self.mtp_cache.counters.graph_mode):
            raise _C.QvexError("this decoder's caches are driven by a GraphedMTPCycle; call its release() "
                               "before eager steps")

    def cycle(self) -> list[int]:
        """One MTP cycle; returns the emitted tokens (n accepted drafts + 1)."""
        self._eager()
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
        sampler.observe(emitted)
        tok_dev = tok_t.reshape(1, 1)
        self.pend_h = [hidden[:, : n + 1]]
        self.pend_ids = [torch.cat([drafts[:n].reshape(1, n), tok_dev], dim=1) if n else tok_dev]
        self.feed = tok_t
        self.stats["emitted"] += len(emitted)
        return emitted

    def plain(self, forced_token: int | None = None) -> int:
        """One non-speculative step (engine/speculative.py:103-118)."""
        self._eager()
        model, dev = self.model, self.model.norm.device
        if self.mtp is not None:
            logits, hidden = model(self.feed.reshape(1, 1), self.cache, return_hidden=True)
        else:
            logits, hidden = model(self.feed.reshape(1, 1), self.cache), None
        if forced_token is not None:
            t = torch.tensor([forced_token], dtype=torch.int32, device=dev)
        else:
            t = self.sampler.pick_logits(logits[0, -1:])
        self.sampler.observe(t)
        self.stats["plain"] += 1
        if self.mtp is not None:
            self.pend_h.append(hidden)
            self.pend_ids.append(t.reshape(1, 1))
            if len(self.pend_h) > MAX_PENDING:
                self.pend_h, self.pend_ids = self.pend_h[-MAX_PENDING:], self.pend_ids[-MAX_PENDING:]
        self.feed = t
        self.stats["emitted"] += 1
        return int(t.item())


# a captured cycle that runs out of KV room grows the caches by at least this
# many positions (or half their capacity) before it is captured again
GRAPH_GROW_MIN = 2048


def grow_kv(caches, extra: int) -> bool:
    """Grow every KV cache among `caches` to hold `extra` positions past its
    offset (KVCache.grow); returns whether any moved."""
    moved = False
    for c in caches:
        if hasattr(c, "grow"):
            moved |= c.grow(c.offset + extra)
    return moved


def decode(model: Qwen35, sampler: Sampler, cache, first_logits, last_hidden=None,
           mtp: MTPHead | None = None, mtp_cache=None,
           use_mtp: Callable[[], bool] = lambda: True, stats: dict | None = None,
           forced: list[int] | None = None, k: int = 1, graph: bool = True):
    """Generator of token ids (engine/speculative.py:44-118). stats gets 'cycles',
    'accepted' (accepted drafts), 'plain' and 'emitted', plus 'graph_cycles'
    (cycles replayed from the captured graph) and 'captures'. forced: tokens
    emitted next, in order, instead of sampled ones (plain steps only).

    With graph (the default) each MTP cycle is a replay of a GraphedMTPCycle:
    one launch of the captured draft -> verify -> accept -> commit graph and one
    host read of its result, the reference's one synchronisation per cycle
    (engine/speculative.py:82-85). use_mtp() and `forced` are looked at before
    every cycle, as the reference does: a plain or forced step releases the
    graph (the caches go back to eager control), and the next MTP cycle
    captures it again (10-30 ms), after one eager cycle when more than k + 1
    (hidden, token) pairs are pending. When the next cycle would not fit a KV
    cache, the caches grow (by GRAPH_GROW_MIN positions or half their capacity)
    and the cycle is captured on the new buffers. The token stream is the one
    graph=False (every cycle launched op by op from the host) emits."""
    forced = forced if forced is not None else []
    dec = MTPDecoder(model, sampler, cache, first_logits, last_hidden, mtp, mtp_cache, k, stats)
    st = dec.stats
    st.setdefault("graph_cycles", 0)
    st.setdefault("captures", 0)
    yield dec.first
    g = None
    try:
        while True:
            if dec.can_speculate() and not forced and use_mtp():
                if graph:
                    if g is None or g.released:
                        if dec.pending() > k + 1:
                            for t in dec.cycle():
                                yield t
                            continue
                        g = GraphedMTPCycle(dec) if g is None else g.attach()
                        st["captures"] += 1
                    if g.room() < 1:
                        g.release()
                        kv = [c for c in dec.cache if hasattr(c, "grow")] + [dec.mtp_cache]
                        grow_kv(kv, max(GRAPH_GROW_MIN, max(c.capacity for c in kv) // 2))
                        g.attach()
                        st["captures"] += 1
                    emitted = g.cycle()
                    st["graph_cycles"] += 1
                    for t in emitted:
                        yield t
                else:
                    for t in dec.cycle():
                        yield t
            else:
                if g is not None and not g.released:
                    g.release()
                yield dec.plain(forced.pop(0) if forced else None)
    finally:
        if g is not None and not g.released:
            g.release()


class GraphedMTPCycle:
    """The MTP cycle of MTPDecoder.cycle() captured as a HIP graph.

    Everything that changes between cycles is device state: the pending
    (hidden, token) pairs of the MTP head (k + 1 fixed rows, the first n_prev + 1
    valid), the feed token, the cache counters (advanced by captured commit
    kernels) and the sampler's uniform draw counter (Philox, advanced by the
    finishing kernel, so the stream is the eager one for any number of cycles).
    The MTP head's first step always runs k + 1 rows and keeps row n_prev on the
    device; rows past it write KV entries beyond the committed position, which
    later cycles overwrite. One replay = one cycle; the host reads
    [n, token, drafts] once and updates its counter mirrors.

    While the object drives the decoder's caches their device counters are
    authoritative: eager model calls, rollbacks and MTPDecoder steps on them
    raise until release() hands the state back; attach() takes it again (and
    captures the cycle again). A cycle that could write past a KV cache's
    capacity raises before it is launched (room() tells how many fit).
    """

    def __init__(self, dec: MTPDecoder):
        if dec.mtp is None or not dec.pend_h:
            raise _C.QvexError("GraphedMTPCycle needs an MTPDecoder with an MTP head and pending pairs")
        self.dec = dec
        model, k = dec.model, dec.k
        self.k = k
        dev = model.norm.device
        H = model.cfg.hidden_size
        self.pend_h = torch.zeros((1, k + 1, H), dtype=torch.bfloat16, device=dev)
        self.pend_ids = torch.zeros((1, k + 1), dtype=torch.int32, device=dev)
        self.n_prev = torch.zeros(1, dtype=torch.int32, device=dev)
        self.n_prev_host = 0
        self.feed = torch.zeros(1, dtype=torch.int32, device=dev)
        # verify input [feed, d_0 .. d_{k-1}]: the drafts are written in place and
        # the finishing kernel stores the next feed in slot 0
        self.ids = torch.zeros((1, k + 1), dtype=torch.int32, device=dev)
        self.drafts = self.ids[0, 1:]
        # the cycle's result [n, token, drafts] and its done flag, in pinned host
        # memory: the finishing kernel writes both, the host polls the flag
        self.out = torch.zeros(2 + k, dtype=torch.int32, pin_memory=True)
        self.done = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._out_np, self._done_np = self.out.numpy(), self.done.numpy()
        self.zero = torch.zeros(1, dtype=torch.int32, device=dev)
        self.u_buf = torch.empty(k + 1, dtype=torch.float32, device=dev)
        # the verify logits' 16-column tile maxima, written by the lm_head's epilogue
        # for the sampler's one-kernel list form
        self.tile_max = torch.empty((k + 1, (model.cfg.vocab_size + 15) // 16), dtype=torch.bfloat16, device=dev)
        # the verify rows' (accept flag, draw) when the sampler's one-kernel form
        # applies: the finishing kernel decides the step from them
        self.rows = torch.zeros((k + 1, 2), dtype=torch.int32, device=dev)
        self._kv = [c for c in dec.cache if hasattr(c, "capacity")]
        self._rec = [c for c in dec.cache if hasattr(c, "last_width")]
        self.released = True
        self.graph = None
        self._pipe = None
        self.attach()

    def attach(self) -> "GraphedMTPCycle":
        """Take the decoder's state (pending pairs, feed, counters) into the device
        buffers and capture the cycle on the caches' current buffers. Called by
        the constructor, and again after release() and eager steps (plain steps,
        forced tokens, an eager cycle, a grown KV cache): the capture is made
        again each time, since a grown cache has moved and attention's key
        bound depends on the position at capture. Needs at most k + 1 pending
        pairs (run one eager cycle first when there are more)."""
        if not self.released:
            return self
        d, k = self.dec, self.k
        if not d.pend_h:
            raise _C.QvexError("GraphedMTPCycle needs pending (hidden, token) pairs")
        h_in = d.pend_h[0] if len(d.pend_h) == 1 else torch.cat(d.pend_h, dim=1)
        id_in = d.pend_ids[0] if len(d.pend_ids) == 1 else torch.cat(d.pend_ids, dim=1)
        P = h_in.shape[1]
        if P > k + 1:
            raise _C.QvexError(f"{P} pending pairs exceed the captured width k + 1 = {k + 1}")
        self.pend_h.zero_()
        self.pend_h[:, :P] = h_in
        self.pend_ids.zero_()
        self.pend_ids[:, :P] = id_in.to(torch.int32)
        self.n_prev.fill_(P - 1)
        self.n_prev_host = P - 1
        self.feed.copy_(d.feed.to(torch.int32).reshape(1))
        self.ids[:, :1] = self.feed.view(1, 1)
        # the first cycle's uniforms; each replay draws the next cycle's at its end
        d.sampler.draw_into(self.u_buf)
        # the sampler's buffers exist, zero-filled, before any capture: the graphs
        # of run() are captured later on them and replayed without this one
        d.sampler.prepare_accept(k, self.u_buf.device)
        # so does the attention's RoPE table (cos, sin per position), for every cache
        cfg = d.model.cfg
        caps = [c.capacity for c in self._kv] + [getattr(d.mtp_cache, "capacity", 0)]
        rope_table(cfg.rotary_dim, cfg.rope_theta, max(caps), self.u_buf.device)
        # device counters must hold the host values before they become authoritative
        d.cache.counters.sync()
        d.mtp_cache.counters.sync()
        torch.cuda.synchronize()
        d.cache.counters.graph_mode = True
        d.mtp_cache.counters.graph_mode = True
        self.released = False
        old = self.graph
        self.graph = self._capture(self.out, pool=None if old is None else old.pool(), done=self.done)
        self._pipe = None
        return self

    def _capture(self, out, pool=None, done=None) -> torch.cuda.CUDAGraph:
        """Capture one cycle writing its result to `out` (and 1 to `done` once
        `out` is visible to the host, when given); the host mirrors the capture
        advances are put back (capture runs no kernels)."""
        d = self.dec
        host_main = d.cache.counters.host.copy()
        host_mtp = d.mtp_cache.counters.host.copy()
        widths = [getattr(c, "last_width", None) for c in d.cache]
        g = torch.cuda.CUDAGraph()
        d.cache.counters.capturing = d.mtp_cache.counters.capturing = True
        try:
            with torch.cuda.graph(g, pool=pool):
                self._body(out, done)
        finally:
            d.cache.counters.capturing = d.mtp_cache.counters.capturing = False
        d.cache.counters.host[:] = host_main
        d.mtp_cache.counters.host[:] = host_mtp
        for c, w in zip(d.cache, widths):
            if w is not None:
                c.last_width = w
        return g

    def _commit(self, counters, n_ptr, extra):
        _C.call("qvex_commit_step", counters.dev.data_ptr(), counters.dev.numel(), _ptr(n_ptr), int(extra), _stream())

    def _body(self, out, done=None):
        d = self.dec
        k, mtp, mc = self.k, d.mtp, d.mtp_cache
        if d.model._deferred_argmax() and mtp.all_packed():
            # Each draft's argmax is reduced inside the next launch (the next
            # step's input, or the verify's embedding), which also stores it into
            # the verify ids; a step's counter advance rides on the next step's
            # input launch. Step 1 takes the k + 1 pending pairs: its lm_head runs
            # on all of them and row n_prev (the hidden of the next step too) is
            # picked on the device.
            am, h = mtp(self.pend_h, self.pend_ids, mc, last_only=False, return_hidden=True, defer_argmax=True)
            sel = self.n_prev
            commit = (mc.counters, self.n_prev, 1)
            for j in range(1, k):
                am, h = mtp(h, None, mc, last_only=True, return_hidden=True, defer_argmax=True,
                            in_argmax=(am, sel, self.ids[0, j:j + 1]), hid_sel=sel, commit=commit)
                sel = None
                commit = (mc.counters, None, 1) if j < k - 1 else None   # the last step's advance folds into the finish
            if commit is not None:               # k = 1: no later draft launch to carry it
                self._commit(mc.counters, self.n_prev, 1)
            logits, _ = d.model(self.ids, d.cache, last_only=False, return_hidden=True, keep_prev=True,
                                hidden_out=self.pend_h, in_argmax=(am, sel, k), tile_max_out=self.tile_max)
        else:
            # greedy drafts straight from the MTP lm_head's argmax epilogue into the verify ids
            _, h = mtp(self.pend_h, self.pend_ids, mc, return_hidden=True, select=self.n_prev,
                       argmax_out=self.ids[0, 1:2])
            self._commit(mc.counters, self.n_prev, 1)
            for j in range(1, k):
                _, h = mtp(h, self.ids[:, j:j + 1], mc, last_only=True, return_hidden=True,
                           argmax_out=self.ids[0, j + 1:j + 2])
                if j < k - 1:                        # the last step's advance folds into the finish
                    self._commit(mc.counters, self.zero, 1)
            logits, _ = d.model(self.ids, d.cache, last_only=False, return_hidden=True, keep_prev=True,
                                hidden_out=self.pend_h, tile_max_out=self.tile_max)
        rows = d.sampler.accept_rows_device(logits[0], self.drafts, self.u_buf, self.tile_max, rows=self.rows)
        if rows is None:
            n, tok = d.sampler.accept_device(logits[0], self.drafts, self.u_buf, tile_max=self.tile_max)
            n_p, tok_p, rows_p = _ptr(n), _ptr(tok), None
        else:
            n_p = tok_p = None
            rows_p = _ptr(rows)
        # verify commit (+n+1 on every main cache), the k - 1 speculative MTP
        # entries rolled back (net -(k-2) after the folded last advance), the
        # next feed and the next cycle's uniforms
        _C.call("qvex_cycle_finish_ex", _ptr(self.drafts), k, n_p, tok_p, _ptr(self.pend_ids),
                _ptr(self.feed), _ptr(self.n_prev), _ptr(out), _ptr(self.ids),
                d.cache.counters.dev.data_ptr(), d.cache.counters.dev.numel(), 1,
                mc.counters.dev.data_ptr(), mc.counters.dev.numel(), -(k - 2) if k > 1 else 0,
                d.sampler.seed, d.sampler.counter(self.u_buf.device).data_ptr(), k + 1, _ptr(self.u_buf),
                None if done is None else done.data_ptr(), rows_p, _stream())
        d.sampler.observe_result(out)

    def room(self) -> int:
        """How many more cycles surely fit every KV cache (none in flight): each
        verify writes k + 1 positions from the main offset and commits at most
        k + 1; the draft steps write k + 1 rows and then k - 1 more from the MTP
        offset (n_prev + 1 + 2k positions past it) and commit n_prev + 1 <= k + 1."""
        if self.released:
            raise _C.QvexError("GraphedMTPCycle was released")
        k, d = self.k, self.dec
        fit = None
        for c in self._kv:
            m = max(0, (c.capacity - c.offset) // (k + 1))
            fit = m if fit is None else min(fit, m)
        mc = d.mtp_cache
        free = mc.capacity - mc.offset
        if free < self.n_prev_host + 1 + 2 * k:
            m = 0
        else:      # the first cycle as above, each later one with n_prev <= k
            m = 1 + max(0, (free - (self.n_prev_host + 1) - (3 * k + 1)) // (k + 1) + 1)
        return m if fit is None else min(fit, m)

    def _check_room(self, n: int = 1) -> None:
        """Raise, before anything is launched, unless n more cycles fit."""
        r = self.room()
        if r < n:
            d = self.dec
            caps = sorted({getattr(c, "capacity", 0) for c in d.cache} - {0})
            raise _C.QvexError(f"KV cache full: {n} more cycle(s) of k + 1 = {self.k + 1} tokens need room, {r} "
                               f"fit (main offset {d.cache[-1].offset}, capacity {caps}; MTP offset "
                               f"{d.mtp_cache.offset}, capacity {d.mtp_cache.capacity}); release() and grow the "
                               "caches, or make them with a larger max_context")

    def cycle(self) -> list[int]:
        """Replay one cycle; returns the emitted tokens (n accepted drafts + 1).

        The one host synchronisation per cycle is a poll of the pinned done flag
        that the cycle's finishing kernel sets after its result: the host sees
        the result as soon as it lands (a device-to-host copy or an event wait
        adds 15-45 us per cycle). The stream keeps running the graph's last
        bookkeeping kernels meanwhile; the next replay is ordered after them."""
        self._check_room()
        flag = self._done_np
        flag[0] = 0
        self.graph.replay()
        spins, t0 = 0, None
        while flag[0] == 0:
            spins += 1
            if spins & 4095 == 0:        # a cycle takes milliseconds: look at the clock now and then
                if t0 is None:
                    t0 = time.perf_counter()
                elif time.perf_counter() - t0 > 10.0:
                    torch.cuda.synchronize()             # raises on a device error
                    if flag[0] == 0:
                        raise _C.QvexError("the replayed cycle finished without setting its done flag")
        return self._account(self._out_np.tolist())

    def run(self, n: int) -> list[list[int]]:
        """n cycles, each launched before the previous one's result is read, so
        the GPU does not wait on the host between cycles. Two graphs alternate;
        each writes its result into its own slot of a pinned host buffer, and the
        host waits on that graph's event rather than on the stream. The next
        cycle only reads device state, so the token stream and the caches are
        those of n cycle() calls, and no cycle is in flight on return. Returns
        each cycle's emitted tokens."""
        if self.released:
            raise _C.QvexError("GraphedMTPCycle was released")
        if self._pipe is None:
            ring = torch.zeros((2, 2 + self.k), dtype=torch.int32, pin_memory=True)
            graphs = [self._capture(ring[s], pool=self.graph.pool()) for s in range(2)]
            self._pipe = (ring, graphs, [torch.cuda.Event(), torch.cuda.Event()])
        ring, graphs, evs = self._pipe
        res = []
        if n <= 0:
            return res
        # room for every cycle is checked before the first launch, so no launched
        # cycle is ever left unaccounted
        self._check_room(n)
        graphs[0].replay()
        evs[0].record()
        for c in range(n):
            s = c % 2
            if c + 1 < n:
                graphs[1 - s].replay()
                evs[1 - s].record()
            evs[s].synchronize()
            res.append(self._account(ring[s].tolist()))
        return res

    def release(self) -> MTPDecoder:
        """Hand the state back to the MTPDecoder (device counters, feed, pending
        pairs) so eager cycle()/plain() steps, model calls and rollbacks work
        again; this object cannot replay until attach(). Returns the decoder."""
        if self.released:
            return self.dec
        torch.cuda.synchronize()
        d = self.dec
        for counters in (d.cache.counters, d.mtp_cache.counters):
            counters.host[:] = counters.dev.cpu().numpy()
            counters.graph_mode = False
            counters.dirty = False
        # the last replay drew the next cycle's uniforms; give that draw back so
        # the next eager draw takes the same event
        d.sampler.counter(self.u_buf.device).sub_(1)
        P = self.n_prev_host + 1
        d.pend_h = [self.pend_h[:, :P].clone()]
        d.pend_ids = [self.pend_ids[:, :P].clone()]
        d.feed = self.feed.clone()
        self.released = True
        return d

    def _account(self, vals) -> list[int]:
        """Host mirrors and stats of one finished cycle from its [n, token, drafts]."""
        n, tok = int(vals[0]), int(vals[1])
        d = self.dec
        d.cache.counters.host += n + 1
        for c in self._rec:
            c.last_width = n + 1              # the verify's k + 1 snapshots, k - n rolled back
        d.mtp_cache.counters.host[d.mtp_cache.index] += self.n_prev_host + 1
        self.n_prev_host = n
        d.cache.counters.dirty = False
        d.mtp_cache.counters.dirty = False
        emitted = [int(t) for t in vals[2:2 + n]] + [tok]
        d.stats["cycles"] += 1
        d.stats["accepted"] += n
        d.stats["emitted"] += len(emitted)
        return emitted
