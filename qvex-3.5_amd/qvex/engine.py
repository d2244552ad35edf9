"""The caller above the decode generator (engine/engine.py:105-118, 280-366):
prefill, the MTP policy, forced tokens, stop ids, max_tokens and the run's
stats, for token ids in and token ids out.

What the reference's Engine adds beyond this - the worker thread and job queue,
tokenizer and chat template, reasoning budget (which feeds `forced`), thermal
governor, power telemetry and the HTTP layer - is outside the decode path and
not reproduced. Without a thermal governor the "auto" MTP mode is "on": the
reference's auto policy only turns MTP off under a tok/s cap or near the die's
thermal target (engine/engine.py:112-118).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from . import _C
from .model import Qwen35
from .mtp import MTPHead
from .sampler import Sampler, SamplingParams
from .speculative import decode, mtp_prefill

MTP_MODES = ("off", "on", "auto")


@dataclass
class GenerateResult:
    tokens: list[int]              # emitted ids, the stop token excluded
    finish_reason: str             # "stop" or "length"
    stats: dict = field(default_factory=dict)


def mtp_policy(mode: str, mtp: MTPHead | None):
    """use_mtp callable of a mode (engine/engine.py:105-118)."""
    if mode not in MTP_MODES:
        raise ValueError(f"unknown MTP mode {mode!r}")
    if mode != "off" and mode != "auto" and mtp is None:
        raise ValueError("MTP head not loaded")
    on = mode != "off" and mtp is not None
    return lambda: on


def prefill(model: Qwen35, ids, cache, mtp: MTPHead | None = None, mtp_cache=None, last_hidden=None,
            chunk: int | None = None):
    """Run a prompt through the model in chunks (engine/engine.py:232-248) and,
    with an MTP cache, hand each chunk's (hidden, next token) pairs to the MTP
    head as it goes (mtp_prefill with the previous chunk's last hidden), so the
    head's attention workspace stays at one chunk's size. ids: [1, L] or [L].
    Returns (logits of the last token [1, 1, V], last hidden [1, 1, H] or the
    given last_hidden without an MTP cache)."""
    ids = torch.as_tensor(ids, dtype=torch.int32).reshape(1, -1).to(model.norm.device)
    step = chunk or model.prefill_chunk
    logits = None
    for i in range(0, ids.shape[1], step):
        part = ids[:, i:i + step]
        if mtp_cache is not None:
            logits, hidden = model(part, cache, return_hidden=True)
            last_hidden = mtp_prefill(mtp, mtp_cache, hidden, part, last_hidden)
        else:
            logits = model(part, cache)
    return logits, last_hidden


def generate(model: Qwen35, prompt_ids, params: SamplingParams, mtp: MTPHead | None = None,
             mtp_mode: str = "auto", k: int = 3, stop_ids=(), forced: list[int] | None = None,
             max_tokens: int | None = None) -> GenerateResult:
    """Prefill the prompt (the model runs it in 512-token chunks), hand the last
    hidden states to the MTP head, then draw tokens through decode() (MTP
    cycles replayed from a captured HIP graph) until a stop id or max_tokens
    (engine/engine.py:280-300). `forced` is shared with the
    generator: ids appended to it while iterating are emitted next, as the
    reference's reasoning budget does. A stop id counts in completion_tokens but
    is not returned. Stats keys follow the reference's (engine/engine.py:340-357)
    where they apply to this path."""
    use_mtp = mtp_policy(mtp_mode, mtp)
    ids = torch.as_tensor(prompt_ids, dtype=torch.int32).reshape(1, -1).to(model.norm.device)
    if ids.shape[1] < 1:
        raise _C.QvexError("generate: empty prompt")
    limit = params.max_tokens if max_tokens is None else max_tokens
    forced = forced if forced is not None else []
    stop = set(int(t) for t in stop_ids)

    t_start = time.perf_counter()
    # room for the prompt, every emitted token and the draft/verify tokens past
    # the last one: the caches grow when they must (engine/model.py:156-170),
    # but sized up front the captured cycle is never captured again for room
    need = ids.shape[1] + limit + 2 * k + 2
    cap = max(model.max_context, need)
    cache = model.make_cache(max_context=cap)
    mcache = mtp.make_cache(max_context=cap) if mtp is not None else None
    logits, last_h = prefill(model, ids, cache, mtp, mcache)
    sampler = Sampler(params, model.cfg.vocab_size)
    spec: dict = {}
    tokens = decode(model, sampler, cache, logits[0, -1], last_h, mtp, mcache, use_mtp, spec, forced, k)

    out: list[int] = []
    n, finish = 0, "length"
    t_first = None
    for t in tokens:
        if t_first is None:
            t_first = time.perf_counter()
        n += 1
        if t in stop:
            finish = "stop"
            break
        out.append(int(t))
        if n >= limit:
            break
    tokens.close()
    torch.cuda.synchronize()
    t_end = time.perf_counter()
    t_first = t_first if t_first is not None else t_end
    decode_s = t_end - t_first
    stats = {
        "prompt_tokens": int(ids.shape[1]),
        "cached_tokens": 0,
        "completion_tokens": n,
        "ttft_s": t_first - t_start,
        "prefill_tps": ids.shape[1] / (t_first - t_start) if t_first > t_start else None,
        "decode_tps": n / decode_s if decode_s > 0 else None,
        "mtp_cycles": spec.get("cycles", 0),
        "mtp_accepted": spec.get("accepted", 0),
        "mtp_graph_cycles": spec.get("graph_cycles", 0),
    }
    return GenerateResult(out, finish, stats)
