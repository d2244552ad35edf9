"""End-to-end MTP decode at the Qwen3.5-9B shape (32 layers: 24 DeltaNet + 8
attention, hidden 4096, MLP 12288, vocab 248,320, 4-bit g64; MTP head k = 3)
after a 4096-token seeded prompt, as the benchmark runs it (GPU):

* rollback (tests/rollback_test.py generalised to n = 0..3): verify 4 tokens,
  keep n + 1, feed one more - logits equal the sequential run bit for bit;
* greedy speculative decoding emits plain greedy decoding's tokens
  (tests/mtp_teacher.py), also when every draft is accepted (zeroed lm_head);
* the graph-replayed cycle emits the eager cycle's tokens and leaves the same
  counters, with the benchmark's sampling (T = 0.7, top-k 20, top-p 0.8) and
  with greedy all-accept cycles; release() hands the state back to eager steps.

These are exact (bitwise) properties, so they hold at full size where an
oracle comparison of a 32-layer 4096-token forward would take too long on the
host. The prompt is prefilled once and its caches cloned for each case."""

import numpy as np
import pytest
import torch

from qvex.engine import prefill
from qvex.model import Config, random_model
from qvex.mtp import random_mtp
from qvex.sampler import Sampler, SamplingParams
from qvex.speculative import GraphedMTPCycle, MTPDecoder

DEV = "cuda:0"
PROMPT = 4096


@pytest.fixture(scope="module")
def big():
    cfg = Config.qwen35_9b()
    m = random_model(cfg, seed=1004, device=DEV, max_context=PROMPT + 256)
    mtp = random_mtp(m, seed=2004)
    ids = np.random.default_rng(1004).integers(0, cfg.vocab_size, PROMPT).astype(np.int32)
    cache, mc = m.make_cache(), mtp.make_cache()
    logits, last_h = prefill(m, torch.from_numpy(ids), cache, mtp, mc)
    torch.cuda.synchronize()
    print(f"prefilled {PROMPT} tokens", flush=True)
    yield m, mtp, cache, mc, logits.clone(), last_h.clone()
    del m, mtp, cache, mc
    torch.cuda.empty_cache()


def branch(big):
    m, mtp, cache, mc, logits, last_h = big
    return m, mtp, cache.clone(), mc.clone(), logits, last_h


@pytest.mark.gpu
@pytest.mark.parametrize("n", [0, 1, 2, 3])
def test_rollback_after_long_prompt_equals_prefix_run(big, n):
    m, _, c1, _, _, _ = branch(big)
    _, _, c2, _, _, _ = branch(big)
    g = np.random.default_rng(40 + n)
    ver = torch.from_numpy(g.integers(0, m.cfg.vocab_size, 4).astype(np.int32)).reshape(1, -1)
    e = torch.from_numpy(g.integers(0, m.cfg.vocab_size, 1).astype(np.int32)).reshape(1, -1)
    m(ver, c1, last_only=False, keep_prev=True)
    for c in c1:
        c.rollback(3 - n)
    l1 = m(e, c1)
    for j in range(n + 1):
        m(ver[:, j:j + 1], c2)
    l2 = m(e, c2)
    torch.cuda.synchronize()
    assert torch.equal(l1.view(torch.int16), l2.view(torch.int16))
    assert [c.offset for c in c1] == [c.offset for c in c2] == [PROMPT + n + 2] * 32


def decoder(big, temp, seed=0, **params):
    m, mtp, cache, mc, logits, last_h = branch(big)
    sp = dict(temperature=temp, top_k=0, top_p=1.0, seed=seed)
    sp.update(params)
    return MTPDecoder(m, Sampler(SamplingParams(**sp), m.cfg.vocab_size), cache, logits[0, -1], last_h, mtp, mc,
                      k=3)


@pytest.mark.gpu
def test_greedy_spec_equals_plain(big):
    spec, plain = decoder(big, 0.0), decoder(big, 0.0)
    ts = [spec.first]
    while len(ts) < 16:
        ts += spec.cycle()
    tp = [plain.first] + [plain.plain() for _ in range(15)]
    print("cycles", spec.stats["cycles"], "accepted", spec.stats["accepted"])
    assert ts[:16] == tp


@pytest.mark.gpu
def test_graphed_equals_eager_bench_sampling_and_release(big):
    params = dict(top_k=20, top_p=0.8)
    eager = decoder(big, 0.7, seed=11, **params)
    graphed = GraphedMTPCycle(decoder(big, 0.7, seed=11, **params))
    te, tg = [], []
    for _ in range(6):
        te += eager.cycle()
    for part in graphed.run(6):
        tg += part
    assert te == tg
    assert [c.offset for c in eager.cache] == [c.offset for c in graphed.dec.cache]
    # the captured cycle has drawn the next cycle's uniforms already
    assert int(eager.sampler.u_counter.item()) + 1 == int(graphed.dec.sampler.u_counter.item())
    # back to eager steps on the graphed decoder: the same stream continues
    dec = graphed.release()
    assert int(eager.sampler.u_counter.item()) == int(dec.sampler.u_counter.item())
    for _ in range(3):
        te += eager.cycle()
        tg += dec.cycle()
    te.append(eager.plain())
    tg.append(dec.plain())
    assert te == tg
    dec.cache.counters.sync()                     # eager steps upload host edits lazily
    assert list(dec.cache.counters.dev.cpu().numpy()) == [c.offset for c in eager.cache]


@pytest.mark.gpu
def test_all_accept_cycles_graphed_equal_eager_and_plain(big):
    """Zeroed lm_head: every logit is 0, so drafts and verify argmax are token 0
    and all k drafts are accepted - the k + 1 pending pairs and n = k commits at
    full size."""
    m = big[0]
    s0, b0 = m.lm_head.scales.clone(), m.lm_head.biases.clone()
    try:
        m.lm_head.scales.zero_()
        m.lm_head.biases.zero_()
        m.lm_head.repack()
        eager, plain = decoder(big, 0.0), decoder(big, 0.0)
        graphed = GraphedMTPCycle(decoder(big, 0.0))
        te, tg = [], []
        for _ in range(4):
            te += eager.cycle()
            tg += graphed.cycle()
        tp = [plain.plain() for _ in range(16)]
        assert te == tg == tp == [0] * 16
        assert eager.stats["accepted"] == 12 and graphed.dec.stats["accepted"] == 12
        assert [c.offset for c in eager.cache] == [c.offset for c in graphed.dec.cache] == [PROMPT + 16] * 32
    finally:
        m.lm_head.scales.copy_(s0)
        m.lm_head.biases.copy_(b0)
        m.lm_head.repack()


def decode_gen(big, graph, forced, flag, stats, **params):
    from qvex.speculative import decode
    m, mtp, cache, mc, logits, last_h = branch(big)
    s = Sampler(SamplingParams(**params), m.cfg.vocab_size)
    gen = decode(m, s, cache, logits[0, -1], last_h, mtp, mc, use_mtp=lambda: flag[0], stats=stats, forced=forced,
                 k=3, graph=graph)
    return gen, cache


@pytest.mark.gpu
def test_decode_graph_equals_eager_bench_sampling_forced_and_toggle(big):
    """decode() as the reference's API drives it (engine/speculative.py:44-118,
    bench/mtp_bench.py:49-55), at the 9B shape after the 4096-token prompt, with
    the benchmark's sampling (T = 0.7, top-k 20, top-p 0.8): the captured-graph
    cycles emit the op-by-op cycles' tokens, also across a forced-token
    insertion and the MTP policy turned off and on again while iterating."""
    params = dict(temperature=0.7, top_k=20, top_p=0.8, seed=13)
    streams, stats, caches = [], [], []
    for graph in (True, False):
        forced, flag, st = [], [True], {}
        gen, cache = decode_gen(big, graph, forced, flag, st, **params)
        toks = []
        for t in gen:
            toks.append(t)
            if len(toks) == 6:
                forced.extend([100, 200])
            if len(toks) == 12:
                flag[0] = False
            if len(toks) == 15:
                flag[0] = True
            if len(toks) >= 26:
                break
        gen.close()
        streams.append(toks)
        stats.append(st)
        caches.append(cache)
    print("graph stats", stats[0], "eager stats", stats[1])
    assert streams[0] == streams[1]
    assert streams[0][6:8] == [100, 200]
    for key in ("cycles", "accepted", "plain", "emitted"):
        assert stats[0][key] == stats[1][key], key
    assert stats[0]["graph_cycles"] > 0 and stats[0]["captures"] >= 2 and stats[1]["graph_cycles"] == 0
    assert [c.offset for c in caches[0]] == [c.offset for c in caches[1]]
