"""Verify forward, rollback and MTP decode on a small random-init model (GPU).

Forward parity vs the numpy restatement of engine/model.py (oracle/model.py):
logits within two bf16 steps at the largest |logit| (logit_tol; the bf16
rounding points of the fused kernels differ from the reference's per-op
roundings, and one step is what is measured). Rollback and
speculative-vs-plain checks are bit-exact: every kernel computes a row the
same way whatever the number of rows in the call.
"""

import numpy as np
import pytest
import torch

from oracle.model import OracleModel
from qvex.model import Config, random_model
from qvex.mtp import random_mtp
from qvex.sampler import Sampler, SamplingParams
from qvex.speculative import decode, mtp_prefill

DEV = "cuda:0"


@pytest.fixture(scope="module")
def tiny():
    torch.manual_seed(0)
    cfg = Config.tiny(layers=4, vocab=4096)
    m = random_model(cfg, seed=7, device=DEV, max_context=1024, max_width=8)
    return m


def logit_tol(ref) -> float:
    """Two bf16 steps at the largest |logit| of the compared rows: the logits
    leave every path rounded to bf16, and the errors measured on MI355X are one
    such step (0.0625 at the tiny model's logits, 0.125 at the 9B width)."""
    return 2.0 * 2.0 ** (np.floor(np.log2(np.abs(ref).max())) - 7)


def prompt(n, V, seed=3):
    return np.random.default_rng(seed).integers(0, V, size=n).astype(np.int32)


def f32(t):
    return t.float().cpu().numpy()


@pytest.mark.gpu
def test_prefill_and_verify_match_oracle(tiny):
    V = tiny.cfg.vocab_size
    ids = prompt(13, V)
    cache = tiny.make_cache()
    logits, hidden = tiny(torch.from_numpy(ids).reshape(1, -1), cache, return_hidden=True)
    orc = OracleModel(tiny)
    ol, oh = orc.forward(ids, last_only=True)
    d = np.abs(f32(logits[0]) - ol).max()
    dh = np.abs(f32(hidden[0]) - oh).max() / (np.abs(oh).max() + 1e-6)
    print(f"prefill: max|dlogit|={d:.4f} rel|dhidden|={dh:.4f} argmax {int(f32(logits[0]).argmax())} vs {int(ol.argmax())}")
    assert d <= logit_tol(ol)
    ver = prompt(4, V, seed=5)
    logits4 = tiny(torch.from_numpy(ver).reshape(1, -1), cache, last_only=False)
    ol4, _ = orc.forward(ver, last_only=False)
    d4 = np.abs(f32(logits4[0]) - ol4).max()
    print(f"verify: max|dlogit|={d4:.4f}")
    assert d4 <= logit_tol(ol4)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [0, 1, 2, 3])
def test_rollback_equals_prefix_run(tiny, n):
    """tests/rollback_test.py generalised: verify [a,b,c,d], keep n + 1 tokens,
    then feed e; logits equal the sequential run a..(n tokens), e bit for bit."""
    V = tiny.cfg.vocab_size
    ids = prompt(11, V, seed=21)
    ver = prompt(4, V, seed=22)
    e = prompt(1, V, seed=23)
    c1 = tiny.make_cache()
    tiny(torch.from_numpy(ids).reshape(1, -1), c1)
    tiny(torch.from_numpy(ver).reshape(1, -1), c1, last_only=False, keep_prev=True)
    for c in c1:
        c.rollback(3 - n)
    l1 = tiny(torch.from_numpy(e).reshape(1, -1), c1)
    c2 = tiny.make_cache()
    tiny(torch.from_numpy(ids).reshape(1, -1), c2)
    for t in ver[: n + 1]:
        tiny(torch.tensor([[int(t)]]), c2)
    l2 = tiny(torch.from_numpy(e).reshape(1, -1), c2)
    torch.cuda.synchronize()
    assert torch.equal(l1.view(torch.int16), l2.view(torch.int16))
    assert [c.offset for c in c1] == [c.offset for c in c2]


def run_decode(model, mtp, k, temp, n_tokens, use_mtp=True, seed=0):
    V = model.cfg.vocab_size
    ids = torch.from_numpy(prompt(17, V, seed=31)).reshape(1, -1)
    cache, mc = model.make_cache(), mtp.make_cache()
    logits, hidden = model(ids, cache, return_hidden=True)
    last_h = mtp_prefill(mtp, mc, hidden, ids.to(DEV), None)
    s = Sampler(SamplingParams(temperature=temp, top_k=0, top_p=1.0, seed=seed), V)
    stats, out = {}, []
    for t in decode(model, s, cache, logits[0, -1], last_h, mtp if use_mtp else None, mc, stats=stats, k=k):
        out.append(t)
        if len(out) >= n_tokens:
            break
    return out, stats


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1, 3])
def test_mtp_greedy_equals_plain_greedy(tiny, k):
    """tests/mtp_teacher.py: greedy speculative decoding emits the main model's
    greedy tokens (here exactly, rows being bit-identical)."""
    mtp = random_mtp(tiny, seed=9)
    spec, st = run_decode(tiny, mtp, k, 0.0, 24)
    plain, _ = run_decode(tiny, mtp, k, 0.0, 24, use_mtp=False)
    print("cycles", st["cycles"], "accepted", st["accepted"])
    assert spec == plain


@pytest.mark.gpu
def test_sampled_decode(tiny):
    mtp = random_mtp(tiny, seed=11)
    out, st = run_decode(tiny, mtp, 3, 0.7, 40, seed=5)
    assert len(out) == 40 and all(0 <= t < tiny.cfg.vocab_size for t in out)
    assert st["emitted"] >= 40 and st["cycles"] >= 1


def flat_head_model(seed=12):
    """Tiny model whose shared lm_head is exactly zero: every logit is 0, so both
    the MTP drafts and the verify argmax are token 0 and every draft is accepted."""
    cfg = Config.tiny(layers=4, vocab=2048)
    m = random_model(cfg, seed=seed, device=DEV, max_context=1024)
    m.lm_head.scales.zero_()
    m.lm_head.biases.zero_()
    m.lm_head.repack()
    return m


def start_decoder(model, mtp, k, temp, seed=0, **params):
    from qvex.speculative import MTPDecoder
    V = model.cfg.vocab_size
    ids = torch.from_numpy(prompt(15, V, seed=41)).reshape(1, -1).to(DEV)
    cache, mc = model.make_cache(), mtp.make_cache()
    logits, hidden = model(ids, cache, return_hidden=True)
    last_h = mtp_prefill(mtp, mc, hidden, ids, None)
    sp = dict(temperature=temp, top_k=0, top_p=1.0, seed=seed)
    sp.update(params)
    s = Sampler(SamplingParams(**sp), V)
    return MTPDecoder(model, s, cache, logits[0, -1], last_h, mtp, mc, k=k)


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1, 3])
@pytest.mark.parametrize("head", ["random", "flat"])
def test_graphed_cycle_equals_eager(k, head):
    """The HIP-graph cycle (device-side pending pairs, counters, uniforms) emits
    the eager cycle's tokens (greedy) and leaves the same cache counters, both
    when every draft is rejected (random head) and when every draft is accepted
    (flat head: n = k, k + 1 pending pairs per cycle)."""
    from qvex.speculative import GraphedMTPCycle
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=12, device=DEV, max_context=1024) \
        if head == "random" else flat_head_model()
    mtp = random_mtp(m, seed=13)
    eager = start_decoder(m, mtp, k, 0.0)
    graphed = GraphedMTPCycle(start_decoder(m, mtp, k, 0.0))
    te, tg = [], []
    for _ in range(12):
        te += eager.cycle()
        tg += graphed.cycle()
    print(head, "accepted", eager.stats["accepted"], "of", 12 * k, "graphed", graphed.dec.stats["accepted"])
    assert te == tg
    assert eager.stats["accepted"] == (0 if head == "random" else 12 * k)
    assert [c.offset for c in eager.cache] == [c.offset for c in graphed.dec.cache]
    assert eager.mtp_cache.offset == graphed.dec.mtp_cache.offset
    assert list(graphed.dec.cache.counters.dev.cpu().numpy()) == [c.offset for c in graphed.dec.cache]
    assert int(graphed.dec.mtp_cache.counters.dev.cpu()[0]) + graphed.n_prev_host + 1 == \
        eager.mtp_cache.offset + len(eager.pend_ids[0][0])


@pytest.mark.gpu
def test_graphed_cycle_with_fused_decode_attention():
    """With the fused decode attention switched on (q/k norms, RoPE and the KV
    append inside the split kernel; off by default), the captured cycle needs
    its RoPE table before the capture: attach() makes it, and the graphed
    cycles emit the eager cycles' tokens (sampling, top-k / top-p)."""
    from qvex.model import Attention
    from qvex.speculative import GraphedMTPCycle
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=14, device=DEV, max_context=1024)
    mtp = random_mtp(m, seed=15)
    was = Attention.fused_decode
    Attention.fused_decode = True
    try:
        params = dict(top_k=20, top_p=0.8)
        eager = start_decoder(m, mtp, 3, 0.7, seed=6, **params)
        graphed = GraphedMTPCycle(start_decoder(m, mtp, 3, 0.7, seed=6, **params))
        te, tg = [], []
        for _ in range(8):
            te += eager.cycle()
            tg += graphed.cycle()
        assert te == tg
        assert [c.offset for c in eager.cache] == [c.offset for c in graphed.dec.cache]
    finally:
        Attention.fused_decode = was


@pytest.mark.gpu
@pytest.mark.parametrize("n", [0, 1, 2, 3])
def test_cycle_finish_bookkeeping(n):
    from qvex import _C
    from qvex.kernels import _ptr, _stream
    k = 3
    drafts = torch.tensor([11, 22, 33], dtype=torch.int32, device=DEV)
    n_t = torch.tensor([n], dtype=torch.int32, device=DEV)
    tok = torch.tensor([99], dtype=torch.int32, device=DEV)
    pend = torch.full((k + 1,), -1, dtype=torch.int32, device=DEV)
    feed, nprev = torch.zeros(1, dtype=torch.int32, device=DEV), torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.zeros(k + 2, dtype=torch.int32, device=DEV)
    _C.call("qvex_cycle_finish", _ptr(drafts), k, _ptr(n_t), _ptr(tok), _ptr(pend), _ptr(feed), _ptr(nprev),
            _ptr(out), _stream())
    counters = torch.tensor([5, 7, 9], dtype=torch.int32, device=DEV)
    _C.call("qvex_commit_step", _ptr(counters), 3, _ptr(n_t), 1, _stream())
    torch.cuda.synchronize()
    assert pend.tolist() == [11, 22, 33][:n] + [99] + [0] * (k - n)
    assert feed.item() == 99 and nprev.item() == n
    assert out.tolist() == [n, 99, 11, 22, 33]
    assert counters.tolist() == [5 + n + 1, 7 + n + 1, 9 + n + 1]


@pytest.mark.gpu
def test_graphed_cycle_sampled_runs():
    from qvex.speculative import GraphedMTPCycle
    m = flat_head_model(seed=14)
    mtp = random_mtp(m, seed=15)
    g = GraphedMTPCycle(start_decoder(m, mtp, 3, 0.7, seed=3))
    out = []
    for _ in range(30):
        out += g.cycle()
    assert all(0 <= t < m.cfg.vocab_size for t in out)


@pytest.mark.gpu
@pytest.mark.parametrize("head", ["random", "flat"])
def test_graphed_cycle_equals_eager_reference_sampling(head):
    """The reference's default sampling (T = 0.6, top-k 20, top-p 0.95) plus a presence
    penalty: the graph replays emit the eager cycles' tokens (same uniform stream) and
    leave the same device presence mask."""
    from qvex.speculative import GraphedMTPCycle
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=16, device=DEV, max_context=1024) \
        if head == "random" else flat_head_model(seed=17)
    mtp = random_mtp(m, seed=18)
    params = dict(top_k=20, top_p=0.95, presence_penalty=0.5)
    eager = start_decoder(m, mtp, 3, 0.6, seed=5, **params)
    graphed = GraphedMTPCycle(start_decoder(m, mtp, 3, 0.6, seed=5, **params))
    te, tg = [], []
    for _ in range(10):
        te += eager.cycle()
        tg += graphed.cycle()
    assert te == tg
    assert torch.equal(eager.sampler.seen, graphed.dec.sampler.seen)
    assert int(eager.sampler.seen.sum().item()) == len(set(te + [eager.first]))


@pytest.mark.gpu
@pytest.mark.parametrize("head", ["random", "flat"])
def test_graphed_run_pipelined_equals_cycles(head):
    """run(n) launches each cycle before reading the previous one's result (two
    graphs writing pinned host slots): same tokens, cache counters and presence
    mask as the same number of cycle() calls, also when the two are mixed."""
    from qvex.speculative import GraphedMTPCycle
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=21, device=DEV, max_context=1024) \
        if head == "random" else flat_head_model(seed=22)
    mtp = random_mtp(m, seed=23)
    params = dict(top_k=20, top_p=0.95, presence_penalty=0.5)
    a = GraphedMTPCycle(start_decoder(m, mtp, 3, 0.6, seed=7, **params))
    b = GraphedMTPCycle(start_decoder(m, mtp, 3, 0.6, seed=7, **params))
    ta = []
    for _ in range(13):
        ta += a.cycle()
    tb = []
    for part in b.run(5):
        tb += part
    tb += b.cycle()
    tb += b.cycle()
    assert b.run(0) == []
    for part in b.run(6):
        tb += part
    assert ta == tb
    assert a.dec.stats["cycles"] == b.dec.stats["cycles"] == 13
    assert [c.offset for c in a.dec.cache] == [c.offset for c in b.dec.cache]
    assert a.dec.mtp_cache.offset == b.dec.mtp_cache.offset
    assert torch.equal(a.dec.cache.counters.dev, b.dec.cache.counters.dev)
    assert torch.equal(a.dec.mtp_cache.counters.dev, b.dec.mtp_cache.counters.dev)
    assert torch.equal(a.dec.sampler.seen, b.dec.sampler.seen)


# ---------------------------------------------------------------- generate() (engine/engine.py:105-118, 280-366)

@pytest.mark.gpu
def test_generate_mtp_on_equals_off_greedy_and_stats(tiny):
    """Greedy generation with the MTP policy on emits the tokens of the policy
    off; stats carry the reference's keys, MTP cycles only when on."""
    from qvex.engine import generate
    mtp = random_mtp(tiny, seed=31)
    prompt = np.random.default_rng(31).integers(0, tiny.cfg.vocab_size, 37).tolist()
    p = SamplingParams(temperature=0.0, max_tokens=20)
    on = generate(tiny, prompt, p, mtp, mtp_mode="on", k=3)
    off = generate(tiny, prompt, p, mtp, mtp_mode="off", k=3)
    assert on.tokens == off.tokens and len(on.tokens) == 20
    assert on.finish_reason == off.finish_reason == "length"
    for key in ("prompt_tokens", "cached_tokens", "completion_tokens", "ttft_s", "prefill_tps", "decode_tps",
                "mtp_cycles", "mtp_accepted"):
        assert key in on.stats
    assert on.stats["prompt_tokens"] == 37 and on.stats["completion_tokens"] == 20
    assert on.stats["mtp_cycles"] > 0 and off.stats["mtp_cycles"] == 0
    auto = generate(tiny, prompt, p, None, mtp_mode="auto")       # auto without a head: plain decoding
    assert auto.tokens == off.tokens and auto.stats["mtp_cycles"] == 0


@pytest.mark.gpu
def test_generate_stop_ids_and_forced_tokens(tiny):
    """A stop id ends the run (counted, not returned); forced ids are emitted next
    in order, and ids appended to the list while iterating too."""
    from qvex.engine import generate
    mtp = random_mtp(tiny, seed=37)
    prompt = np.random.default_rng(37).integers(0, tiny.cfg.vocab_size, 20).tolist()
    p = SamplingParams(temperature=0.0, max_tokens=12)
    base = generate(tiny, prompt, p, mtp, mtp_mode="on")
    stop = base.tokens[4]
    first = base.tokens.index(stop)
    r = generate(tiny, prompt, p, mtp, mtp_mode="on", stop_ids=[stop])
    assert r.finish_reason == "stop" and r.tokens == base.tokens[:first]
    assert r.stats["completion_tokens"] == first + 1
    f = generate(tiny, prompt, p, mtp, mtp_mode="on", forced=[11, 12, 13])
    assert f.tokens[0] == base.tokens[0] and f.tokens[1:4] == [11, 12, 13]


@pytest.mark.gpu
def test_generate_policy_errors(tiny):
    from qvex.engine import generate
    p = SamplingParams(temperature=0.0, max_tokens=2)
    with pytest.raises(ValueError):
        generate(tiny, [1, 2, 3], p, None, mtp_mode="on")
    with pytest.raises(ValueError):
        generate(tiny, [1, 2, 3], p, None, mtp_mode="sometimes")


# ---------------------------------------------------------------- decode() on the captured cycle

def decode_pair(model, mtp, k, temp, seed, prompt_len=15, **params):
    """Two decode() generators from one prefilled prompt (separate caches, same
    sampler seed): the captured-graph one and the op-by-op one. Returns
    ((gen, forced, flag, stats), ...) for graph=True and graph=False."""
    from qvex.speculative import decode
    V = model.cfg.vocab_size
    ids = torch.from_numpy(prompt(prompt_len, V, seed=41)).reshape(1, -1).to(DEV)
    out = []
    for graph in (True, False):
        cache, mc = model.make_cache(), mtp.make_cache()
        logits, hidden = model(ids, cache, return_hidden=True)
        last_h = mtp_prefill(mtp, mc, hidden, ids, None)
        sp = dict(temperature=temp, top_k=0, top_p=1.0, seed=seed)
        sp.update(params)
        s = Sampler(SamplingParams(**sp), V)
        forced, flag, stats = [], [True], {}
        gen = decode(model, s, cache, logits[0, -1], last_h, mtp, mc, use_mtp=lambda f=flag: f[0], stats=stats,
                     forced=forced, k=k, graph=graph)
        out.append((gen, forced, flag, stats, cache, mc))
    return out


def drive(gen, forced, flag, n, force_at=None, off_at=None, on_at=None):
    """Consume n tokens; at the given token counts append forced ids (a list)
    or turn the MTP policy off / on, as a caller does between tokens."""
    toks = []
    for t in gen:
        toks.append(t)
        if force_at is not None and len(toks) == force_at[0]:
            forced.extend(force_at[1])
        if off_at is not None and len(toks) == off_at:
            flag[0] = False
        if on_at is not None and len(toks) == on_at:
            flag[0] = True
        if len(toks) >= n:
            break
    gen.close()
    return toks


@pytest.mark.gpu
@pytest.mark.parametrize("head", ["random", "flat"])
def test_decode_graph_equals_eager_across_forced_and_toggle(head):
    """decode() replays the captured cycle (graph=True, the default) and emits
    the op-by-op cycle's tokens (graph=False), also across a forced-token
    insertion and the MTP policy turned off and on again while iterating, with
    the reference's MTP benchmark sampling (T = 0.7, top-k 20, top-p 0.8) plus a
    presence penalty; the graph is released for the plain steps and captured
    again afterwards, and closing the generator hands the caches back."""
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=71, device=DEV, max_context=1024) \
        if head == "random" else flat_head_model(seed=72)
    mtp = random_mtp(m, seed=73)
    params = dict(top_k=20, top_p=0.8, presence_penalty=0.4)
    (ga, fa, la, sa, ca, _), (ge, fe, le, se, ce, _) = decode_pair(m, mtp, 3, 0.7, 9, **params)
    plan = dict(force_at=(7, [5, 6, 7]), off_at=15, on_at=19)
    ta = drive(ga, fa, la, 48, **plan)
    te = drive(ge, fe, le, 48, **plan)
    print(head, "cycles", sa["cycles"], "accepted", sa["accepted"], "plain", sa["plain"], "graph cycles",
          sa["graph_cycles"], "captures", sa["captures"])
    assert ta == te
    assert ta[7:10] == [5, 6, 7]
    for key in ("cycles", "accepted", "plain", "emitted"):
        assert sa[key] == se[key], key
    assert 0 < sa["graph_cycles"] <= sa["cycles"]
    assert se["graph_cycles"] == 0 and sa["captures"] >= 2
    assert not ca.counters.graph_mode and [c.offset for c in ca] == [c.offset for c in ce]


@pytest.mark.gpu
def test_decode_graph_grows_kv_caches():
    """A cache too small for the run: the op-by-op path grows every KV cache in
    256-token steps as it goes (engine/model.py:156-170); the captured path
    releases, grows and captures again. Same tokens, and the keys written
    before a growth stay visible after it (all drafts accepted, 4 tokens a
    cycle)."""
    m = flat_head_model(seed=74)
    m.max_context = 256
    mtp = random_mtp(m, seed=75)
    (ga, fa, la, sa, ca, mca), (ge, fe, le, se, ce, mce) = decode_pair(m, mtp, 3, 0.0, 0, prompt_len=230)
    assert mca.capacity == 256
    ta = drive(ga, fa, la, 120)
    te = drive(ge, fe, le, 120)
    assert ta == te
    assert sa["captures"] >= 2 and sa["graph_cycles"] == sa["cycles"]
    assert [c.offset for c in ca] == [c.offset for c in ce]
    assert all(c.capacity >= c.offset for c in ca if hasattr(c, "capacity")) and mca.capacity > 256
    assert min(c.capacity for c in ce if hasattr(c, "capacity")) > 256


# Regression: this test once faulted the GPU (both heads, in different runs).
# The sampler's workspace was first made inside the capture of the decoder's
# graph, so its zero fill was only recorded there; run() replays two graphs
# captured later, the step counters of the one-kernel sampler started from stale
# memory, no row decided, and the finishing kernel advanced the caches by an
# uninitialised accept count. The buffers are now made before any capture
# (Sampler.prepare_accept) and refused inside one.
@pytest.mark.gpu
@pytest.mark.parametrize("head", ["random", "flat"])
def test_graphed_run_checks_room_before_launching(head):
    """run(n) past the caches' room raises before any launch (no cycle is left
    in flight and unaccounted); run(room()) then fills the caches, release()
    hands back a state from which eager cycles (growing the caches) continue the
    stream of a decoder that ran eagerly throughout."""
    from qvex import _C
    from qvex.speculative import GraphedMTPCycle
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=76, device=DEV, max_context=256) \
        if head == "random" else flat_head_model(seed=77)
    m.max_context = 256
    mtp = random_mtp(m, seed=78)
    params = dict(top_k=20, top_p=0.8)
    a = start_decoder(m, mtp, 3, 0.7, seed=4, **params)
    b = start_decoder(m, mtp, 3, 0.7, seed=4, **params)
    g = GraphedMTPCycle(b)
    r = g.room()
    assert r > 0
    before = (b.cache.counters.dev.clone(), b.mtp_cache.counters.dev.clone(), b.stats["cycles"])
    with pytest.raises(_C.QvexError, match="KV cache full"):
        g.run(r + 1)
    torch.cuda.synchronize()
    assert torch.equal(before[0], b.cache.counters.dev) and torch.equal(before[1], b.mtp_cache.counters.dev)
    assert b.stats["cycles"] == before[2]
    tb = [t for part in g.run(r) for t in part]
    with pytest.raises(_C.QvexError, match="KV cache full"):
        g.run(g.room() + 1)
    ta = []
    for _ in range(r):
        ta += a.cycle()
    assert ta == tb
    g.release()
    while max(c.offset for c in a.cache) <= 300:     # past the old capacity: eager calls grow the caches
        ta += a.cycle()
        tb += b.cycle()
    assert ta == tb
    assert min(c.capacity for c in b.cache if hasattr(c, "capacity")) > 256
    assert [c.offset for c in a.cache] == [c.offset for c in b.cache]
    assert a.mtp_cache.offset == b.mtp_cache.offset
