"""The sampler's device uniform stream and API edges (GPU).

* qvex_philox_uniforms and the cycle's finishing kernel draw exactly the
  oracle's Philox4x32-10 stream (bit for bit), across the 32-bit counter edge;
* Sampler.pick takes scores, as engine/sampler.py:57-58 (temperature applied
  once when composed as pick(scores(logits)));
* a captured cycle refuses to run past a KV cache's capacity, and eager calls
  on caches it drives raise until release()."""

import numpy as np
import pytest
import torch

import oracle
from qvex import _C
from qvex.kernels import _ptr, _stream
from qvex.model import Config, random_model
from qvex.mtp import random_mtp
from qvex.sampler import Sampler, SamplingParams
from qvex.speculative import GraphedMTPCycle, MTPDecoder, mtp_prefill

DEV = "cuda:0"


@pytest.mark.gpu
def test_device_uniforms_equal_oracle_stream():
    seed = 0x123456789ABCDEF0
    ev0 = (3 << 32) + 0xFFFFFFFE                 # the low counter word wraps inside the run
    counter = torch.tensor([ev0], dtype=torch.int64, device=DEV)
    outs = []
    for n in (5, 1, 256, 9):
        out = torch.empty(n, dtype=torch.float32, device=DEV)
        _C.call("qvex_philox_uniforms", seed, counter.data_ptr(), n, out.data_ptr(), _stream())
        outs.append(out)
    # the finishing kernel draws the next event the same way
    k = 3
    ids = torch.zeros(k + 1, dtype=torch.int32, device=DEV)
    n_t = torch.zeros(1, dtype=torch.int32, device=DEV)
    tok = torch.zeros(1, dtype=torch.int32, device=DEV)
    pend, feed, nprev = (torch.zeros(k + 1, dtype=torch.int32, device=DEV), torch.zeros(1, dtype=torch.int32, device=DEV),
                         torch.zeros(1, dtype=torch.int32, device=DEV))
    res = torch.zeros(k + 2, dtype=torch.int32, device=DEV)
    u = torch.empty(k + 1, dtype=torch.float32, device=DEV)
    _C.call("qvex_cycle_finish_ex", _ptr(ids) + 4, k, _ptr(n_t), _ptr(tok), _ptr(pend), _ptr(feed), _ptr(nprev),
            _ptr(res), _ptr(ids), None, 0, 0, None, 0, 0, seed, counter.data_ptr(), k + 1, _ptr(u), None, None,
            _stream())
    torch.cuda.synchronize()
    for j, out in enumerate(outs):
        np.testing.assert_array_equal(out.cpu().numpy(), oracle.philox_uniforms(seed, ev0 + j, out.numel()))
    np.testing.assert_array_equal(u.cpu().numpy(), oracle.philox_uniforms(seed, ev0 + 4, k + 1))
    assert int(counter.item()) == ev0 + 5


@pytest.mark.gpu
def test_cycle_finish_done_flag_in_pinned_memory():
    """With `done`, the finishing kernel writes [n, token, drafts] into pinned
    host memory and then sets the flag: a host polling the flag (no stream
    synchronisation) reads the complete result, and the device-side
    bookkeeping (pending ids, feed, n_prev, next ids) is the same as without."""
    k = 3
    ids = torch.tensor([7, 11, 22, 33], dtype=torch.int32, device=DEV)
    n_t = torch.tensor([2], dtype=torch.int32, device=DEV)
    tok = torch.tensor([99], dtype=torch.int32, device=DEV)
    pend, feed, nprev = (torch.zeros(k + 1, dtype=torch.int32, device=DEV), torch.zeros(1, dtype=torch.int32, device=DEV),
                         torch.zeros(1, dtype=torch.int32, device=DEV))
    out = torch.full((k + 2,), -5, dtype=torch.int32, pin_memory=True)
    done = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    flag = done.numpy()
    _C.call("qvex_cycle_finish_ex", _ptr(ids) + 4, k, _ptr(n_t), _ptr(tok), _ptr(pend), _ptr(feed), _ptr(nprev),
            out.data_ptr(), _ptr(ids), None, 0, 0, None, 0, 0, 0, None, 0, None, done.data_ptr(), None, _stream())
    ev = torch.cuda.Event()
    ev.record()
    spins = 0
    while flag[0] == 0:
        spins += 1
        assert not (spins % 1024 == 0 and ev.query() and flag[0] == 0), "done flag never set"
    assert out.numpy().tolist() == [2, 99, 11, 22, 33]
    torch.cuda.synchronize()
    assert pend.tolist() == [11, 22, 99, 0] and int(feed) == 99 and int(nprev) == 2 and int(ids[0]) == 99


@pytest.mark.gpu
@pytest.mark.parametrize("flags,n_want", [([1, 1, 1, 0], 3), ([1, 0, 1, 0], 1), ([0, 1, 1, 0], 0)])
def test_cycle_finish_decides_from_rows(flags, n_want):
    """With rows (each verify row's accept flag and draw), the finishing kernel
    takes the first rejection's draw (or the bonus row's) and does the same
    bookkeeping as when given (n, token)."""
    k = 3
    draws = [101, 202, 303, 404]
    rows = torch.tensor([[f, d] for f, d in zip(flags, draws)], dtype=torch.int32, device=DEV)
    outs = []
    for use_rows in (True, False):
        ids = torch.tensor([7, 11, 22, 33], dtype=torch.int32, device=DEV)
        n_t = torch.tensor([n_want], dtype=torch.int32, device=DEV)
        tok = torch.tensor([draws[n_want]], dtype=torch.int32, device=DEV)
        pend, feed, nprev = (torch.zeros(k + 1, dtype=torch.int32, device=DEV),
                             torch.zeros(1, dtype=torch.int32, device=DEV), torch.zeros(1, dtype=torch.int32, device=DEV))
        ctr = torch.tensor([5, 9], dtype=torch.int32, device=DEV)
        res = torch.zeros(k + 2, dtype=torch.int32, device=DEV)
        _C.call("qvex_cycle_finish_ex", _ptr(ids) + 4, k, None if use_rows else _ptr(n_t),
                None if use_rows else _ptr(tok), _ptr(pend), _ptr(feed), _ptr(nprev), _ptr(res), _ptr(ids),
                _ptr(ctr), 2, 1, None, 0, 0, 0, None, 0, None, None, _ptr(rows) if use_rows else None, _stream())
        torch.cuda.synchronize()
        outs.append([t.cpu().tolist() for t in (res, pend, feed, nprev, ids, ctr)])
    assert outs[0] == outs[1]
    assert outs[0][0][:2] == [n_want, draws[n_want]] and outs[0][5] == [5 + n_want + 1, 9 + n_want + 1]


@pytest.mark.gpu
def test_pick_takes_scores():
    """logits [0, ln 4] at T = 0.5: scores give p(1) = 16/17; applying the
    temperature twice would give 256/257."""
    V = 8
    logits = torch.full((V,), -1e4, dtype=torch.float32, device=DEV)
    logits[1] = float(np.log(4.0))
    logits[0] = 0.0
    s = Sampler(SamplingParams(temperature=0.5, top_k=0, top_p=1.0, seed=3), V)
    sc = s.scores(logits)
    toks = torch.cat([s.pick(sc) for _ in range(3000)]).cpu().numpy()
    n0 = int((toks == 0).sum())
    assert set(np.unique(toks)) <= {0, 1}
    assert abs(n0 - 3000 / 17) < 5 * np.sqrt(3000 * (1 / 17) * (16 / 17)), n0
    g = Sampler(SamplingParams(temperature=0.0), V)
    assert int(g.pick(g.scores(logits)).item()) == 1 == int(g.pick_logits(logits.reshape(1, -1)).item())


def start(m, mtp, k=3, prompt=20, seed=0):
    V = m.cfg.vocab_size
    ids = torch.from_numpy(np.random.default_rng(5).integers(0, V, prompt).astype(np.int32)).reshape(1, -1).to(DEV)
    cache, mc = m.make_cache(), mtp.make_cache()
    logits, hidden = m(ids, cache, return_hidden=True)
    last_h = mtp_prefill(mtp, mc, hidden, ids, None)
    s = Sampler(SamplingParams(temperature=0.7, top_k=20, top_p=0.9, presence_penalty=0.3, seed=seed), V)
    return MTPDecoder(m, s, cache, logits[0, -1], last_h, mtp, mc, k=k)


@pytest.mark.gpu
def test_graphed_cycle_stops_at_capacity_and_release():
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=61, device=DEV, max_context=256)
    mtp = random_mtp(m, seed=62)
    dec = start(m, mtp, prompt=236)
    g = GraphedMTPCycle(dec)
    with pytest.raises(_C.QvexError, match="GraphedMTPCycle"):
        dec.cycle()
    with pytest.raises(_C.QvexError, match="captured cycle"):
        dec.cache[0].rollback(1)
    emitted = 0
    with pytest.raises(_C.QvexError, match="KV cache full"):
        for _ in range(64):
            emitted += len(g.cycle())
    assert emitted > 0
    assert all(c.offset <= 256 for c in dec.cache) and dec.mtp_cache.offset <= 256
    assert list(dec.cache.counters.dev.cpu().numpy()) == [c.offset for c in dec.cache]
    g.release()
    with pytest.raises(_C.QvexError, match="released"):
        g.cycle()


@pytest.mark.gpu
def test_release_then_eager_equals_eager_throughout():
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=63, device=DEV, max_context=1024)
    mtp = random_mtp(m, seed=64)
    a, b = start(m, mtp, seed=9), start(m, mtp, seed=9)
    ta = [a.first]
    for _ in range(10):
        ta += a.cycle()
    g = GraphedMTPCycle(b)
    tb = [b.first]
    for _ in range(5):
        tb += g.cycle()
    g.release()
    for _ in range(5):
        tb += b.cycle()
    assert ta == tb
    assert [c.offset for c in a.cache] == [c.offset for c in b.cache]
    assert torch.equal(a.sampler.seen, b.sampler.seen)


@pytest.mark.gpu
def test_sampler_buffers_made_before_capture():
    """The presence mask, the workspace and the draw counter are made (zero-filled)
    by prepare_accept outside a capture; inside one they are refused, since the
    zero fill would only be recorded and a graph captured later on the same
    buffers would start from stale memory."""
    V = 2048
    s = Sampler(SamplingParams(temperature=0.7, top_k=20, top_p=0.8, presence_penalty=0.3, seed=1), V)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(_C.QvexError, match="before a graph capture"):
        with torch.cuda.graph(g):
            s.prepare_accept(3, torch.device(DEV))
    s.prepare_accept(3, torch.device(DEV))
    ws = s._workspace(1, 3, False, torch.device(DEV))
    torch.cuda.synchronize()
    assert int(ws.abs().sum().item()) == 0 and int(s.seen.sum().item()) == 0
    assert int(s.counter(torch.device(DEV)).item()) == 0
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(_C.QvexError, match="before the graph capture"):
        with torch.cuda.graph(g2):
            from qvex import kernels
            kernels.spec_workspace(1, 3, V, False, torch.device(DEV), 20)
