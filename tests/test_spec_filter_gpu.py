"""Fused acceptance with the reference's score filtering (presence penalty, top-k,
top-p; engine/sampler.py:30-52) vs the fp32-emulation oracle: accept counts and
tokens identical (GPU)."""

import numpy as np
import pytest
import torch

import oracle
from qvex import kernels, synth
from test_spec_gpu import DEV, assert_same, inv


def make_case(S, k, V, seed, bf16=False, draft_logits=False):
    g = np.random.default_rng(seed)
    target = (g.standard_normal((S, k + 1, V)) * 3.0).astype(np.float32)
    for s in range(S):
        for i in range(k + 1):
            target[s, i, g.integers(0, V, 3)] += 8.0
    if bf16:
        target = synth.bf16_to_f32(synth.bf16_bits(target))          # heavy exact ties
    ids = np.empty((S, k), np.int32)
    for s in range(S):
        for i in range(k):
            top = np.argsort(-target[s, i])[:40]
            ids[s, i] = top[0] if g.random() < 0.6 else top[g.integers(1, 40)]
    draft = (target[:, :k] + g.standard_normal((S, k, V)).astype(np.float32)) if draft_logits else None
    ua = g.random((S, k)).astype(np.float32)
    us = g.random(S).astype(np.float32)
    seen = (g.random(V) < 0.05).astype(np.float32)
    return target, draft, ids, ua, us, seen


def run_both(target, draft, ids, ua, us, T, seen=None, **kw):
    t = torch.from_numpy(target).to(DEV)
    d = torch.from_numpy(draft).to(DEV) if draft is not None else None
    sd = torch.from_numpy(seen).to(DEV) if seen is not None else None
    n, tok = kernels.spec_accept(t, d, torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV),
                                 torch.from_numpy(us).to(DEV), T, seen=sd, **kw)
    torch.cuda.synchronize()
    n_o, tok_o = oracle.spec_accept(target, draft, ids, ua, us, inv(T), threads=16, seen=seen, **kw)
    return n.cpu().numpy(), tok.cpu().numpy(), n_o, tok_o


CASES = [
    # S, k, V, T, top_k, top_p, penalty, bf16, draft_logits
    (12, 3, 248320, 0.7, 20, 0.95, 0.0, False, False),     # the reference's defaults
    (12, 3, 248320, 0.6, 20, 0.95, 1.2, True, False),      # + presence penalty, bf16 ties
    (16, 2, 50000, 1.0, 8, 1.0, 0.0, True, False),         # top-k only, ties at the k-th value
    (16, 4, 20000, 0.7, 64, 0.5, 0.5, False, False),       # wide k, tight p
    (16, 1, 8192, 0.9, 1, 1.0, 0.0, False, False),         # top-1
    (8, 3, 30000, 0.7, 20, 0.9, 0.8, False, True),         # draft logits (q unfiltered)
    (24, 0, 248320, 0.7, 20, 0.95, 0.3, True, False),      # plain sampling (k = 0)
    (6, 3, 248320, 0.8, 64, 0.9, 0.0, True, False),        # 31 x 64 candidates: the 16-slot merge
    # wide form: top-p over the whole vocabulary, top-k > 64
    (12, 3, 248320, 0.7, 0, 0.9, 0.0, False, False),       # whole-vocabulary top-p
    (8, 3, 248320, 0.6, 200, 0.95, 1.2, True, False),      # top-k 200 + top-p + penalty, bf16 ties
    (8, 2, 248320, 1.0, 1000, 1.0, 0.0, True, False),      # top-k only, 1000 candidates
    (6, 3, 50000, 0.7, 0, 0.5, 0.5, False, True),          # tight whole-vocabulary p, draft logits
    (16, 4, 20000, 0.7, 20000, 0.8, 0.0, False, False),    # top_k = V: no top-k (the reference's rule)
    (8, 3, 248320, 1.5, 0, 0.9, 0.0, False, False),        # flat: tens of thousands of tokens kept
    (4, 2, 248320, 2.0, 3000, 0.7, 0.4, True, False),      # flat, top-k 3000 then top-p, ties
]


@pytest.mark.gpu
@pytest.mark.parametrize("S,k,V,T,top_k,top_p,pen,bf16,dl", CASES)
def test_filtered_accept_bit_exact(S, k, V, T, top_k, top_p, pen, bf16, dl):
    target, draft, ids, ua, us, seen = make_case(S, k, V, seed=S * 7 + k + top_k, bf16=bf16, draft_logits=dl)
    assert_same(*run_both(target, draft, ids, ua, us, T, seen=seen if pen else None, presence_penalty=pen,
                          top_k=top_k, top_p=top_p))


@pytest.mark.gpu
@pytest.mark.parametrize("top_k,top_p", [(20, 0.8), (1, 1.0), (64, 0.95), (5, 1.0)])
def test_list_form_ties_bit_exact(top_k, top_p):
    """The list form without draft logits draws from each part's stored candidates
    (indices with z at or above the part's k-th value, at most 96 per part) and
    falls back to the full pass when a part holds more ties at the cutoff. Rows:
    all logits equal (every part overflows at the cutoff), three distinct values
    (thousands of ties), values on a 0.25 grid (ties at the cutoff in some parts),
    and ordinary rows; S = 8 steps of k = 3 drafts, V = 248,320."""
    S, k, V = 8, 3, 248320
    target, _, ids, ua, us, _ = make_case(S, k, V, seed=300 + top_k, bf16=True)
    g = np.random.default_rng(301 + top_k)
    target[0] = 1.5
    target[1] = g.integers(0, 3, size=(k + 1, V)).astype(np.float32)
    target[2] = np.round(g.standard_normal((k + 1, V)) * 4.0).astype(np.float32) / 4.0
    target[3, 1:] = 0.0                          # rows after the first tied
    ids[:4] = g.integers(0, V, size=(4, k)).astype(np.int32)
    ua[:4] = g.random((4, k)).astype(np.float32) * 0.5
    assert_same(*run_both(target, None, ids, ua, us, 0.7, top_k=top_k, top_p=top_p))


@pytest.mark.gpu
@pytest.mark.parametrize("top_k,top_p", [(20, 0.8), (32, 1.0), (7, 0.95)])
def test_list_form_clustered_kept_set(top_k, top_p):
    """Kept tokens packed into few walk slots and groups, bit-exact with the
    oracle: the largest logits at indices 0..39 (part 0, wave quarter 0: ten
    thread slots of four elements, so one part holds the whole kept set, slots
    hold several weights and one group holds many slots), a step with them
    spread over two quarters of one part, and a step with ties across parts;
    S = 6 steps of k = 7 drafts (two rows per wave of the finish kernel)."""
    S, k, V = 6, 7, 248320
    target, _, ids, ua, us, _ = make_case(S, k, V, seed=500 + top_k, bf16=True)
    g = np.random.default_rng(501 + top_k)
    base = synth.bf16_to_f32(synth.bf16_bits(40.0 + 2.0 * g.standard_normal((S, k + 1, 40)).astype(np.float32)))
    target[0, :, :40] = base[0]
    target[1, :, 256:276] = base[1, :, :20]                  # quarter 1 of part 0
    target[1, :, 1024:1044] = base[1, :, 20:40]              # quarter 0 again, next i
    target[2, :, ::8192] = 40.0                              # one tie in every part
    target[3, :, :64] = 40.0                                 # 64 equal maxima in one part
    ids[:4] = g.integers(0, 40, size=(4, k)).astype(np.int32)
    ua[:4] = g.random((4, k)).astype(np.float32) * 0.3
    assert_same(*run_both(target, None, ids, ua, us, 0.7, top_k=top_k, top_p=top_p))


def run_tiles(target, ids, ua, us, T, **kw):
    """spec_accept through the one-kernel list form (tile maxima of bf16 target
    rows), against the oracle on the same inputs."""
    t = torch.from_numpy(target).to(DEV).to(torch.bfloat16)
    S, k1, V = target.shape
    tm = kernels.tile_max(t.reshape(S * k1, V))
    n, tok = kernels.spec_accept(t, None, torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV),
                                 torch.from_numpy(us).to(DEV), T, tile_max=tm, **kw)
    torch.cuda.synchronize()
    n_o, tok_o = oracle.spec_accept(target, None, ids, ua, us, inv(T), threads=16, **kw)
    return n.cpu().numpy(), tok.cpu().numpy(), n_o, tok_o


TILE_CASES = [
    # S, k, V, T, top_k, top_p, penalty
    (12, 3, 248320, 0.7, 20, 0.8, 0.0),          # the decode cycle's call
    (12, 3, 248320, 0.7, 20, 0.95, 0.0),
    (16, 2, 50048, 1.0, 8, 1.0, 0.0),            # top-k only, ties at the k-th value
    (16, 4, 20096, 0.7, 64, 0.5, 0.0),           # wide k, tight p
    (16, 1, 8192, 0.9, 1, 1.0, 0.0),             # top-1
    (8, 7, 248320, 0.6, 32, 0.9, 0.0),           # k = 7
    (24, 0, 248320, 0.7, 20, 0.95, 0.0),         # plain sampling (k = 0)
    (6, 3, 248320, 0.8, 64, 0.9, 0.0),
    (12, 3, 248320, 0.6, 20, 0.95, 1.2),         # presence penalty: the two-kernel path
]


@pytest.mark.gpu
@pytest.mark.parametrize("S,k,V,T,top_k,top_p,pen", TILE_CASES)
def test_tiles_form_bit_exact(S, k, V, T, top_k, top_p, pen):
    target, _, ids, ua, us, seen = make_case(S, k, V, seed=S * 13 + k + top_k, bf16=True)
    kw = dict(top_k=top_k, top_p=top_p)
    if pen:
        kw.update(seen=seen, presence_penalty=pen)
        t = torch.from_numpy(target).to(DEV).to(torch.bfloat16)
        tm = kernels.tile_max(t.reshape(-1, V))
        n, tok = kernels.spec_accept(t, None, torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV),
                                     torch.from_numpy(us).to(DEV), T, tile_max=tm, seen=torch.from_numpy(seen).to(DEV),
                                     presence_penalty=pen, top_k=top_k, top_p=top_p)
        torch.cuda.synchronize()
        n_o, tok_o = oracle.spec_accept(target, None, ids, ua, us, inv(T), threads=16, seen=seen,
                                        presence_penalty=pen, top_k=top_k, top_p=top_p)
        assert_same(n.cpu().numpy(), tok.cpu().numpy(), n_o, tok_o)
        return
    assert_same(*run_tiles(target, ids, ua, us, T, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("top_k,top_p", [(20, 0.8), (1, 1.0), (64, 0.95), (5, 1.0), (32, 1.0)])
def test_tiles_form_ties_and_clusters(top_k, top_p):
    """The one-kernel list form on rows that leave its fast path (all logits
    equal, three distinct values: too many candidate tiles or values, so the
    block runs the two-kernel path's code; a 0.25 grid: ties at the cutoff), on
    kept sets packed into few walk slots and groups (the largest logits at
    indices 0..39, or in two quarters of one part; one tie in every part; 64
    equal maxima in one part), and on ordinary rows; S = 10, k = 3, bit-exact
    with the oracle."""
    S, k, V = 10, 3, 248320
    target, _, ids, ua, us, _ = make_case(S, k, V, seed=700 + top_k, bf16=True)
    g = np.random.default_rng(701 + top_k)
    target[0] = 1.5
    target[1] = g.integers(0, 3, size=(k + 1, V)).astype(np.float32)
    target[2] = np.round(g.standard_normal((k + 1, V)) * 4.0).astype(np.float32) / 4.0
    target[3, 1:] = 0.0
    base = synth.bf16_to_f32(synth.bf16_bits(40.0 + 2.0 * g.standard_normal((k + 1, 40)).astype(np.float32)))
    target[4, :, :40] = base
    target[5, :, 256:276] = base[:, :20]
    target[5, :, 1024:1044] = base[:, 20:40]
    target[6, :, ::8192] = 40.0
    target[7, :, :64] = 40.0
    ids[:8] = g.integers(0, 40, size=(8, k)).astype(np.int32)
    ua[:8] = g.random((8, k)).astype(np.float32) * 0.3
    assert_same(*run_tiles(target, ids, ua, us, 0.7, top_k=top_k, top_p=top_p))


def decide_rows(rows, S, k):
    """A step's (n, token) from its rows' (accept flag, draw), as the decode
    loop decides (engine/speculative.py:74-81): the first rejected draft's draw,
    or the bonus row's when all k are accepted."""
    rows = rows.reshape(S, k + 1, 2)
    n = np.full(S, k, dtype=np.int32)
    for s in range(S):
        for r in range(k):
            if rows[s, r, 0] == 0:
                n[s] = r
                break
    return n, rows[np.arange(S), n, 1].astype(np.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("S,k,V,T,top_k,top_p,pen", [c for c in TILE_CASES if c[6] == 0.0])
def test_tiles_rows_form_bit_exact(S, k, V, T, top_k, top_p, pen):
    """The one-kernel form without the step decision (spec_accept_rows, what the
    decode cycle runs): deciding each step from its rows gives the oracle's
    (n, token), and rows on which ties force the in-block slow path do too."""
    target, _, ids, ua, us, _ = make_case(S, k, V, seed=S * 17 + k + top_k, bf16=True)
    if S >= 3 and V >= 8192:
        target[0] = 1.5                                   # all equal: the slow path
        target[1, :, :64] = 40.0                          # 64 equal maxima
    t = torch.from_numpy(target).to(DEV).to(torch.bfloat16)
    tm = kernels.tile_max(t.reshape(-1, V))
    assert kernels.tiles_rows_apply(S, k, V, T, top_k, 0.0)
    rows = kernels.spec_accept_rows(t, torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV),
                                    torch.from_numpy(us).to(DEV), T, tm, top_k=top_k, top_p=top_p)
    torch.cuda.synchronize()
    n, tok = decide_rows(rows.cpu().numpy(), S, k)
    n_o, tok_o = oracle.spec_accept(target, None, ids, ua, us, inv(T), threads=16, top_k=top_k, top_p=top_p)
    assert_same(n, tok, n_o, tok_o)


def test_tiles_rows_apply_conditions():
    """The one-kernel form serves bf16 sampling with 1 <= top_k <= 64, no
    penalty and V a multiple of 128 (the C-ABI query, no GPU call)."""
    assert kernels.tiles_rows_apply(1, 3, 248320, 0.7, 20, 0.0)
    assert not kernels.tiles_rows_apply(1, 3, 248320, 0.7, 20, 0.3)     # penalty
    assert not kernels.tiles_rows_apply(1, 3, 248320, 0.0, 20, 0.0)     # greedy
    assert not kernels.tiles_rows_apply(1, 3, 248320, 0.7, 0, 0.0)      # no top-k
    assert not kernels.tiles_rows_apply(1, 3, 248320, 0.7, 65, 0.0)     # wide top-k
    assert not kernels.tiles_rows_apply(1, 3, 248328, 0.7, 20, 0.0)     # V % 128


@pytest.mark.gpu
def test_tiles_form_counters_stay_zero():
    """The one-kernel form counts each step's finished rows in the workspace and
    leaves the count at zero: many calls on one workspace, alternating with the
    two-kernel path on the same workspace, all bit-exact."""
    S, k, V = 4, 3, 248320
    ws = kernels.spec_workspace(S, k, V, False, DEV, 20)
    for rep in range(6):
        target, _, ids, ua, us, _ = make_case(S, k, V, seed=900 + rep, bf16=True)
        t = torch.from_numpy(target).to(DEV).to(torch.bfloat16)
        tm = kernels.tile_max(t.reshape(-1, V)) if rep % 2 == 0 else None
        n, tok = kernels.spec_accept(t, None, torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV),
                                     torch.from_numpy(us).to(DEV), 0.7, workspace=ws, tile_max=tm, top_k=20,
                                     top_p=0.8)
        torch.cuda.synchronize()
        n_o, tok_o = oracle.spec_accept(target, None, ids, ua, us, inv(0.7), threads=16, top_k=20, top_p=0.8)
        assert_same(n.cpu().numpy(), tok.cpu().numpy(), n_o, tok_o)


@pytest.mark.gpu
def test_list_form_cycle_shape_many_seeds():
    """The decode cycle's call (one step, k = 3, top-k 20, top-p 0.8, T = 0.7, bf16
    logits) over 48 seeded rows of steps, bit-exact with the oracle."""
    target, _, ids, ua, us, _ = make_case(48, 3, 248320, seed=777, bf16=True)
    assert_same(*run_both(target, None, ids, ua, us, 0.7, top_k=20, top_p=0.8))


@pytest.mark.gpu
@pytest.mark.parametrize("k", [0, 3])
def test_greedy_presence_penalty_bit_exact(k):
    target, _, ids, ua, us, seen = make_case(16, k, 248320, seed=90 + k, bf16=True)
    assert_same(*run_both(target, None, ids, ua, us, 0.0, seen=seen, presence_penalty=2.0))


@pytest.mark.gpu
def test_filtered_tokens_stay_in_the_kept_set():
    """Every emitted token has a target score >= the row's cutoff (checked on the oracle's
    restated kept set for k = 0)."""
    S, V, T = 64, 30000, 0.7
    target, _, _, _, us, _ = make_case(S, 0, V, seed=95, bf16=True)
    n, tok, _, _ = run_both(target, None, np.zeros((S, 0), np.int32), np.zeros((S, 0), np.float32), us, T,
                            top_k=10, top_p=0.8)
    for s in range(S):
        z = target[s, 0] * np.float32(inv(T))
        kth = np.sort(z)[::-1][9]
        assert z[tok[s]] >= kth


@pytest.mark.gpu
@pytest.mark.parametrize("S,k,V,T,top_k,top_p,pen,dl", [
    (1, 3, 248320, 0.7, 20, 0.8, 0.0, False),
    (1, 3, 248320, 0.0, 0, 1.0, 0.0, False),
    (2, 4, 50000, 1.0, 0, 1.0, 0.5, True),
    (1, 0, 4096, 0.6, 64, 0.95, 1.5, False),
    (3, 2, 4100, 0.0, 0, 1.0, 1.0, False),
])
def test_bf16_logits_equal_their_fp32_copies(S, k, V, T, top_k, top_p, pen, dl):
    """qvex_spec_accept_filtered_bf16 on bf16 logits == the fp32 entry on the same
    values widened (exact), bit for bit in n and token."""
    target, draft, ids, ua, us, seen = make_case(S, k, V, seed=S * 31 + k + V, bf16=True, draft_logits=dl)
    if draft is not None:
        draft = synth.bf16_to_f32(synth.bf16_bits(draft))
    t32 = torch.from_numpy(target).to(DEV)
    d32 = torch.from_numpy(draft).to(DEV) if draft is not None else None
    args = (torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV), torch.from_numpy(us).to(DEV), T)
    kw = dict(seen=torch.from_numpy(seen).to(DEV) if pen else None, presence_penalty=pen, top_k=top_k, top_p=top_p)
    n1, tok1 = kernels.spec_accept(t32, d32, *args, **kw)
    n2, tok2 = kernels.spec_accept(t32.to(torch.bfloat16), None if d32 is None else d32.to(torch.bfloat16),
                                   *args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(n1, n2) and torch.equal(tok1, tok2)


# ---------------------------------------------------------------- Sampler.scores (engine/sampler.py:30-52)

@pytest.mark.gpu
@pytest.mark.parametrize("V,T,top_k,top_p,pen,bf16", [
    (248320, 0.7, 20, 0.95, 0.0, True), (248320, 0.6, 0, 0.9, 1.2, False), (50000, 1.0, 200, 1.0, 0.0, True),
    (4096, 0.0, 20, 0.9, 0.7, False), (4096, 0.8, 0, 1.0, 0.0, False), (20000, 0.7, 64, 0.5, 0.5, True),
    (248320, 1.5, 0, 0.9, 0.0, False), (248320, 2.0, 3000, 0.7, 0.4, True)])
def test_scores_kept_set_and_values(V, T, top_k, top_p, pen, bf16):
    """Sampler.scores on the device: the kept set is exactly z >= the oracle's
    cutoff (the rule the accept kernels use); values equal z - c_0 - log(S) of
    the oracle's record within fp32 rounding; greedy gives the penalised logits;
    extra_seen counts for this call only."""
    from qvex.sampler import Sampler, SamplingParams
    g = np.random.default_rng(V + top_k)
    logits = (g.standard_normal(V) * 3.0).astype(np.float32)
    logits[g.integers(0, V, 3)] += 8.0
    if bf16:
        logits = synth.bf16_to_f32(synth.bf16_bits(logits))
    seen = (g.random(V) < 0.05).astype(np.float32)
    extra = g.integers(0, V, 3)
    s = Sampler(SamplingParams(temperature=T, top_k=top_k, top_p=top_p, presence_penalty=pen), V)
    if pen:
        s.seen = torch.from_numpy(seen).to(DEV)
    lt = torch.from_numpy(logits).to(DEV)
    got = s.scores(lt.to(torch.bfloat16) if bf16 else lt, extra_seen=extra).cpu().numpy().astype(np.float64)
    if pen:
        assert torch.equal(s.seen.cpu(), torch.from_numpy(seen))            # extra_seen left no mark
    sv = seen.copy()
    sv[extra] = 1.0
    x = logits - np.float32(pen) * sv if pen else logits
    if T <= 0:
        np.testing.assert_array_equal(got, x.astype(np.float64))
        return
    c0, S, cut = oracle.row_filter(logits, inv(T), seen=sv if pen else None, presence_penalty=pen, top_k=top_k,
                                   top_p=top_p)
    z = (x.astype(np.float32) * np.float32(inv(T))).astype(np.float64)
    kept = z >= cut
    assert np.array_equal(np.isfinite(got), kept)
    ref = z[kept] - float(c0) - np.log(float(S))
    assert np.abs(got[kept] - ref).max() <= 1e-5 * (1.0 + np.abs(ref).max())
    print(f"V={V} top_k={top_k} top_p={top_p}: kept {int(kept.sum())}")
