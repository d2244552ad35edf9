"""Pins the filtered acceptance oracle (presence penalty, top-k, top-p; oracle/spec.c)
against a float64 restatement of Sampler.scores written step for step like the
reference (engine/sampler.py:30-52: argpartition, sort, softmax, cumsum - probs,
mask, log-softmax), by enumerating uniforms. CPU only."""

import numpy as np
import pytest

import oracle


def ref_scores(logits, T, seen=None, penalty=0.0, top_k=0, top_p=1.0, extra=()):
    x = np.asarray(logits, np.float64).copy()
    if seen is not None:
        s = np.asarray(seen, np.float64).copy()
        for e in extra:
            s[e] = min(s[e] + 1.0, 1.0)
        x = x - penalty * s
    if T <= 0:
        return x
    x = x / T
    V = x.shape[-1]
    cand = x[np.argpartition(-x, top_k - 1)[:top_k]] if 0 < top_k < V else x
    cand = np.sort(cand)[::-1]
    cutoff = cand[-1]
    if 0 < top_p < 1:
        probs = np.exp(cand - cand.max())
        probs /= probs.sum()
        keep = (np.cumsum(probs) - probs) < top_p
        cutoff = np.min(np.where(keep, cand, np.inf))
    x = np.where(x >= cutoff, x, -np.inf)
    return x - (np.log(np.exp(x - x.max()).sum()) + x.max())


def grid(n):
    return ((np.arange(n) + 0.5) / n).astype(np.float32)


def bonus_law(logits, T, n=8192, **kw):
    """Law of the k = 0 draw (plain sampling from the filtered p) over a grid of u."""
    V = logits.shape[0]
    target = np.broadcast_to(logits.astype(np.float32), (n, 1, V)).copy()
    nacc, tok = oracle.spec_accept(target, None, np.zeros((n, 0), np.int32), np.zeros((n, 0), np.float32),
                                   grid(n), 1.0 / T, threads=4, **kw)
    return np.bincount(tok, minlength=V) / n


@pytest.mark.parametrize("top_k,top_p,penalty", [(8, 1.0, 0.0), (8, 0.8, 0.0), (20, 0.95, 1.3), (1, 1.0, 0.0),
                                                 (5, 0.5, 2.0), (64, 0.9, 0.7),
                                                 # wide form: top-k > 64, top-p over the whole vocabulary
                                                 (80, 1.0, 0.0), (70, 0.8, 0.7), (0, 0.9, 0.0), (0, 0.5, 1.3),
                                                 (96, 0.8, 0.0), (500, 0.95, 0.0)])
def test_filtered_law_matches_reference_scores(top_k, top_p, penalty):
    g = np.random.default_rng(top_k * 10 + int(top_p * 100))
    V, T = 96, 0.7
    logits = (g.standard_normal(V) * 2.0).astype(np.float32)
    seen = (g.random(V) < 0.3).astype(np.float32)
    p = np.exp(ref_scores(logits, T, seen, penalty, top_k, top_p))
    law = bonus_law(logits, T, seen=seen, presence_penalty=penalty, top_k=top_k, top_p=top_p)
    np.testing.assert_allclose(law, p, atol=2.5e-3)
    assert set(np.flatnonzero(law)) <= set(np.flatnonzero(p > 0))


@pytest.mark.parametrize("top_k,top_p", [(10, 1.0), (70, 1.0), (70, 0.9), (0, 0.6)])
def test_ties_at_the_cutoff_are_all_kept(top_k, top_p):
    """bf16-like logits with many exact ties: every token equal to the cutoff
    value stays (list form for top_k <= 64, wide form otherwise)."""
    g = np.random.default_rng(7)
    V, T = 400, 1.0
    logits = np.round(g.standard_normal(V) * 2.0).astype(np.float32)   # integers: heavy ties
    p = np.exp(ref_scores(logits, T, top_k=top_k, top_p=top_p))
    kept = p > 0
    if top_k:
        assert kept.sum() > top_k     # the tie really extends past k
    law = bonus_law(logits, T, n=1 << 15, top_k=top_k, top_p=top_p)
    np.testing.assert_allclose(law, p, atol=1e-3)
    assert set(np.flatnonzero(law)) == set(np.flatnonzero(kept))


def test_wide_cutoff_is_the_cumulative_rule():
    """Whole-vocabulary top-p on a row with known masses: values 3, 2, 1, 0 with
    multiplicities 1, 2, 4, 8 at T = 1 / ln 2 (masses 8, 2 x 4, 4 x 2, 8 x 1 of 32).
    Mass above 2 is 8/32 = 0.25, above 1 is 16/32, above 0 is 24/32: top_p = 0.5
    keeps {3, 2} (0.5 is not < 0.5), 0.51 keeps down to 1, 0.76 everything."""
    vals = np.array([3.0] + [2.0] * 2 + [1.0] * 4 + [0.0] * 8 + [-60.0] * 1, np.float32)
    V = vals.size
    perm = np.random.default_rng(3).permutation(V)
    logits = vals[perm]
    inv_t = float(np.log(2.0))
    for top_p, lowest in ((0.25, 3.0), (0.26, 2.0), (0.5, 2.0), (0.51, 1.0), (0.75, 1.0), (0.76, 0.0)):
        law = bonus_law(logits, 1.0 / inv_t, n=4096, top_k=0, top_p=top_p)
        kept = set(np.flatnonzero(law))
        assert kept == set(np.flatnonzero(logits >= lowest)), (top_p, lowest)


@pytest.mark.parametrize("top_k,top_p", [(6, 1.0), (12, 0.7), (0, 0.7), (30, 0.8)])
def test_filtered_accept_probability(top_k, top_p):
    """One-hot draft d: P(accept) = p(d) of the filtered target; a filtered-out d is
    never accepted, and the first emitted token still follows p."""
    g = np.random.default_rng(11)
    V, T, n = 48, 0.8, 4096
    logits = (g.standard_normal(V) * 2.0).astype(np.float32)
    p = np.exp(ref_scores(logits, T, top_k=top_k, top_p=top_p))
    u = grid(n)
    ua, us = np.meshgrid(grid(64), grid(64), indexing="ij")
    first = np.zeros(V)
    for d in range(V):
        target = np.broadcast_to(np.stack([logits, logits]), (n, 2, V)).copy()
        nacc, tok = oracle.spec_accept(target, None, np.full((n, 1), d, np.int32), ua.reshape(n, 1),
                                       us.reshape(n), 1.0 / T, threads=4, top_k=top_k, top_p=top_p)
        assert abs((nacc == 1).mean() - p[d]) <= 1.0 / 64 + 1e-6
        if p[d] == 0:
            assert not nacc.any()
        f = np.bincount(np.where(nacc == 1, d, tok), minlength=V) / n
        first += f / V
    # drafts drawn uniformly: the first token's law is still p (speculative sampling)
    np.testing.assert_allclose(first, p, atol=0.02)


def test_greedy_presence_penalty_and_draft_extends_seen():
    """Greedy scores are the penalised logits; verify row 1 also counts draft d_0 as seen
    (the reference's extra_seen=draft for its bonus row)."""
    V = 32
    row0 = np.zeros(V, np.float32)
    row0[5] = 10.0                       # argmax of row 0 is 5: draft 5 is accepted
    row1 = np.zeros(V, np.float32)
    row1[5], row1[9] = 3.0, 2.5          # without the penalty row 1 picks 5
    seen = np.zeros(V, np.float32)
    target = np.stack([row0, row1])[None]
    n, tok = oracle.spec_accept(target, None, np.array([[5]], np.int32), np.zeros((1, 1), np.float32),
                                np.array([0.5], np.float32), 0.0, seen=seen, presence_penalty=1.0)
    assert n[0] == 1 and tok[0] == 9    # 3 - 1 < 2.5
    n, tok = oracle.spec_accept(target, None, np.array([[5]], np.int32), np.zeros((1, 1), np.float32),
                                np.array([0.5], np.float32), 0.0)
    assert n[0] == 1 and tok[0] == 5
    seen[5] = 1.0                        # now row 0 is penalised too: 10 - 1 still wins
    n, tok = oracle.spec_accept(target, None, np.array([[5]], np.int32), np.zeros((1, 1), np.float32),
                                np.array([0.5], np.float32), 0.0, seen=seen, presence_penalty=1.0)
    assert n[0] == 1 and tok[0] == 9


def test_unfiltered_call_is_unchanged():
    """Default arguments give the plain temperature rule bit for bit (same entry point)."""
    g = np.random.default_rng(12)
    S, k, V = 6, 2, 3000
    target = g.standard_normal((S, k + 1, V)).astype(np.float32)
    ids = g.integers(0, V, (S, k)).astype(np.int32)
    ua, us = g.random((S, k)).astype(np.float32), g.random(S).astype(np.float32)
    a = oracle.spec_accept(target, None, ids, ua, us, 1.0 / 0.7)
    b = oracle.spec_accept(target, None, ids, ua, us, 1.0 / 0.7, seen=np.zeros(V, np.float32),
                           presence_penalty=0.0, top_k=0, top_p=1.0)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
