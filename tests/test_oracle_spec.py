"""Pins the speculative-acceptance oracle against the textbook rule (CPU only)."""

import math

import numpy as np
import pytest

import oracle


def test_expf_within_two_ulp():
    xs = np.concatenate([np.linspace(-69, 0, 20001, dtype=np.float32),
                         -np.geomspace(1e-7, 1, 2001).astype(np.float32), np.float32([0.0])])
    for x in xs:
        got = np.float32(oracle.expf(float(x)))
        ref = math.exp(float(x))
        ulp = np.spacing(np.float32(ref))
        assert abs(float(got) - ref) <= 2 * float(ulp), (x, got, ref)
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-70.0) == 0.0 and oracle.expf(float("-inf")) == 0.0


def softmax(z):
    e = np.exp(z - z.max())
    return e / e.sum()


def test_enumeration_first_token_law():
    """Over all drafts d (weight q(d)) and a grid of uniforms, the first emitted
    token is distributed as p and the accept rate is sum(min(p, q))."""
    V, T = 8, 1.0
    g = np.random.default_rng(0)
    tl = g.standard_normal(V).astype(np.float32) * 1.5
    dl = g.standard_normal(V).astype(np.float32) * 1.5
    p, q = softmax(tl.astype(np.float64)), softmax(dl.astype(np.float64))
    n = 60
    grid = ((np.arange(n) + 0.5) / n).astype(np.float32)
    ua, us = np.meshgrid(grid, grid, indexing="ij")
    S = n * n
    freq = np.zeros(V)
    acc = 0.0
    for d in range(V):
        target = np.broadcast_to(np.stack([tl, tl]), (S, 2, V)).copy()
        draft = np.broadcast_to(dl, (S, 1, V)).copy()
        nacc, tok = oracle.spec_accept(target, draft, np.full((S, 1), d, np.int32), ua.reshape(S, 1),
                                       us.reshape(S), 1.0 / T, threads=4)
        first = np.where(nacc >= 1, d, tok)
        freq += q[d] * np.bincount(first, minlength=V) / S
        acc += q[d] * (nacc >= 1).mean()
    np.testing.assert_allclose(freq, p, atol=0.02)
    assert abs(acc - np.minimum(p, q).sum()) < 0.02


def test_identical_distributions_accept_all():
    g = np.random.default_rng(1)
    S, k, V = 16, 3, 4096
    target = g.standard_normal((S, k + 1, V)).astype(np.float32)
    draft = target[:, :k].copy()
    ids = g.integers(0, V, size=(S, k)).astype(np.int32)
    nacc, tok = oracle.spec_accept(target, draft, ids, g.random((S, k), dtype=np.float32),
                                   g.random(S, dtype=np.float32), 1 / 0.7)
    assert np.all(nacc == k)
    assert np.all((tok >= 0) & (tok < V))


def test_zero_target_probability_rejects():
    g = np.random.default_rng(2)
    S, k, V = 8, 2, 1024
    target = g.standard_normal((S, k + 1, V)).astype(np.float32)
    ids = g.integers(0, V, size=(S, k)).astype(np.int32)
    for s in range(S):
        target[s, 0, ids[s, 0]] = -1e4
    nacc, tok = oracle.spec_accept(target, None, ids, np.zeros((S, k), np.float32) + 0.5,
                                   g.random(S, dtype=np.float32), 1.0)
    assert np.all(nacc == 0)
    assert np.all(tok != ids[:, 0])  # residual excludes the rejected draft


def test_one_hot_draft_rule_matches_reference():
    """q one-hot (engine/speculative.py:79-80): accept iff u < p(d); the residual
    never returns d."""
    g = np.random.default_rng(3)
    S, V = 400, 64
    target = (2.0 * g.standard_normal((S, 2, V))).astype(np.float32)
    ids = g.integers(0, V, size=(S, 1)).astype(np.int32)
    u = g.random((S, 1), dtype=np.float32)
    nacc, tok = oracle.spec_accept(target, None, ids, u, g.random(S, dtype=np.float32), 1.0)
    for s in range(S):
        p = softmax(target[s, 0].astype(np.float64))
        pd = p[ids[s, 0]]
        if abs(u[s, 0] - pd) > 1e-5:
            assert nacc[s] == (1 if u[s, 0] < pd else 0)
        if nacc[s] == 0:
            assert tok[s] != ids[s, 0]


def test_greedy_limit():
    g = np.random.default_rng(4)
    S, k, V = 32, 3, 2048
    target = g.standard_normal((S, k + 1, V)).astype(np.float32)
    am = target.argmax(-1).astype(np.int32)
    ids = am[:, :k].copy()
    ids[::2, 1] = (ids[::2, 1] + 1) % V   # even steps reject at position 1
    nacc, tok = oracle.spec_accept(target, None, ids, np.zeros((S, k), np.float32),
                                   np.zeros(S, np.float32), 0.0)
    assert np.all(nacc[::2] == 1) and np.all(tok[::2] == am[::2, 1])
    assert np.all(nacc[1::2] == k) and np.all(tok[1::2] == am[1::2, k])


def test_chi2_bonus_token_law():
    """k = 0 is plain sampling from p: chi-square of 20000 draws."""
    g = np.random.default_rng(5)
    V, S = 32, 20000
    logits = (1.5 * g.standard_normal(V)).astype(np.float32)
    target = np.broadcast_to(logits, (S, 1, V)).copy()
    _, tok = oracle.spec_accept(target, None, np.zeros((S, 0), np.int32), np.zeros((S, 0), np.float32),
                                g.random(S, dtype=np.float32), 1.0, threads=4)
    p = softmax(logits.astype(np.float64))
    cnt = np.bincount(tok, minlength=V)
    chi2 = ((cnt - S * p) ** 2 / (S * p)).sum()
    assert chi2 < 70  # df = 31: p < 1e-4 tail


def test_out_of_range_draft_is_rejected():
    target = np.zeros((1, 2, 8), np.float32)
    nacc, tok = oracle.spec_accept(target, None, np.array([[9]], np.int32), np.zeros((1, 1), np.float32),
                                   np.array([0.3], np.float32), 1.0)
    assert nacc[0] == 0 and 0 <= tok[0] < 8
