"""Fused speculative-acceptance HIP kernel vs the fp32-emulation oracle:
accept counts and tokens must be identical (GPU)."""

import numpy as np
import pytest
import torch

import oracle
from qvex import kernels, synth

DEV = "cuda:0"


def inv(T):
    return float(np.float32(1.0) / np.float32(T)) if T > 0 else 0.0


def run_both(target, draft, ids, ua, us, T, threads=16):
    t = torch.from_numpy(target).to(DEV)
    d = torch.from_numpy(draft).to(DEV) if draft is not None else None
    n, tok = kernels.spec_accept(t, d, torch.from_numpy(ids).to(DEV), torch.from_numpy(ua).to(DEV),
                                 torch.from_numpy(us).to(DEV), T)
    torch.cuda.synchronize()
    n_o, tok_o = oracle.spec_accept(target, draft, ids, ua, us, inv(T), threads=threads)
    return n.cpu().numpy(), tok.cpu().numpy(), n_o, tok_o


def assert_same(n, tok, n_o, tok_o):
    print(f"accept mean {n.mean():.3f}; mismatches n={int((n != n_o).sum())} tok={int((tok != tok_o).sum())}")
    assert np.array_equal(n, n_o)
    assert np.array_equal(tok, tok_o)


@pytest.mark.gpu
def test_config3_sample_full_vocab():
    """All 256 steps of the config-3 workload (k = 4, V = 248,320, T = 0.7), the
    seeded inputs the benchmark's spec_config3 figure runs on: accept counts and
    tokens equal the oracle's for every step."""
    inp = synth.spec_inputs(range(256), k=4, threads=16)
    assert_same(*run_both(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"], inp["u_sample"], 0.7))


@pytest.mark.gpu
def test_greedy_draft_reference_rule():
    inp = synth.spec_inputs(range(100, 116), k=3)
    ids = inp["target"][:, :3].argmax(-1).astype(np.int32)  # draft = target argmax: high acceptance
    ids[::3, 1] = inp["draft_ids"][::3, 1]
    assert_same(*run_both(inp["target"], None, ids, inp["u_accept"][:, :3], inp["u_sample"], 0.7))


@pytest.mark.gpu
def test_greedy_temperature_zero():
    inp = synth.spec_inputs(range(200, 216), k=4)
    ids = inp["target"][:, :4].argmax(-1).astype(np.int32)
    ids[::2, 2] = (ids[::2, 2] + 7) % inp["target"].shape[-1]
    n, tok, n_o, tok_o = run_both(inp["target"], inp["draft"], ids, inp["u_accept"], inp["u_sample"], 0.0)
    assert_same(n, tok, n_o, tok_o)
    assert np.all(n[::2] == 2) and np.all(n[1::2] == 4)


@pytest.mark.gpu
@pytest.mark.parametrize("V", [4, 12, 1000, 8192, 8196, 20000])
@pytest.mark.parametrize("k", [0, 1, 3])
def test_vocab_edges(V, k):
    g = np.random.default_rng(V * 10 + k)
    S = 64
    target = (3 * g.standard_normal((S, k + 1, V))).astype(np.float32)
    draft = (target[:, :k] + g.standard_normal((S, k, V))).astype(np.float32)
    ids = g.integers(0, V, size=(S, k)).astype(np.int32)
    ua = g.random((S, k), dtype=np.float32)
    us = g.random(S, dtype=np.float32)
    assert_same(*run_both(target, draft, ids, ua, us, 0.7))
    assert_same(*run_both(target, None, ids, ua, us, 1.3))


@pytest.mark.gpu
def test_adversarial_rows():
    g = np.random.default_rng(9)
    S, k, V = 12, 3, 30000
    target = (3 * g.standard_normal((S, k + 1, V))).astype(np.float32)
    draft = target[:, :k].copy()                 # p == q: all accepted
    ids = g.integers(0, V, size=(S, k)).astype(np.int32)
    draft[4:8] += 0.5 * g.standard_normal((4, k, V)).astype(np.float32)
    target[8:, 0, ids[8:, 0]] = -1e4             # p(d) = 0: reject at 0
    ids[11, 0] = V + 5                           # out-of-range draft id
    ua = g.random((S, k), dtype=np.float32)
    us = g.random(S, dtype=np.float32)
    n, tok, n_o, tok_o = run_both(target, draft, ids, ua, us, 0.7)
    assert_same(n, tok, n_o, tok_o)
    assert np.all(n[:4] == k) and np.all(n[8:] == 0)
