"""Committed golden fixtures (tests/golden/make_golden.py): the oracle must keep
reproducing them (CPU), and the HIP kernels must match them (GPU)."""

from pathlib import Path

import numpy as np
import pytest

import oracle

G = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(G / f"{name}.npz"))


def test_oracle_qmv_fixture():
    d = load("qmv_small")
    np.testing.assert_array_equal(oracle.qmv_f64(d["x"], d["w"], d["scales"], d["biases"]), d["y"])


def test_oracle_gdn_fixture():
    d = load("gdn_small")
    f = oracle.bf16_to_f32
    y, st, sn = oracle.gated_delta_f64(f(d["q"]), f(d["k"]), f(d["v"]), f(d["a"]), f(d["b"]), d["A_log"],
                                       f(d["dt_bias"]), d["state"])
    np.testing.assert_array_equal(y, d["y"])
    np.testing.assert_array_equal(st.astype(np.float32), d["state_final"])
    np.testing.assert_array_equal(sn[2].astype(np.float32), d["state_t2"])


def test_oracle_spec_fixture():
    d = load("spec_small")
    inv = float(np.float32(1.0) / np.float32(0.7))
    n, tok = oracle.spec_accept(d["target"], d["draft"], d["draft_ids"], d["u_accept"], d["u_sample"], inv)
    np.testing.assert_array_equal(n, d["n_accept"])
    np.testing.assert_array_equal(tok, d["out_token"])
    n, tok = oracle.spec_accept(d["target"], None, d["draft_ids"], d["u_accept"], d["u_sample"], inv)
    np.testing.assert_array_equal(n, d["n_accept_onehot"])
    np.testing.assert_array_equal(tok, d["out_token_onehot"])


@pytest.mark.gpu
def test_kernels_match_fixtures():
    import torch
    from qvex import kernels
    dev = "cuda:0"

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)

    d = load("qmv_small")
    y = kernels.quantized_matmul(bf(d["x"]), torch.from_numpy(d["w"].view(np.int32)).to(dev), bf(d["scales"]),
                                 bf(d["biases"]))
    got = oracle.bf16_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
    assert np.all(np.abs(got - d["y"]) <= 2.0 ** -7 * np.abs(d["y"]) + 1e-3)

    g = load("gdn_small")
    yy, sn = kernels.gated_delta_snapshots(*(bf(g[n]) for n in ("q", "k", "v", "a", "b")),
                                           torch.from_numpy(g["A_log"]).to(dev), bf(g["dt_bias"]),
                                           torch.from_numpy(g["state"]).to(dev))
    torch.cuda.synchronize()
    assert np.abs(sn[-1].cpu().numpy() - g["state_final"]).max() < 1e-5
    assert np.abs(sn[2].cpu().numpy() - g["state_t2"]).max() < 1e-5

    s = load("spec_small")
    t = lambda a: torch.from_numpy(a).to(dev)
    n, tok = kernels.spec_accept(t(s["target"]), t(s["draft"]), t(s["draft_ids"]), t(s["u_accept"]),
                                 t(s["u_sample"]), 0.7)
    assert np.array_equal(n.cpu().numpy(), s["n_accept"]) and np.array_equal(tok.cpu().numpy(), s["out_token"])
