"""Writes the committed golden fixtures of the verify path (tests/golden/*.npz).

The reference ships no golden vectors for this path (its parity files are
generated at run time and git-ignored), so these fixtures are written from the
CPU oracle and cross-checked here against independent formulations before
saving: the qmv against a dense numpy dequantisation (np.unpackbits in the MLX
bit order), the DeltaNet against the matrix form S = g S (I - b k k^T) + b v k^T,
and the sampler against a float64 evaluation of the textbook accept rule away
from ties. Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "qvex-3.5_amd"))

import oracle  # noqa: E402
from qvex import synth  # noqa: E402


def qmv_fixture():
    M, N, K = 5, 96, 384
    w, s, b = synth.qmv_weights(N, K, seed=4242)
    x = synth.qmv_x(M, K, seed=4242)
    y = oracle.qmv_f64(x, w, s, b)
    dense = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.dequant_w4_f64(w, s, b, K).T
    assert np.allclose(y, dense, rtol=1e-12, atol=1e-12)
    return dict(x=x, w=w, scales=s, biases=b, y=y)


def gdn_fixture():
    inp = synth.gdn_inputs(5, seed=4243, Hk=2, Hv=4)
    f = synth.bf16_to_f32
    q, k, v, a, b = (f(inp[n]) for n in ("q", "k", "v", "a", "b"))
    y, st, sn = oracle.gated_delta_f64(q, k, v, a, b, inp["A_log"], f(inp["dt_bias"]), inp["state"])
    # matrix form, float64
    S = inp["state"].astype(np.float64).copy()
    for t in range(5):
        for hv in range(4):
            kk = k[0, t, hv // 2].astype(np.float64)
            xx = float(a[0, t, hv])
            g = np.exp(-np.log1p(np.exp(xx)))
            beta = 1 / (1 + np.exp(-float(b[0, t, hv])))
            S[0, hv] = g * S[0, hv] @ (np.eye(128) - beta * np.outer(kk, kk)) + beta * np.outer(v[0, t, hv], kk)
            assert np.allclose(S[0, hv] @ q[0, t, hv // 2], y[0, t, hv], rtol=1e-9, atol=1e-12)
        assert np.allclose(S, sn[t], rtol=1e-9, atol=1e-12)
    # stored in float32: the final state and the state after token 2 (a rollback target)
    return dict(**inp, y=y, state_final=sn[-1].astype(np.float32), state_t2=sn[2].astype(np.float32))


def spec_fixture():
    inp = synth.spec_inputs(range(8), k=3, V=4096, temperature=0.7, seed=4244)
    inv = float(np.float32(1.0) / np.float32(0.7))
    n, tok = oracle.spec_accept(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"], inp["u_sample"], inv)
    # float64 textbook check of every accept decision that is not within 1e-5 of a tie
    for s in range(8):
        for i in range(3):
            p = np.exp((inp["target"][s, i] * inv).astype(np.float64))
            q = np.exp((inp["draft"][s, i] * inv).astype(np.float64))
            p /= p.sum()
            q /= q.sum()
            d = inp["draft_ids"][s, i]
            ratio = p[d] / q[d]
            u = float(inp["u_accept"][s, i])
            if i < n[s]:
                assert u < ratio + 1e-5
            elif i == n[s]:
                assert u >= ratio - 1e-5
                break
    n_g, tok_g = oracle.spec_accept(inp["target"], None, inp["draft_ids"], inp["u_accept"], inp["u_sample"], inv)
    return dict(**inp, n_accept=n, out_token=tok, n_accept_onehot=n_g, out_token_onehot=tok_g)


def main():
    for name, fn in (("qmv_small", qmv_fixture), ("gdn_small", gdn_fixture), ("spec_small", spec_fixture)):
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **fn())
        print("wrote", path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
