"""Pins the Gated DeltaNet oracle against a matrix formulation and the
delta-rule invariants (CPU only)."""

import numpy as np

import oracle
from qvex import synth


def small(T=5, B=1, Hk=2, Hv=4, D=16, seed=0):
    g = np.random.default_rng(seed)
    q = g.standard_normal((B, T, Hk, D)).astype(np.float32)
    k = g.standard_normal((B, T, Hk, D)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = g.standard_normal((B, T, Hv, D)).astype(np.float32)
    a = g.standard_normal((B, T, Hv)).astype(np.float32)
    b = g.standard_normal((B, T, Hv)).astype(np.float32)
    A_log = (0.3 * g.standard_normal(Hv)).astype(np.float32)
    dt = (0.3 * g.standard_normal(Hv)).astype(np.float32)
    s0 = (0.1 * g.standard_normal((B, Hv, D, D))).astype(np.float32)
    return q, k, v, a, b, A_log, dt, s0


def matrix_form(q, k, v, a, b, A_log, dt, s0):
    """S_t = g S_{t-1} (I - beta k k^T) + beta v k^T, y_t = S_t q (float64)."""
    B, T, Hk, D = k.shape
    Hv = v.shape[2]
    S = s0.astype(np.float64).copy()
    y = np.zeros((B, T, Hv, D))
    I = np.eye(D)
    for bi in range(B):
        for hv in range(Hv):
            hk = hv // (Hv // Hk)
            for t in range(T):
                x = float(a[bi, t, hv]) + float(dt[hv])
                sp = x if x > 20 else np.log1p(np.exp(x))
                g = np.exp(-np.exp(float(A_log[hv])) * sp)
                beta = 1 / (1 + np.exp(-float(b[bi, t, hv])))
                kk = k[bi, t, hk].astype(np.float64)
                S[bi, hv] = g * S[bi, hv] @ (I - beta * np.outer(kk, kk)) + beta * np.outer(v[bi, t, hv], kk)
                y[bi, t, hv] = S[bi, hv] @ q[bi, t, hk].astype(np.float64)
    return y, S


def test_matches_matrix_form():
    args = small()
    y, st, sn = oracle.gated_delta_f64(*args)
    ym, Sm = matrix_form(*args)
    np.testing.assert_allclose(y, ym, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(st, Sm, rtol=1e-10, atol=1e-12)
    np.testing.assert_array_equal(sn[-1], st)


def test_identity_gate_zero_beta_keeps_state():
    q, k, v, a, b, A_log, dt, s0 = small(seed=1)
    a[:] = -1000.0      # softplus -> 0, g -> 1
    b[:] = -1000.0      # beta -> 0
    y, st, _ = oracle.gated_delta_f64(q, k, v, a, b, np.zeros_like(A_log), np.zeros_like(dt), s0)
    np.testing.assert_array_equal(st, s0.astype(np.float64))
    for t in range(q.shape[1]):
        for hv in range(4):
            np.testing.assert_allclose(y[0, t, hv], s0[0, hv].astype(np.float64) @ q[0, t, hv // 2], rtol=1e-12)


def test_unit_beta_writes_value():
    # g = 1, beta = 1, |k| = 1  =>  S_new k = v  (delta rule)
    q, k, v, a, b, A_log, dt, s0 = small(T=1, seed=2)
    a[:] = -1000.0
    b[:] = 1000.0
    _, st, _ = oracle.gated_delta_f64(q, k, v, a, b, np.zeros_like(A_log), np.zeros_like(dt), s0)
    for hv in range(4):
        # |k| = 1 holds to fp32 precision only
        np.testing.assert_allclose(st[0, hv] @ k[0, 0, hv // 2].astype(np.float64), v[0, 0, hv], atol=1e-6)


def test_t_steps_equal_single_steps():
    args = small(T=6, seed=3)
    q, k, v, a, b, A_log, dt, s0 = args
    y, st, sn = oracle.gated_delta_f64(*args)
    s = s0.astype(np.float64)
    for t in range(6):
        yt, s, _ = oracle.gated_delta_f64(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], a[:, t:t + 1],
                                          b[:, t:t + 1], A_log, dt, s)
        np.testing.assert_allclose(yt[:, 0], y[:, t], rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(s, sn[t], rtol=1e-12, atol=1e-14)


def test_softplus_threshold_branch():
    # x > 20 takes softplus(x) = x (engine/kernels.py:37)
    q, k, v, a, b, A_log, dt, s0 = small(T=1, seed=4)
    a[:] = 25.0
    A_log[:] = -5.0
    y1, st1, _ = oracle.gated_delta_f64(q, k, v, a, b, A_log, np.zeros_like(dt), s0)
    ym, Sm = matrix_form(q, k, v, a, b, A_log, np.zeros_like(dt), s0)
    np.testing.assert_allclose(st1, Sm, rtol=1e-12)


def test_f32_baseline_close_to_f64():
    inp = synth.gdn_inputs(5, Hk=4, Hv=8)
    f = lambda x: synth.bf16_to_f32(x)
    args = (f(inp["q"]), f(inp["k"]), f(inp["v"]), f(inp["a"]), f(inp["b"]), inp["A_log"],
            f(inp["dt_bias"]), inp["state"])
    y64, s64, _ = oracle.gated_delta_f64(*args)
    y32, s32, _ = oracle.gated_delta_f32(*args, threads=2)
    np.testing.assert_allclose(y32, y64, atol=1e-5)
    np.testing.assert_allclose(s32, s64, atol=1e-5)
