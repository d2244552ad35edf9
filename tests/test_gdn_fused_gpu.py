"""Fused GDN decode mixer (qvex_gdn_decode_fused) vs the three-kernel path
(qvex_gdn_conv_qk -> qvex_gdn_recurrent_ring -> qvex_gated_rmsnorm) (GPU).

The fused kernel keeps every rounding and reduction order of the three
kernels, so the out_proj input, the conv ring and the state ring must agree
bit for bit, for every token count 1..8, GQA ratio, ring position (including
wrap-around of both rings) and with or without per-token snapshots. The three
kernels themselves are pinned against the oracle by the GDN and model tests.
"""

import numpy as np
import pytest
import torch

from qvex import _C

DEV = "cuda:0"
KC = 4


def ptr(t):
    return t.data_ptr()


def make(T, Hk, Hv, counter, seed, max_width=8):
    g = torch.Generator().manual_seed(seed)
    key_dim, value_dim = Hk * 128, Hv * 128
    C = 2 * key_dim + value_dim
    p_stride = C + value_dim + 2 * Hv + 6          # padded row, as a fused projection may be
    R = max(max_width, 64) + KC - 1
    n_slots = max_width + 1
    d = dict(T=T, Hk=Hk, Hv=Hv, C=C, key_dim=key_dim, value_dim=value_dim, p_stride=p_stride, R=R,
             n_slots=n_slots)
    d["proj"] = (torch.randn(T, p_stride, generator=g) * 1.5).to(torch.bfloat16).to(DEV)
    d["ring"] = torch.randn(R, C, generator=g).to(torch.bfloat16).to(DEV)
    d["cw"] = (torch.randn(C, KC, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    d["A_log"] = (torch.rand(Hv, generator=g) * 2 - 1).float().to(DEV)
    d["dt_bias"] = torch.randn(Hv, generator=g).to(torch.bfloat16).to(DEV)
    d["state"] = (torch.randn(n_slots, 1, Hv, 128, 128, generator=g) * 0.1).float().to(DEV)
    d["norm_w"] = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV)
    d["counter"] = torch.tensor([counter], dtype=torch.int32, device=DEV)
    return d


def run_unfused(d, ring, state, snap):
    T, Hk, Hv, C = d["T"], d["Hk"], d["Hv"], d["C"]
    kd, vd = d["key_dim"], d["value_dim"]
    inv = 128 ** -0.5
    q = torch.empty(T, kd, dtype=torch.bfloat16, device=DEV)
    k = torch.empty_like(q)
    v = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    a = torch.empty(T, Hv, dtype=torch.bfloat16, device=DEV)
    b = torch.empty_like(a)
    y = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    s = 0
    _C.call("qvex_gdn_conv_qk", ptr(d["proj"]), d["p_stride"], ptr(ring), d["R"], ptr(d["counter"]), ptr(d["cw"]),
            KC, ptr(q), ptr(k), ptr(v), ptr(a), ptr(b), T, C, kd, Hv, C + vd, inv * inv, inv, 1e-6, s)
    _C.call("qvex_gdn_recurrent_ring", ptr(q), ptr(k), ptr(v), ptr(a), ptr(b), ptr(d["A_log"]), ptr(d["dt_bias"]),
            ptr(state), d["n_slots"], ptr(d["counter"]), int(snap), ptr(y), 1, T, Hk, Hv, 128, 128, s)
    _C.call("qvex_gated_rmsnorm", ptr(y), ptr(d["proj"]) + 2 * C, d["p_stride"], Hv, ptr(d["norm_w"]), ptr(out),
            T * Hv, 128, 1e-6, s)
    return out


def run_fused(d, ring, state, snap):
    T, Hk, Hv, C = d["T"], d["Hk"], d["Hv"], d["C"]
    kd, vd = d["key_dim"], d["value_dim"]
    inv = 128 ** -0.5
    out = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    _C.call("qvex_gdn_decode_fused", ptr(d["proj"]), d["p_stride"], ptr(ring), d["R"], ptr(d["counter"]),
            ptr(d["cw"]), KC, C, kd, inv * inv, inv, 1e-6, ptr(d["A_log"]), ptr(d["dt_bias"]), C, C + vd,
            ptr(state), d["n_slots"], int(snap), ptr(d["norm_w"]), 1e-6, ptr(out), T, Hk, Hv, 128, 128, 0)
    return out


def bits_equal(a, b):
    return torch.equal(a.contiguous().view(torch.int16 if a.element_size() == 2 else torch.int32),
                       b.contiguous().view(torch.int16 if b.element_size() == 2 else torch.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("Hk,Hv", [(2, 4), (4, 4), (2, 8)])
@pytest.mark.parametrize("counter", [0, 6, 1001])
def test_fused_equals_three_kernels(T, Hk, Hv, counter):
    d = make(T, Hk, Hv, counter, seed=T * 100 + Hv * 10 + Hk + counter)
    r1, r2 = d["ring"].clone(), d["ring"].clone()
    s1, s2 = d["state"].clone(), d["state"].clone()
    o1 = run_unfused(d, r1, s1, snap=True)
    o2 = run_fused(d, r2, s2, snap=True)
    torch.cuda.synchronize()
    assert bits_equal(o1, o2), f"out differs: max {float((o1.float() - o2.float()).abs().max())}"
    assert bits_equal(r1, r2), "conv ring differs"
    assert bits_equal(s1, s2), "state ring differs"


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 4])
def test_fused_without_snapshots(T):
    """snap_every = 0: only the last token's state is written (slot c + T)."""
    d = make(T, 2, 4, counter=3, seed=55 + T)
    r1, r2 = d["ring"].clone(), d["ring"].clone()
    s1, s2 = d["state"].clone(), d["state"].clone()
    o1 = run_unfused(d, r1, s1, snap=False)
    o2 = run_fused(d, r2, s2, snap=False)
    torch.cuda.synchronize()
    assert bits_equal(o1, o2) and bits_equal(r1, r2) and bits_equal(s1, s2)


@pytest.mark.gpu
def test_fused_qwen35_9b_shape():
    """Hk = 16, Hv = 32 (the 9B layer), verify width 4."""
    d = make(4, 16, 32, counter=4099, seed=9)
    r1, r2 = d["ring"].clone(), d["ring"].clone()
    s1, s2 = d["state"].clone(), d["state"].clone()
    o1 = run_unfused(d, r1, s1, snap=True)
    o2 = run_fused(d, r2, s2, snap=True)
    torch.cuda.synchronize()
    assert bits_equal(o1, o2) and bits_equal(r1, r2) and bits_equal(s1, s2)
    assert np.isfinite(o2.float().cpu().numpy()).all()


# ---------------------------------------------------------------- split mixer + out_proj with the head scale
#
# qvex_gdn_decode_split leaves the gated norm's per-head scale to the out_proj
# (qvex_qmv_w4g64_packed_gnorm_resid). Its conv and state rings must equal the
# fused kernel's bit for bit; its outputs are pinned against the three-kernel
# path's recurrence output y: u = bf16(silu(z) * (w * y)) within one bf16 step
# (torch's exp against the kernel's), and each workgroup's sum of y^2 over its
# rows to fp32 rounding. The product is pinned in float64 against
# sum_h rsqrt(S_h / 128 + eps) * (u_h W_h^T), S_h summed from y directly.

def run_three(d, ring, state, snap):
    """The three-kernel path; returns (gated-norm output, recurrence output y)."""
    T, Hk, Hv, C = d["T"], d["Hk"], d["Hv"], d["C"]
    kd, vd = d["key_dim"], d["value_dim"]
    inv = 128 ** -0.5
    q = torch.empty(T, kd, dtype=torch.bfloat16, device=DEV)
    k = torch.empty_like(q)
    v = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    a = torch.empty(T, Hv, dtype=torch.bfloat16, device=DEV)
    b = torch.empty_like(a)
    y = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    _C.call("qvex_gdn_conv_qk", ptr(d["proj"]), d["p_stride"], ptr(ring), d["R"], ptr(d["counter"]), ptr(d["cw"]),
            KC, ptr(q), ptr(k), ptr(v), ptr(a), ptr(b), T, C, kd, Hv, C + vd, inv * inv, inv, 1e-6, 0)
    _C.call("qvex_gdn_recurrent_ring", ptr(q), ptr(k), ptr(v), ptr(a), ptr(b), ptr(d["A_log"]), ptr(d["dt_bias"]),
            ptr(state), d["n_slots"], ptr(d["counter"]), int(snap), ptr(y), 1, T, Hk, Hv, 128, 128, 0)
    _C.call("qvex_gated_rmsnorm", ptr(y), ptr(d["proj"]) + 2 * C, d["p_stride"], Hv, ptr(d["norm_w"]), ptr(out),
            T * Hv, 128, 1e-6, 0)
    return out, y


def run_split(d, ring, state, snap, nb):
    T, Hk, Hv, C = d["T"], d["Hk"], d["Hv"], d["C"]
    kd, vd = d["key_dim"], d["value_dim"]
    inv = 128 ** -0.5
    u = torch.empty(T, vd, dtype=torch.bfloat16, device=DEV)
    ss = torch.empty(T, Hv, nb, dtype=torch.float32, device=DEV)
    _C.call("qvex_gdn_decode_split", ptr(d["proj"]), d["p_stride"], ptr(ring), d["R"], ptr(d["counter"]),
            ptr(d["cw"]), KC, C, kd, inv * inv, inv, 1e-6, ptr(d["A_log"]), ptr(d["dt_bias"]), C, C + vd,
            ptr(state), d["n_slots"], int(snap), ptr(d["norm_w"]), ptr(u), ptr(ss), T, Hk, Hv, 128, 128, nb, 0)
    return u, ss


def check_split_outputs(d, u, ss, y, nb):
    T, Hv = d["T"], d["Hv"]
    vd = d["value_dim"]
    z = d["proj"][:, d["C"]:d["C"] + vd].float()
    w = d["norm_w"].float().repeat(Hv)
    u_ref = (z / (1 + torch.exp(-z)) * (w * y.float())).to(torch.bfloat16).float()
    err = (u.float() - u_ref).abs()
    assert bool((err <= 2.0 ** -7 * u_ref.abs() + 1e-30).all()), f"u differs by {float(err.max())}"
    yy = y.double().cpu().numpy().reshape(T, Hv, nb, 128 // nb)
    np.testing.assert_allclose(ss.cpu().numpy(), (yy ** 2).sum(-1), rtol=1e-5, atol=1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("Hk,Hv", [(2, 4), (2, 8)])
@pytest.mark.parametrize("nb", [2, 4, 8])
@pytest.mark.parametrize("counter", [0, 1001])
def test_split_rings_equal_fused(T, Hk, Hv, nb, counter):
    d = make(T, Hk, Hv, counter, seed=T * 100 + Hv * 10 + nb + counter)
    r1, r2, r3 = d["ring"].clone(), d["ring"].clone(), d["ring"].clone()
    s1, s2, s3 = d["state"].clone(), d["state"].clone(), d["state"].clone()
    run_fused(d, r1, s1, snap=True)
    u, ss = run_split(d, r2, s2, snap=True, nb=nb)
    _, y = run_three(d, r3, s3, snap=True)
    torch.cuda.synchronize()
    assert bits_equal(r1, r2), "conv ring differs"
    assert bits_equal(s1, s2), "state ring differs"
    check_split_outputs(d, u, ss, y, nb)


@pytest.mark.gpu
def test_split_without_snapshots():
    d = make(4, 2, 4, counter=3, seed=77)
    r1, r2 = d["ring"].clone(), d["ring"].clone()
    s1, s2 = d["state"].clone(), d["state"].clone()
    run_fused(d, r1, s1, snap=False)
    run_split(d, r2, s2, snap=False, nb=8)
    torch.cuda.synchronize()
    assert bits_equal(r1, r2) and bits_equal(s1, s2)


def _gnorm_case(T, Hk, Hv, nb, N, seed):
    from qvex import kernels, synth
    from test_norm_fusion_gpu import dequant
    from test_qmv_gpu import to_dev
    d = make(T, Hk, Hv, counter=11, seed=seed)
    K = d["value_dim"]
    u, ss = run_split(d, d["ring"].clone(), d["state"].clone(), snap=True, nb=nb)
    _, y = run_three(d, d["ring"].clone(), d["state"].clone(), snap=True)
    w, s, b = synth.qmv_weights(N, K, seed=seed, tag=N)
    packed = kernels.pack_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    return d, u, ss, y, packed, dequant(w, s, b)


@pytest.mark.gpu
@pytest.mark.parametrize("T,Hk,Hv,nb,N", [(1, 2, 4, 8, 1024), (4, 2, 4, 4, 1024), (3, 2, 8, 2, 512),
                                          (4, 16, 32, 8, 4096), (6, 2, 8, 4, 1024), (8, 16, 32, 4, 4096)])
def test_gnorm_out_proj_matches_float64(T, Hk, Hv, nb, N):
    from qvex import kernels
    d, u, ss, y, packed, W = _gnorm_case(T, Hk, Hv, nb, N, seed=T + Hv + N)
    K = d["value_dim"]
    zero = torch.zeros(T, N, dtype=torch.bfloat16, device=DEV)
    nw = torch.ones(N, dtype=torch.bfloat16, device=DEV)
    h, un, parts = kernels.qmv_packed_gnorm_resid(u, ss, packed, N, 1e-6, zero, nw)
    torch.cuda.synchronize()
    uu = u.double().cpu().numpy()
    yy = y.double().cpu().numpy().reshape(T, Hv, 128)
    rstd = 1.0 / np.sqrt((yy ** 2).sum(-1) / 128 + 1e-6)                   # [T, Hv]
    us = (uu.reshape(T, Hv, 128) * rstd[:, :, None]).reshape(T, K)
    ref = us @ W.T
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -13 * (np.abs(us) @ np.abs(W).T)
    err = np.abs(h.double().cpu().numpy() - ref)
    assert (err <= bound + 1e-6).all(), f"max excess {float((err - bound).max())}"
    # the epilogue: u = bf16(h * 1) = h, parts = sums of h^2 per 16 columns
    assert torch.equal(un.view(torch.int16), h.view(torch.int16))
    hh = h.double().cpu().numpy()
    np.testing.assert_allclose(parts.cpu().numpy(), (hh ** 2).reshape(T, -1, 16).sum(-1), rtol=1e-5, atol=1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [4, 7])
def test_gnorm_rows_independent_of_width(T):
    from qvex import kernels
    N = 1024
    d, u, ss, y, packed, W = _gnorm_case(T, 2, 8, 8, N, seed=5)
    g = torch.Generator().manual_seed(3)
    resid = torch.randn(T, N, generator=g).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(DEV)
    h, un, parts = kernels.qmv_packed_gnorm_resid(u, ss, packed, N, 1e-6, resid, nw)
    for r in range(T):
        h1, u1, p1 = kernels.qmv_packed_gnorm_resid(u[r:r + 1].contiguous(), ss[r:r + 1].contiguous(), packed, N,
                                                    1e-6, resid[r:r + 1].contiguous(), nw)
        torch.cuda.synchronize()
        assert torch.equal(h1.view(torch.int16), h[r:r + 1].view(torch.int16))
        assert torch.equal(u1.view(torch.int16), un[r:r + 1].view(torch.int16))
        assert torch.equal(p1, parts[r:r + 1])


@pytest.mark.gpu
def test_gnorm_close_to_fused_path():
    """out_proj(gated_rmsnorm(y, z)) through the fused mixer and the plain
    residual product, against the split mixer and the head-scaled product."""
    from qvex import kernels
    T, N = 4, 1024
    d, u, ss, y, packed, W = _gnorm_case(T, 2, 8, 8, N, seed=8)
    g_fused = run_fused(d, d["ring"].clone(), d["state"].clone(), snap=True)
    zero = torch.zeros(T, N, dtype=torch.bfloat16, device=DEV)
    nw = torch.ones(N, dtype=torch.bfloat16, device=DEV)
    h_a, _, _ = kernels.qmv_packed_resid(g_fused, packed, N, zero, nw)
    h_b, _, _ = kernels.qmv_packed_gnorm_resid(u, ss, packed, N, 1e-6, zero, nw)
    torch.cuda.synchronize()
    gg = g_fused.double().cpu().numpy()
    scale = np.abs(gg) @ np.abs(W).T                                     # sum_k |g_k W_nk|
    # inputs: g rounds twice, u once (2^-8 each, relative), plus exp: < 2^-6;
    # outputs: one rounding each
    ha, hb = h_a.double().cpu().numpy(), h_b.double().cpu().numpy()
    err = np.abs(ha - hb)
    bound = 2.0 ** -6 * scale + 2.0 ** -8 * (np.abs(ha) + np.abs(hb))
    assert (err <= bound + 1e-6).all(), f"max excess {float((err - bound).max())}"
