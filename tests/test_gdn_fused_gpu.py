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
