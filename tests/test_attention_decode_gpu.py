"""The fused decode attention step (qvex_attention_decode: q/k RMSNorm, partial
RoPE and the cache append inside the split kernel, engine/model.py:213-232)
against float64 restatements, and against the two-launch path
(qvex_attn_qk_rope + qvex_attention) on the same inputs (GPU).

Cases: 1..8 new tokens, both head sizes, GQA 4 and 2, new keys straddling a
split boundary, an empty history, two query tiles (L = 8 at GQA 4), and a grid
sized for the whole capacity (what a captured graph launches).

Tolerances: the new cache keys as in test_qk_rope_gpu (normalised dims within
one bf16 step, rotated dims within 2^-7 of their pair's norm), V and the old
keys bit for bit; outputs within 1.5e-2 absolute of a float64 attention over
the keys the kernel wrote and the float64 normed, rotated queries (bf16 P and
output rounding as in test_attention_gpu), scaled by the largest visible |v| / 4
(the new V rows here are twice unit scale), and within the same bound of the
two-launch path."""

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import round_bf16
from qvex import _C
from qvex.kernels import _ptr, _stream, kv_tile_k, kv_tile_v, kv_untile_k, kv_untile_v
from qvex.model import rope_table

DEV = "cuda:0"


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)


def tof(t):
    return t.float().cpu().numpy()


def rope64(x, pos0, dims, base):
    """NeoX rotation of the first `dims` dims of x [heads, L, D] at positions
    pos0 + l, in float64 complex form; also each value's pair norm."""
    half = dims // 2
    L = x.shape[1]
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:dims].astype(np.float64)
    theta = np.exp(-np.log(base) * (2.0 * np.arange(half) / dims))
    zr = z * np.exp(1j * (pos0 + np.arange(L))[:, None] * theta[None, :])[None]
    y = x.astype(np.float64).copy()
    y[..., :half], y[..., half:dims] = zr.real, zr.imag
    pair = np.abs(x.astype(np.float64))
    pair[..., :half] = pair[..., half:dims] = np.abs(z)
    return y, pair


def workspace(L, Hq, Hkv, D, max_keys, kps):
    need = int(_C.lib().qvex_attn_workspace_bytes(L, Hq, Hkv, D, max_keys, kps))
    return torch.empty((need + 3) // 4, dtype=torch.float32, device=DEV)


CASES = [
    (4, 16, 4, 256, 64, 4348, 0), (1, 16, 4, 256, 64, 700, 0), (4, 16, 4, 256, 64, 126, 0),
    (8, 16, 4, 256, 64, 1020, 0), (4, 16, 4, 256, 64, 0, 0), (3, 4, 2, 128, 32, 31, 0),
    (8, 4, 2, 128, 64, 77, 0), (2, 8, 2, 128, 32, 129, 0), (5, 16, 4, 256, 64, 250, 0),
    (4, 16, 4, 256, 64, 1000, 2048), (1, 16, 4, 256, 64, 4095, 1024)]


@pytest.mark.gpu
@pytest.mark.parametrize("L,Hq,Hkv,D,rot,pos0,spare", CASES)
def test_attention_decode(L, Hq, Hkv, D, rot, pos0, spare):
    g = np.random.default_rng(L * 131 + pos0 + D)
    cap = ((pos0 + L + spare + 255) // 256) * 256
    width = Hq * 2 * D + 2 * Hkv * D
    proj = round_bf16(g.standard_normal((L, width)).astype(np.float32) * 2.0)
    qn = round_bf16(1 + 0.1 * g.standard_normal(D).astype(np.float32))
    kn = round_bf16(1 + 0.1 * g.standard_normal(D).astype(np.float32))
    hist_k = round_bf16(g.standard_normal((Hkv, cap, D)).astype(np.float32))
    hist_v = round_bf16(g.standard_normal((Hkv, cap, D)).astype(np.float32))
    eps, theta = 1e-6, 1e7
    kps = 128
    max_keys = cap if spare else pos0 + L
    pt, qnt, knt = bf(proj), bf(qn), bf(kn)
    pos = torch.tensor([pos0], dtype=torch.int32, device=DEV)

    # fused path
    kc, vc = kv_tile_k(bf(hist_k)), kv_tile_v(bf(hist_v))
    out = torch.empty((L, Hq * D), dtype=torch.bfloat16, device=DEV)
    ws = workspace(L, Hq, Hkv, D, max_keys, kps)
    tab = rope_table(rot, theta, cap, DEV)
    _C.call("qvex_attention_decode", _ptr(pt), pt.stride(0), _ptr(qnt), _ptr(knt), _ptr(pos), L, Hq, Hkv, D, rot,
            eps, _ptr(tab), tab.shape[0], _ptr(kc), _ptr(vc), cap, max_keys, kps, _ptr(out), _ptr(ws),
            ws.numel() * 4, _stream())
    # two-launch path on copies of the same caches
    kc2, vc2 = kv_tile_k(bf(hist_k)), kv_tile_v(bf(hist_v))
    q2 = torch.empty((L, Hq, D), dtype=torch.bfloat16, device=DEV)
    out2 = torch.empty((L, Hq * D), dtype=torch.bfloat16, device=DEV)
    ws2 = workspace(L, Hq, Hkv, D, max_keys, kps)
    _C.call("qvex_attn_qk_rope", _ptr(pt), pt.stride(0), _ptr(qnt), _ptr(knt), _ptr(pos), L, Hq, Hkv, D, rot,
            theta, eps, _ptr(q2), _ptr(kc2), _ptr(vc2), cap, 0, 0, _stream())
    _C.call("qvex_attention", _ptr(q2), _ptr(kc2), _ptr(vc2), _ptr(pos), L, Hq, Hkv, D, cap, max_keys, max_keys, kps,
            _ptr(pt), pt.stride(0), _ptr(out2), _ptr(ws2), ws2.numel() * 4, _stream())
    torch.cuda.synchronize()

    keys, vals = tof(kv_untile_k(kc)), tof(kv_untile_v(vc))
    new = slice(pos0, pos0 + L)
    # the cache outside this call's keys is untouched; V is copied bit for bit
    np.testing.assert_array_equal(keys[:, :pos0], hist_k[:, :pos0])
    np.testing.assert_array_equal(keys[:, pos0 + L:], hist_k[:, pos0 + L:])
    np.testing.assert_array_equal(vals[:, :pos0], hist_v[:, :pos0])
    np.testing.assert_array_equal(vals[:, pos0 + L:], hist_v[:, pos0 + L:])
    v_new = proj[:, Hq * 2 * D + Hkv * D:].reshape(L, Hkv, D)
    np.testing.assert_array_equal(vals[:, new].transpose(1, 0, 2), v_new)
    # new keys: normed and rotated
    k_raw = proj[:, Hq * 2 * D:Hq * 2 * D + Hkv * D].reshape(L, Hkv, D)
    n = om.rms_norm(k_raw, kn, eps)                                  # [L, Hkv, D]
    ref, pair = rope64(n.transpose(1, 0, 2), pos0, rot, theta)       # [Hkv, L, D]
    got = keys[:, new]
    tail = np.abs(got[..., rot:] - n.transpose(1, 0, 2)[..., rot:])
    assert np.all(tail <= 2.0 ** -8 * np.abs(n.transpose(1, 0, 2)[..., rot:]) + 1e-30), "k: normalised dims"
    err = np.abs(got[..., :rot] - ref[..., :rot]) / pair[..., :rot]
    assert np.all(err <= 2.0 ** -7), f"k: rotated dims, worst {err.max():.3e} of the pair norm"

    # attention over the keys the kernel wrote, queries normed and rotated in float64
    q_raw = proj[:, :Hq * 2 * D].reshape(L, Hq, 2 * D)[..., :D]
    qnorm = om.rms_norm(q_raw, qn, eps)
    qref, _ = rope64(qnorm.transpose(1, 0, 2), pos0, rot, theta)     # [Hq, L, D]
    gate = proj[:, :Hq * 2 * D].reshape(L, Hq, 2 * D)[..., D:].astype(np.float64)
    kf, vf = keys.astype(np.float64), vals.astype(np.float64)
    want = np.zeros((L, Hq, D))
    for h in range(Hq):
        kh = h // (Hq // Hkv)
        for l in range(L):
            nk = pos0 + l + 1
            s = kf[kh, :nk] @ qref[h, l] / np.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            want[l, h] = (p @ vf[kh, :nk]) / (1 + np.exp(-gate[l, h]))
    have = tof(out).reshape(L, Hq, D)
    err_ref = np.abs(have - want).max()
    err_two = np.abs(have - tof(out2).reshape(L, Hq, D)).max()
    # the bf16 rounding of P scales with the values: the bar of test_attention_gpu
    # (unit-normal V, |v| < ~4) scaled by the largest visible |v| (the new rows are 2x)
    tol = 1.5e-2 * max(1.0, float(np.abs(vf[:, :pos0 + L]).max()) / 4.0)
    print(f"L={L} Hq={Hq} Hkv={Hkv} D={D} pos={pos0}: max abs err {err_ref:.4f} vs float64, "
          f"{err_two:.4f} vs the two-launch path (tolerance {tol:.4f})")
    assert err_ref < tol
    assert err_two < tol
