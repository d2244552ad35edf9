"""q/k RMSNorm + partial RoPE + KV append (qvex_attn_qk_rope) against the
oracle's rms_norm and a float64 complex-rotation RoPE (engine/model.py:218-226,
mx.fast.rope with traditional=False), at large positions and for rotary
widths whose half is not a power of two (GPU).

Tolerances: the normalised values within one bf16 step; rotated values within
2^-7 of their pair's norm (fp32 sincos of angles up to ~8k rad, then one bf16
rounding); V copied bit for bit."""

import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import round_bf16
from qvex import _C
from qvex.kernels import _ptr, _stream, kv_untile_k, kv_untile_v

DEV = "cuda:0"


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)


def tof(t):
    return t.float().cpu().numpy()


def rope64(x, pos0, dims, base):
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


def run_qk_rope(pt, qnt, knt, L, Hq, Hkv, D, rot, pos0, cap, theta, eps, table_rows=0):
    """One qvex_attn_qk_rope call into fresh tiled caches; with table_rows > 0 the
    angles come from a qvex_rope_table of that many positions."""
    q_out = torch.empty((L, Hq, D), dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros((Hkv, cap // 16, D // 32, 64, 8), dtype=torch.bfloat16, device=DEV)   # tiled caches
    vc = torch.zeros((Hkv, cap // 32, D, 32), dtype=torch.bfloat16, device=DEV)
    pos = torch.tensor([pos0], dtype=torch.int32, device=DEV)
    tab = None
    if table_rows:
        tab = torch.empty((table_rows, rot // 2, 2), dtype=torch.float32, device=DEV)
        _C.call("qvex_rope_table", rot, theta, table_rows, _ptr(tab), _stream())
    _C.call("qvex_attn_qk_rope", _ptr(pt), pt.stride(0), _ptr(qnt), _ptr(knt), _ptr(pos), L, Hq, Hkv, D, rot,
            theta, eps, _ptr(q_out), _ptr(kc), _ptr(vc), cap, _ptr(tab) if tab is not None else 0, table_rows,
            _stream())
    torch.cuda.synchronize()
    return q_out, kc, vc


@pytest.mark.gpu
@pytest.mark.parametrize("L,Hq,Hkv,D,rot,pos0", [
    (4, 16, 4, 256, 64, 4348), (1, 16, 4, 256, 64, 8000), (5, 4, 2, 128, 48, 777), (3, 4, 2, 256, 48, 6001),
    (2, 4, 2, 128, 32, 0), (4, 8, 2, 128, 40, 123)])
@pytest.mark.parametrize("table", [False, True])
def test_qk_rope_matches_fp64(L, Hq, Hkv, D, rot, pos0, table):
    g = np.random.default_rng(L * 97 + rot + pos0)
    cap = ((pos0 + L + 255) // 256) * 256
    width = Hq * 2 * D + 2 * Hkv * D
    proj = round_bf16(g.standard_normal((L, width)).astype(np.float32) * 2.0)
    qn = round_bf16(1 + 0.1 * g.standard_normal(D).astype(np.float32))
    kn = round_bf16(1 + 0.1 * g.standard_normal(D).astype(np.float32))
    eps, theta = 1e-6, 1e7
    pt, qnt, knt = bf(proj), bf(qn), bf(kn)          # held: the kernel runs after this line
    q_out, kc, vc = run_qk_rope(pt, qnt, knt, L, Hq, Hkv, D, rot, pos0, cap, theta, eps, cap if table else 0)
    qg = proj[:, :Hq * 2 * D].reshape(L, Hq, 2 * D)[..., :D]
    k = proj[:, Hq * 2 * D:Hq * 2 * D + Hkv * D].reshape(L, Hkv, D)
    v = proj[:, Hq * 2 * D + Hkv * D:].reshape(L, Hkv, D)
    worst = 0.0
    for name, x, w, got in (("q", qg, qn, tof(q_out)),
                            ("k", k, kn, tof(kv_untile_k(kc))[:, pos0:pos0 + L].transpose(1, 0, 2))):
        n = om.rms_norm(x, w, eps)                                   # [L, heads, D] bf16 values
        ref, pair = rope64(n.transpose(1, 0, 2), pos0, rot, theta)
        ref, pair = ref.transpose(1, 0, 2), pair.transpose(1, 0, 2)
        tail = np.abs(got[..., rot:] - n[..., rot:])
        assert np.all(tail <= 2.0 ** -8 * np.abs(n[..., rot:]) + 1e-30), f"{name}: normalised dims"
        err = np.abs(got[..., :rot] - ref[..., :rot]) / pair[..., :rot]
        worst = max(worst, float(err.max()))
        assert np.all(err <= 2.0 ** -7), f"{name}: rotated dims, worst {err.max():.3e} of the pair norm"
    np.testing.assert_array_equal(tof(kv_untile_v(vc))[:, pos0:pos0 + L].transpose(1, 0, 2), v)
    print(f"L={L} D={D} rot={rot} pos={pos0}: worst rotated error {worst:.3e} of the pair norm")


@pytest.mark.gpu
@pytest.mark.parametrize("L,Hq,Hkv,D,rot,pos0,rows", [
    (4, 16, 4, 256, 64, 4348, 4608),      # the 9B verify shape, table covering the cache
    (5, 4, 2, 128, 48, 777, 780),         # positions 780, 781 past the table: evaluated
    (3, 4, 2, 128, 32, 0, 1)])            # only position 0 in the table
def test_qk_rope_table_equals_evaluated(L, Hq, Hkv, D, rot, pos0, rows):
    """The table path loads the (cos, sin) pairs the kernel would evaluate:
    q, the appended keys and values are bit-identical to the evaluated path."""
    g = np.random.default_rng(rows + rot)
    cap = ((pos0 + L + 255) // 256) * 256
    width = Hq * 2 * D + 2 * Hkv * D
    pt = bf(round_bf16(g.standard_normal((L, width)).astype(np.float32) * 2.0))
    qnt = bf(round_bf16(1 + 0.1 * g.standard_normal(D).astype(np.float32)))
    knt = bf(round_bf16(1 + 0.1 * g.standard_normal(D).astype(np.float32)))
    a = run_qk_rope(pt, qnt, knt, L, Hq, Hkv, D, rot, pos0, cap, 1e7, 1e-6, 0)
    b = run_qk_rope(pt, qnt, knt, L, Hq, Hkv, D, rot, pos0, cap, 1e7, 1e-6, rows)
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
