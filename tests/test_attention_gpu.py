"""Verify attention kernel (qvex_attention) vs a float64 causal GQA softmax
attention times sigmoid(gate) (GPU). Tolerance: 1.5e-2 absolute on outputs of
order 1 (bf16 P and output rounding; 7.7e-3 is the largest error measured on
MI355X)."""

import numpy as np
import pytest
import torch

from qvex import _C
from qvex.kernels import _ptr, _stream, kv_tile_k, kv_tile_v

DEV = "cuda:0"


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)


def tof(t):
    return t.float().cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("L,Hq,Hkv,D,pos0,kps,spare", [
    (4, 16, 4, 256, 4348, 128, 0), (1, 16, 4, 256, 700, 128, 0), (4, 16, 4, 256, 0, 128, 0),
    (64, 16, 4, 256, 300, 512, 0), (4, 16, 4, 256, 4348, 512, 0), (8, 4, 2, 128, 77, 128, 0),
    (3, 4, 2, 128, 31, 256, 0),
    # graph-mode sizing: max_keys = capacity, far past the visible keys
    (4, 16, 4, 256, 1000, 128, 2048), (2, 4, 2, 128, 129, 128, 1024)])
def test_attention_matches_reference(L, Hq, Hkv, D, pos0, kps, spare):
    g = np.random.default_rng(L * 1000 + pos0)
    cap = ((pos0 + L + spare + 255) // 256) * 256
    q = g.standard_normal((L, Hq, D)).astype(np.float32)
    kc = g.standard_normal((Hkv, cap, D)).astype(np.float32)
    vc = g.standard_normal((Hkv, cap, D)).astype(np.float32)
    gate_rows = g.standard_normal((L, Hq, 2 * D)).astype(np.float32)
    qt, kt = bf(q), kv_tile_k(bf(kc))                              # tiled caches
    vt = kv_tile_v(bf(vc))
    gt = bf(gate_rows.reshape(L, -1))
    pos = torch.tensor([pos0], dtype=torch.int32, device=DEV)
    out = torch.empty((L, Hq * D), dtype=torch.bfloat16, device=DEV)
    max_keys = cap if spare else pos0 + L
    known = pos0 if spare else max_keys     # graph sizing: splits past the position read it first
    need = int(_C.lib().qvex_attn_workspace_bytes(L, Hq, Hkv, D, max_keys, kps))
    ws = torch.empty((need + 3) // 4, dtype=torch.float32, device=DEV)
    _C.call("qvex_attention", _ptr(qt), _ptr(kt), _ptr(vt), _ptr(pos), L, Hq, Hkv, D, cap, max_keys, known, kps,
            _ptr(gt), gt.stride(0), _ptr(out), _ptr(ws), ws.numel() * 4, _stream())
    torch.cuda.synchronize()
    qf, kf = tof(qt).astype(np.float64), tof(bf(kc)).astype(np.float64)
    vf = tof(bf(vc)).astype(np.float64)
    gf = tof(gt).astype(np.float64).reshape(L, Hq, 2 * D)[..., D:]
    ref = np.zeros((L, Hq, D))
    for h in range(Hq):
        kh = h // (Hq // Hkv)
        for l in range(L):
            n = pos0 + l + 1
            s = kf[kh, :n] @ qf[l, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            ref[l, h] = (p @ vf[kh, :n]) / (1 + np.exp(-gf[l, h]))
    got = tof(out).reshape(L, Hq, D)
    err = np.abs(got - ref).max()
    print(f"max abs err {err:.4f}")
    assert err < 1.5e-2
