"""Fused cycle inputs (GPU): each launch equals, bit for bit, the launches it replaces.

qvex_mtp_input: the MTP head's input x = [rms(embed(tok)) * w_emb | rms(h) * w_hid]
(engine/mtp.py:61-63) against qvex_embed_w4g64 + qvex_rmsnorm_pair; the token
from a deferred lm_head argmax against qvex_qmv_w4g64_packed_argmax's own
reduction; the folded counter advance against qvex_commit_step.
qvex_embed_rms_parts: the verify rows' embedding and first-norm inputs
(engine/model.py:126-130, 309-310) against qvex_embed_w4g64 + qvex_rms_parts, with
and without the last draft's argmax folded in.
"""

import numpy as np
import pytest
import torch

from qvex import _C, kernels, synth
from qvex.kernels import _ptr, _stream
from qvex.model import QEmbedding, _rand_qlinear

DEV = "cuda:0"
EPS = 1e-6


def same(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def embedding(V, H, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    q = _rand_qlinear(V, H, g, 0.05, DEV, pack=False)
    return QEmbedding(q.w, q.scales, q.biases)


def weights(H, seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(DEV)


def rmsnorm_pair(emb, ids, w_emb, hid, w_hid, H):
    e = emb(ids)
    T = ids.numel()
    x_in = torch.empty((T, 2 * H), dtype=torch.bfloat16, device=DEV)
    _C.call("qvex_rmsnorm_pair", _ptr(e), e.stride(0), _ptr(w_emb), _ptr(x_in), _ptr(hid), hid.stride(0),
            _ptr(w_hid), _ptr(x_in) + 2 * H, x_in.stride(0), T, H, float(EPS), _stream())
    return x_in


def lm_head_pairs(V, H, M, seed):
    """A packed lm_head and the deferred argmax pairs of M normed rows, plus the
    tokens its own reduction gives."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    lm = _rand_qlinear(V, H, g, 0.5 / np.sqrt(21.25 * H), DEV)
    x = torch.randn(M, H, generator=g, device=DEV).to(torch.bfloat16)
    nw = weights(H, seed + 1)
    u, parts = kernels.rms_parts(x, nw)
    tok = torch.empty(M, dtype=torch.int32, device=DEV)
    kernels.qmv_packed_argmax(u, lm.packed, V, tok, parts, EPS)
    ws = torch.empty(int(_C.lib().qvex_qmv_w4g64_argmax_workspace_bytes(M, V)) // 4, dtype=torch.float32,
                     device=DEV)
    am = kernels.qmv_packed_argmax(u, lm.packed, V, None, parts, EPS, workspace=ws)
    return am, tok


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 2, 4, 5, 12])
@pytest.mark.parametrize("V,H", [(2048, 512), (4096, 4096)])
def test_mtp_input_equals_embed_and_norm_pair(T, V, H):
    emb = embedding(V, H, 7 + T)
    ids = torch.randint(0, V, (T,), dtype=torch.int32, device=DEV)
    ids[0] = V + 5                                   # clamped, as the gather clamps
    hid = torch.randn(T + 3, H, device=DEV).to(torch.bfloat16)
    w_emb, w_hid = weights(H, 1), weights(H, 2)
    ref = rmsnorm_pair(emb, ids, w_emb, hid[:T], w_hid, H)
    x_in = torch.empty((T, 2 * H), dtype=torch.bfloat16, device=DEV)
    kernels.mtp_input(emb, ids, T, w_emb, hid[:T], w_hid, EPS, x_in)
    torch.cuda.synchronize()
    assert same(x_in, ref)
    # hidden row chosen on the device
    sel = torch.tensor([T + 1], dtype=torch.int32, device=DEV)
    ref_sel = rmsnorm_pair(emb, ids[:1], w_emb, hid[T + 1:T + 2], w_hid, H)
    x1 = torch.empty((1, 2 * H), dtype=torch.bfloat16, device=DEV)
    kernels.mtp_input(emb, ids[:1].contiguous(), 1, w_emb, hid, w_hid, EPS, x1, hid_sel=sel)
    torch.cuda.synchronize()
    assert same(x1, ref_sel)


@pytest.mark.gpu
@pytest.mark.parametrize("M,row", [(1, None), (4, 0), (4, 3)])
def test_mtp_input_argmax_and_commit(M, row):
    V, H = 248320, 4096
    am, tok = lm_head_pairs(V, H, M, 31 + M)
    emb = embedding(V, H, 3)
    hid = torch.randn(M, H, device=DEV).to(torch.bfloat16)
    w_emb, w_hid = weights(H, 4), weights(H, 5)
    r = 0 if row is None else row
    am_row = None if row is None else torch.tensor([row], dtype=torch.int32, device=DEV)
    ids_out = torch.full((2,), -7, dtype=torch.int32, device=DEV)
    counters = torch.tensor([100, 3], dtype=torch.int32, device=DEV)
    n_acc = torch.tensor([2], dtype=torch.int32, device=DEV)
    x_in = torch.empty((1, 2 * H), dtype=torch.bfloat16, device=DEV)
    kernels.mtp_input(emb, None, 1, w_emb, hid, w_hid, EPS, x_in, hid_sel=am_row, am=am, am_row=am_row,
                      ids_out=ids_out[1:], counters=counters, n_accept=n_acc, extra=1)
    torch.cuda.synchronize()
    assert int(ids_out[1]) == int(tok[r])
    assert int(ids_out[0]) == -7
    assert counters.tolist() == [103, 6]
    ref = rmsnorm_pair(emb, tok[r:r + 1].contiguous(), w_emb, hid[r:r + 1], w_hid, H)
    assert same(x_in, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("L", [1, 4, 5, 8])
@pytest.mark.parametrize("V,H", [(2048, 512), (4096, 4096)])
def test_embed_rms_parts_equals_two_launches(L, V, H):
    emb = embedding(V, H, 11 + L)
    ids = torch.randint(0, V, (L,), dtype=torch.int32, device=DEV)
    nw = weights(H, 9)
    x_ref = emb(ids)
    u_ref, p_ref = kernels.rms_parts(x_ref, nw)
    h, u, parts = kernels.embed_rms_parts(emb, ids, nw)
    torch.cuda.synchronize()
    assert same(h, x_ref) and same(u, u_ref)
    assert torch.equal(parts.view(torch.int32), p_ref.view(torch.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("M,row", [(1, None), (4, 2)])
def test_embed_rms_parts_with_last_draft(M, row):
    V, H = 248320, 4096
    am, tok = lm_head_pairs(V, H, M, 57 + M)
    emb = embedding(V, H, 13)
    nw = weights(H, 10)
    r = 0 if row is None else row
    am_row = None if row is None else torch.tensor([row], dtype=torch.int32, device=DEV)
    ids = torch.tensor([5, 17, 123, -1], dtype=torch.int32, device=DEV)
    h, u, parts = kernels.embed_rms_parts(emb, ids, nw, am=am, am_row=am_row, am_slot=3)
    torch.cuda.synchronize()
    assert ids.tolist()[:3] == [5, 17, 123] and int(ids[3]) == int(tok[r])
    x_ref = emb(ids)
    u_ref, p_ref = kernels.rms_parts(x_ref, nw)
    torch.cuda.synchronize()
    assert same(h, x_ref) and same(u, u_ref)
    assert torch.equal(parts.view(torch.int32), p_ref.view(torch.int32))
