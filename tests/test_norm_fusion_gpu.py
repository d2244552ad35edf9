"""Residual RMSNorm folded into the neighbouring products (GPU).

Producer (qvex_qmv_w4g64_packed_resid): h = bf16(resid + delta) and
u = bf16(h * w) are bit-exact against the plain product followed by the same
bf16 arithmetic in torch; the per-16-column sums of h^2 match a float64 sum to
fp32 rounding (rel 1e-5). Consumer (qvex_qmv_w4g64_packed_rstd): the output
equals rsqrt(mean(h^2) + eps) * (u W^T) in float64 (u the kernel's own bf16
input, h the residual rows), i.e. rms_norm(h) W^T (engine/model.py:309-317 then
87-91) up to the rounding of u, within bf16 output rounding plus fp32
accumulation: |y - ref| <= 2^-8 |ref| + 2^-13 rstd sum_k |u_k| |W_nk|.
Model: the fused forward agrees with the unfused one within 0.1 on unit-scale
logits, and with itself bit for bit whatever the number of rows (rollback).
"""

import numpy as np
import pytest
import torch

from qvex import kernels, synth
from qvex.model import Config, NormedRows, random_model
from test_qmv_gpu import to_dev

DEV = "cuda:0"
EPS = 1e-6


def dequant(w, s, b):
    N, KW = w.shape
    K = KW * 8
    codes = np.stack([(w.astype(np.uint32) >> (4 * j)) & 0xF for j in range(8)], axis=-1).reshape(N, K)
    sc = np.repeat(synth.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bi = np.repeat(synth.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    return codes * sc + bi


def bf(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("N,K", [(4096, 12288), (512, 1024), (4096, 4096)])
def test_producer_epilogue(M, N, K):
    w, s, b = synth.qmv_weights(N, K, seed=41, tag=N)
    x = to_dev(synth.qmv_x(M, K, seed=41, tag=M), torch.bfloat16)
    g = torch.Generator().manual_seed(M + N)
    resid = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(DEV)
    packed = kernels.pack_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    delta = kernels.quantized_matmul_packed(x, packed, N)
    h, u, parts = kernels.qmv_packed_resid(x, packed, N, resid, nw)
    torch.cuda.synchronize()
    h_ref = (resid.float() + delta.float()).to(torch.bfloat16)
    u_ref = (h_ref.float() * nw.float()).to(torch.bfloat16)
    assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16))
    assert torch.equal(u.view(torch.int16), u_ref.view(torch.int16))
    p_ref = (bf(h_ref) ** 2).reshape(M, -1, 16).sum(-1)
    np.testing.assert_allclose(parts.cpu().numpy(), p_ref, rtol=1e-5, atol=1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3, 4, 6, 8])
@pytest.mark.parametrize("N,K,swiglu", [(12352, 4096, False), (24576, 4096, True), (1024, 512, False),
                                        (2048, 512, True)])
def test_consumer_scales_rows_by_rstd(M, N, K, swiglu):
    """y = bf16(rstd_r * (u W^T)) with rstd_r = rsqrt(sum_k h_k^2 / K + eps): float64
    reference from the kernel's own u, so a wrong scale, eps or row pairing fails."""
    w, s, b = synth.qmv_weights(N, K, seed=42, tag=N)
    g = torch.Generator().manual_seed(7 * M + K)
    hrow = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).to(DEV)
    st = NormedRows.of(hrow, nw, EPS)
    wd, sd, bd = to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16)
    packed = kernels.pack_w4(wd, sd, bd, swiglu=swiglu)
    y = kernels.qmv_packed_rstd(st.u, packed, N, st.parts, EPS, swiglu=swiglu)
    torch.cuda.synchronize()
    hh, uu = bf(hrow), bf(st.u)
    assert np.array_equal(uu, bf((hrow.float() * nw.float()).to(torch.bfloat16)))
    rstd = 1.0 / np.sqrt((hh ** 2).sum(-1, keepdims=True) / K + EPS)
    W = dequant(w, s, b)
    acc = rstd * (uu @ W.T)
    acc_err = 2.0 ** -13 * rstd * (np.abs(uu) @ np.abs(W).T)       # fp32 accumulation, rstd in fp32
    if not swiglu:
        ref, bound = acc, 2.0 ** -8 * np.abs(acc) + acc_err
    else:
        half = N // 2
        gt, up = acc[:, :half], acc[:, half:]
        dg = 2.0 ** -8 * np.abs(gt) + acc_err[:, :half]                # gate and up rounded to bf16
        du = 2.0 ** -8 * np.abs(up) + acc_err[:, half:]
        sg = gt / (1 + np.exp(-gt))
        ref = sg * up
        bound = 1.1 * (np.abs(up) + du) * dg + (np.abs(sg) + 1.1 * dg) * du + 2.0 ** -8 * np.abs(ref)
    err = np.abs(bf(y) - ref)
    assert (err <= bound + 1e-6).all(), f"max excess {float((err - bound).max())}"


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4, 8])
@pytest.mark.parametrize("N,K", [(248320, 4096), (1040, 512), (12352, 4096)])
def test_tile_max_epilogue(M, N, K):
    """The product with the tile-maxima epilogue writes the same logits bit for
    bit and, per row and 16-column tile, exactly their maximum (checked against
    numpy on the written logits and against the separate tile_max pass)."""
    w, s, b = synth.qmv_weights(N, K, seed=43, tag=N)
    g = torch.Generator().manual_seed(11 * M + K)
    hrow = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).to(DEV)
    st = NormedRows.of(hrow, nw, EPS)
    packed = kernels.pack_w4(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16))
    y0 = kernels.qmv_packed_rstd(st.u, packed, N, st.parts, EPS)
    tm = torch.full((M, (N + 15) // 16), float("nan"), dtype=torch.bfloat16, device=DEV)
    y1 = kernels.qmv_packed_rstd(st.u, packed, N, st.parts, EPS, tile_max=tm)
    tm2 = kernels.tile_max(y1)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    yn = y1.float().cpu().numpy()
    pad = (-N) % 16
    ref = np.pad(yn, ((0, 0), (0, pad)), constant_values=-np.inf).reshape(M, -1, 16).max(-1)
    assert np.array_equal(tm.float().cpu().numpy(), ref)
    assert torch.equal(tm.view(torch.int16), tm2.view(torch.int16))


@pytest.fixture(scope="module")
def tiny():
    cfg = Config.tiny(layers=4, vocab=4096)
    return random_model(cfg, seed=17, device=DEV, max_context=256, max_width=8)


def run(model, ids_list, fuse):
    old = type(model).fuse_norms
    type(model).fuse_norms = fuse
    try:
        cache = model.make_cache()
        outs = []
        for ids in ids_list:
            outs.append(model(torch.tensor(ids, dtype=torch.int32).reshape(1, -1), cache, last_only=False).float())
        torch.cuda.synchronize()
        return outs
    finally:
        type(model).fuse_norms = old


@pytest.mark.gpu
def test_model_fused_norms_close_to_unfused(tiny):
    V = tiny.cfg.vocab_size
    rng = np.random.default_rng(5)
    seq = [rng.integers(0, V, 4).tolist() for _ in range(4)] + [[int(rng.integers(0, V))]]
    a = run(tiny, seq, True)
    b = run(tiny, seq, False)
    for x, y in zip(a, b):
        d = float((x - y).abs().max())
        assert d < 0.1, d


@pytest.mark.gpu
def test_model_fused_rows_independent_of_width(tiny):
    """Four tokens in one call and the same tokens one by one give the same bits."""
    V = tiny.cfg.vocab_size
    ids = np.random.default_rng(6).integers(0, V, 4).tolist()
    wide = run(tiny, [ids], True)[0][0]
    narrow = torch.cat([o[0] for o in run(tiny, [[t] for t in ids], True)])
    assert torch.equal(wide, narrow)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 3])
def test_mtp_first_norm_from_fc_epilogue(tiny, T):
    """The MTP block's first norm inputs from the fc product's residual epilogue
    (zero residual) give the same bits as fc followed by rms_parts: logits and
    the block output of a draft step, for T rows."""
    from qvex.mtp import MTPHead, random_mtp
    mtp = random_mtp(tiny, seed=23)
    H, V = tiny.cfg.hidden_size, tiny.cfg.vocab_size
    g = torch.Generator().manual_seed(29)
    hidden = (torch.randn(1, T, H, generator=g) * 2).to(torch.bfloat16).to(DEV)
    ids = torch.randint(0, V, (1, T), generator=g, dtype=torch.int32).to(DEV)
    outs = []
    old = MTPHead.fc_epilogue
    try:
        for flag in (False, True):
            MTPHead.fc_epilogue = flag
            cache = mtp.make_cache()
            logits, h = mtp(hidden, ids, cache, last_only=False, return_hidden=True)
            torch.cuda.synchronize()
            outs.append((logits.float().cpu(), h.float().cpu()))
    finally:
        MTPHead.fc_epilogue = old
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.gpu
@pytest.mark.parametrize("R,D", [(1, 4096), (4, 4096), (3, 512)])
def test_rmsnorm_pair_equals_two_calls(R, D):
    """qvex_rmsnorm_pair (the MTP head's two input norms into the halves of the fc
    input) = two qvex_rmsnorm calls bit for bit, and rms_norm(x) * w in float64
    within bf16 rounding (engine/mtp.py:63-65)."""
    from qvex import _C
    from qvex.kernels import _ptr, _stream
    from qvex.model import rms_norm
    g = torch.Generator().manual_seed(R * 7 + D)
    x0 = (torch.randn(R, D, generator=g) * 3).to(torch.bfloat16).to(DEV)
    x1 = torch.randn(R, D + 64, generator=g).to(torch.bfloat16).to(DEV)[:, :D]       # strided rows
    w0 = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    w1 = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    pair = torch.empty(R, 2 * D, dtype=torch.bfloat16, device=DEV)
    _C.call("qvex_rmsnorm_pair", _ptr(x0), x0.stride(0), _ptr(w0), _ptr(pair), _ptr(x1), x1.stride(0), _ptr(w1),
            _ptr(pair) + 2 * D, pair.stride(0), R, D, EPS, _stream())
    two = torch.empty_like(pair)
    rms_norm(x0, w0, EPS, out=two[:, :D])
    rms_norm(x1, w1, EPS, out=two[:, D:])
    torch.cuda.synchronize()
    assert torch.equal(pair.view(torch.int16), two.view(torch.int16))
    for x, w, o in ((x0, w0, pair[:, :D]), (x1, w1, pair[:, D:])):
        xx = bf(x)
        ref = xx / np.sqrt((xx ** 2).mean(-1, keepdims=True) + EPS) * bf(w)
        assert (np.abs(bf(o) - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6).all()
