"""The MTP head (qvex/mtp.py) against the oracle's restatement of
engine/mtp.py:58-68 (GPU): logits and block output for a prefill-style call
(T = 12 rows, separate norm kernels), a verify-width call (T = k + 1 = 4, norms
folded into the products), one-row chained draft steps (the block output fed
back with its draft), the device row select and the greedy argmax epilogue.

The head reads the GPU model's hidden rows on both sides, so only the head is
under test. Tolerance: two bf16 steps at the largest |logit| (logit_tol; one
step is measured on MI355X), and HID_TOL of the largest |x| of the block
output (about twice the 0.0069 measured); the bf16 rounding points of the fused
kernels differ from the per-op roundings of the reference."""

import numpy as np
import pytest
import torch

from oracle.model import OracleModel
from qvex.model import Config, random_model
from qvex.mtp import random_mtp
from test_model_gpu import logit_tol

DEV = "cuda:0"
HID_TOL = 0.015         # of the largest |x| of the block output


def f32(t):
    return t.float().cpu().numpy()


@pytest.fixture(scope="module")
def setup():
    cfg = Config.tiny(layers=4, vocab=4096)
    m = random_model(cfg, seed=71, device=DEV, max_context=1024)
    mtp = random_mtp(m, seed=72)
    g = np.random.default_rng(73)
    ids = torch.from_numpy(g.integers(0, cfg.vocab_size, 13).astype(np.int32)).reshape(1, -1).to(DEV)
    ver = torch.from_numpy(g.integers(0, cfg.vocab_size, 4).astype(np.int32)).reshape(1, -1).to(DEV)
    cache = m.make_cache()
    _, hidden = m(ids, cache, return_hidden=True)
    _, vhid = m(ver, cache, last_only=False, return_hidden=True)
    torch.cuda.synchronize()
    return m, mtp, ids, hidden, ver, vhid


def check(tag, gl, ol, gx=None, ox=None):
    d = float(np.abs(gl - ol).max())
    msg = f"{tag}: max|dlogit| {d:.4f}"
    if gx is not None:
        dh = float(np.abs(gx - ox).max() / (np.abs(ox).max() + 1e-9))
        msg += f" rel|dhidden| {dh:.4f}"
        assert dh < HID_TOL, msg
    print(msg)
    assert d <= logit_tol(ol), msg


@pytest.mark.gpu
def test_mtp_head_prefill_verify_and_chained_steps(setup):
    m, mtp, ids, hidden, ver, vhid = setup
    orc = OracleModel(m)
    oc = orc.new_kv_cache()
    mc = mtp.make_cache()
    # prefill pairs (h_i, t_{i+1}) of the 13-token prompt: 12 rows
    gl, gx = mtp(hidden[:, :-1], ids[:, 1:], mc, last_only=False, return_hidden=True)
    ol, ox = orc.mtp(mtp, f32(hidden[0, :-1]), ids[0, 1:].cpu().numpy(), oc, last_only=False)
    check("T=12 prefill", f32(gl[0]), ol, f32(gx[0]), ox)
    # verify width (k + 1 = 4 rows): the folded-norm path
    pairs_h = torch.cat([hidden[:, -1:], vhid[:, :3]], dim=1)
    gl4, gx4 = mtp(pairs_h, ver, mc, last_only=False, return_hidden=True)
    ol4, ox4 = orc.mtp(mtp, f32(pairs_h[0]), ver[0].cpu().numpy(), oc, last_only=False)
    check("T=4 verify", f32(gl4[0]), ol4, f32(gx4[0]), ox4)
    # two chained draft steps: (block output of the last row, its greedy draft)
    gh, oh = gx4[:, -1:], ox4[-1:]
    for step in range(2):
        d_o = int(np.argmax(ol4[-1] if step == 0 else olc[-1]))
        glc, gxc = mtp(gh, torch.tensor([[d_o]], dtype=torch.int32, device=DEV), mc, return_hidden=True)
        olc, oxc = orc.mtp(mtp, oh, np.array([d_o]), oc)
        check(f"chained step {step + 1}", f32(glc[0]), olc, f32(gxc[0]), oxc)
        gh, oh = gxc, oxc
    assert mc.offset == 12 + 4 + 2 and oc["k"].shape[1] == 18


@pytest.mark.gpu
def test_mtp_select_and_argmax_epilogue(setup):
    """select=row on the device runs every row through the block but only that
    row through the lm_head; argmax_out writes the greedy draft of that row
    (what the captured cycle uses)."""
    m, mtp, ids, hidden, ver, vhid = setup
    pairs_h = torch.cat([hidden[:, -1:], vhid[:, :3]], dim=1)
    orc = OracleModel(m)
    oc = orc.new_kv_cache()
    ol, ox = orc.mtp(mtp, f32(pairs_h[0]), ver[0].cpu().numpy(), oc, last_only=False)
    for row in range(4):
        mc = mtp.make_cache()
        sel = torch.tensor([row], dtype=torch.int32, device=DEV)
        gl, gx = mtp(pairs_h, ver, mc, return_hidden=True, select=sel)
        check(f"select row {row}", f32(gl[0]), ol[row:row + 1], f32(gx[0]), ox[row:row + 1])
        mc2 = mtp.make_cache()
        am = torch.empty(1, dtype=torch.int32, device=DEV)
        mtp(pairs_h, ver, mc2, return_hidden=True, select=sel, argmax_out=am)
        top2 = np.sort(ol[row])[-2:]
        if top2[1] - top2[0] > 2 * logit_tol(ol):    # a clear winner: the draft must be it
            assert int(am.item()) == int(np.argmax(ol[row]))
        assert int(am.item()) == int(np.argmax(f32(gl[0, -1])))
