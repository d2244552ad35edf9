"""Gated DeltaNet recurrent HIP kernel vs the fp64 oracle (GPU).

Tolerances: state and snapshots |s - s64| <= 1e-5 + 1e-4 |s64| (fp32 state,
128-term dot products); y (bf16 output) |y - y64| <= 2^-7 |y64| + 1e-5 (one ulp).
"""

import numpy as np
import pytest
import torch

import oracle
from qvex import kernels, synth

DEV = "cuda:0"


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV).view(torch.bfloat16)


def f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV)


def to_np_bf16(t):
    return synth.bf16_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))


def dev_inputs(inp):
    return (bf(inp["q"]), bf(inp["k"]), bf(inp["v"]), bf(inp["a"]), bf(inp["b"]), f32(inp["A_log"]),
            bf(inp["dt_bias"]))


def oracle_run(inp, state=None, T=None):
    f = synth.bf16_to_f32
    sl = slice(None) if T is None else slice(0, T)
    return oracle.gated_delta_f64(f(inp["q"])[:, sl], f(inp["k"])[:, sl], f(inp["v"])[:, sl],
                                  f(inp["a"])[:, sl], f(inp["b"])[:, sl], inp["A_log"],
                                  f(inp["dt_bias"]), inp["state"] if state is None else state)


def check_y(y, y64):
    err = np.abs(y - y64)
    tol = 2.0 ** -7 * np.abs(y64) + 1e-5   # one bf16 ulp
    print(f"y max_abs={err.max():.3e} worst={(err / tol).max():.3f}")
    assert np.all(err <= tol)


def check_s(s, s64):
    err = np.abs(s - s64)
    tol = 1e-5 + 1e-4 * np.abs(s64)
    print(f"state max_abs={err.max():.3e} worst={(err / tol).max():.3f}")
    assert np.all(err <= tol)


@pytest.mark.gpu
def test_verify_t5_snapshots():
    inp = synth.gdn_inputs(5)
    y, snaps = kernels.gated_delta_snapshots(*dev_inputs(inp), f32(inp["state"]))
    torch.cuda.synchronize()
    y64, s64, sn64 = oracle_run(inp)
    check_y(to_np_bf16(y), y64)
    sn = snaps.cpu().numpy()
    for t in range(5):
        check_s(sn[t], sn64[t])


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 2, 3, 9, 17])
def test_lengths(T):
    inp = synth.gdn_inputs(T, seed=77, Hk=4, Hv=8)
    y, snaps = kernels.gated_delta_snapshots(*dev_inputs(inp), f32(inp["state"]))
    torch.cuda.synchronize()
    y64, s64, sn64 = oracle_run(inp)
    check_y(to_np_bf16(y), y64)
    check_s(snaps.cpu().numpy()[-1], s64)


@pytest.mark.gpu
def test_keep_mid_matches_reference_semantics():
    inp = synth.gdn_inputs(2, seed=5)
    y, st, mid = kernels.gated_delta(*dev_inputs(inp), f32(inp["state"]), keep_mid=True)
    torch.cuda.synchronize()
    _, s1, _ = oracle_run(inp, T=1)
    _, s2, _ = oracle_run(inp)
    check_s(mid.cpu().numpy(), s1)
    check_s(st.cpu().numpy(), s2)
    y2, st2 = kernels.gated_delta(*dev_inputs(inp), f32(inp["state"]))
    torch.cuda.synchronize()
    assert torch.equal(st2, st) and torch.equal(y2.view(torch.int16), y.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("L", range(0, 6))
def test_rollback_is_prefix_run(L):
    """State after keeping L of 5 verify tokens == running only the first L
    tokens (bit-exact: the same kernel does the same arithmetic per token)."""
    inp = synth.gdn_inputs(5, seed=11)
    d = dev_inputs(inp)
    s0 = f32(inp["state"])
    _, snaps = kernels.gated_delta_snapshots(*d, s0)
    picked = s0 if L == 0 else snaps[L - 1]
    if L > 0:
        sub = tuple(t[:, :L].contiguous() for t in d[:5]) + d[5:]
        _, snaps_l = kernels.gated_delta_snapshots(*sub, s0)
        torch.cuda.synchronize()
        assert torch.equal(snaps_l[L - 1], picked)
    # continue with 3 new tokens from the rolled-back state
    nxt = synth.gdn_inputs(3, seed=12)
    y_a, sn_a = kernels.gated_delta_snapshots(*dev_inputs(nxt), picked.contiguous())
    torch.cuda.synchronize()
    state_l = inp["state"] if L == 0 else oracle_run(inp, T=L)[1]
    nxt_o = dict(nxt)
    nxt_o["state"] = state_l
    y64, s64, _ = oracle_run(nxt_o)
    check_y(to_np_bf16(y_a), y64)
    check_s(sn_a[-1].cpu().numpy(), s64)


@pytest.mark.gpu
def test_ring_slots_and_aliasing():
    """Ring form: state from slot c, token t to slot (c+1+t) % n; the source slot
    may be any slot, including one the same launch overwrites later."""
    inp = synth.gdn_inputs(5, seed=21)
    d = dev_inputs(inp)
    n = 6
    ring = torch.zeros((n, 1, 32, 128, 128), dtype=torch.float32, device=DEV)
    y_ref, sn_ref = kernels.gated_delta_snapshots(*d, f32(inp["state"]))
    for c in (0, 3, 5):
        ring.zero_()
        ring[c] = f32(inp["state"])
        cur = torch.tensor([c], dtype=torch.int32, device=DEV)
        y = kernels.gated_delta_ring(*d, ring, cur)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
        for t in range(5):
            assert torch.equal(ring[(c + 1 + t) % n], sn_ref[t])
    # aliasing in the plain form: state_in is snapshot slot 2 of the output buffer
    buf = torch.zeros((5, 1, 32, 128, 128), dtype=torch.float32, device=DEV)
    buf[2] = f32(inp["state"])
    y2, _ = kernels.gated_delta_snapshots(*d, buf[2], snapshots=buf)
    torch.cuda.synchronize()
    assert torch.equal(buf, sn_ref)


@pytest.mark.gpu
def test_prefill_length_recurrent():
    inp = synth.gdn_inputs(512, seed=31)
    y, st = kernels.gated_delta(*dev_inputs(inp), f32(inp["state"]))
    torch.cuda.synchronize()
    y64, s64, _ = oracle_run(inp)
    check_y(to_np_bf16(y), y64)
    check_s(st.cpu().numpy(), s64)
