"""Pins the layer-level oracle (oracle/model.py) on the CPU: RoPE against the
complex-rotation form and its invariants, the conv window against numpy's
correlate and one-hot taps, the attention core against closed forms, and the
MTP head's input order and chained hidden (engine/mtp.py:58-68).

Each check is chosen so a plausible slip (interleaved instead of half-split
pairs, a wrong frequency exponent, a reversed conv tap order, a swapped
[embedding | hidden] concatenation) fails it."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from oracle import model as om

ULP = 2.0 ** -8          # one bf16 step relative to the value


def bfv(a):
    """float32 array of bf16-representable values."""
    return oracle.round_bf16(np.asarray(a, np.float32))


# ---------------------------------------------------------------- RoPE (mx.fast.rope, traditional=False)

def rope_complex(x, pos0, dims, base):
    """Half-split pairs as complex numbers: (x_i + i x_{i+dims/2}) e^{i (pos) base^(-2i/dims)}."""
    H, L, D = x.shape
    half = dims // 2
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:dims].astype(np.float64)
    theta = np.exp(-np.log(base) * (2.0 * np.arange(half) / dims))
    rot = np.exp(1j * (pos0 + np.arange(L))[:, None] * theta[None, :])
    zr = z * rot[None]
    y = x.astype(np.float64).copy()
    y[..., :half], y[..., half:dims] = zr.real, zr.imag
    return y


@pytest.mark.parametrize("dims,D,pos0", [(64, 256, 4348), (48, 256, 777), (32, 128, 0), (64, 64, 8191)])
def test_rope_equals_complex_rotation(dims, D, pos0):
    g = np.random.default_rng(dims + pos0)
    x = bfv(g.standard_normal((3, 5, D)))
    got = om.rope(x, pos0, dims, 1e7)
    ref = rope_complex(x, pos0, dims, 1e7)
    assert np.all(np.abs(got - ref) <= ULP * np.abs(ref) + 1e-30)


def test_rope_position_zero_is_identity_and_tail_untouched():
    g = np.random.default_rng(1)
    x = bfv(g.standard_normal((2, 1, 256)))
    np.testing.assert_array_equal(om.rope(x, 0, 64, 1e7), x)
    y = om.rope(bfv(g.standard_normal((2, 4, 256))), 1234, 64, 1e7)
    x2 = bfv(g.standard_normal((2, 4, 256)))
    y = om.rope(x2, 1234, 64, 1e7)
    np.testing.assert_array_equal(y[..., 64:], x2[..., 64:])


def test_rope_half_split_pairing_and_frequencies():
    """A unit vector on dim 0 (frequency index 0, theta = 1) moves to dim dims/2
    (the half-split partner), not to dim 1 (the interleaved partner); dim
    dims/2 - 1 turns at base^(-(dims-2)/dims)."""
    dims, D, base, pos = 64, 256, 1e7, 3
    x = np.zeros((1, 1, D), np.float32)
    x[0, 0, 0] = 1.0
    y = om.rope(x, pos, dims, base)
    assert abs(y[0, 0, 0] - np.cos(pos)) <= ULP and abs(y[0, 0, dims // 2] - np.sin(pos)) <= ULP
    assert y[0, 0, 1] == 0.0
    x = np.zeros((1, 1, D), np.float32)
    x[0, 0, dims // 2 - 1] = 1.0
    y = om.rope(x, 1000, dims, base)
    ang = 1000 * base ** (-(dims - 2) / dims)
    assert abs(y[0, 0, dims // 2 - 1] - np.cos(ang)) <= ULP
    assert abs(y[0, 0, dims - 1] - np.sin(ang)) <= ULP


def test_rope_keeps_pair_norms_and_scores_depend_on_offset_only():
    g = np.random.default_rng(2)
    dims, D = 64, 256
    q = bfv(g.standard_normal((1, 1, D)))
    k = bfv(g.standard_normal((1, 1, D)))
    half = dims // 2
    for pos in (0, 17, 4096):
        y = om.rope(q, pos, dims, 1e7)
        n0 = np.hypot(q[..., :half], q[..., half:dims])
        n1 = np.hypot(y[..., :half], y[..., half:dims])
        assert np.all(np.abs(n1 - n0) <= 2 * ULP * n0 + 1e-30)

    def score(m, n):
        return float((om.rope(q, m, dims, 1e7)[0, 0].astype(np.float64) *
                      om.rope(k, n, dims, 1e7)[0, 0].astype(np.float64)).sum())
    scale = float(np.linalg.norm(q) * np.linalg.norm(k))
    for m, n, s in ((10, 3, 500), (4000, 4000, 97), (0, 9, 2048)):
        assert abs(score(m, n) - score(m + s, n + s)) <= 4 * ULP * scale


# ---------------------------------------------------------------- conv window (mx.conv1d, groups = C)

def test_conv_window_equals_numpy_correlate():
    g = np.random.default_rng(3)
    K, C, S = 4, 6, 9
    state = bfv(g.standard_normal((K - 1, C)))
    x = bfv(g.standard_normal((S, C)))
    w = bfv(g.standard_normal((C, K)))
    out, new_state = om.conv1d_window(state, x, w)
    conv_in = np.concatenate([state, x]).astype(np.float64)
    for c in range(C):
        ref = np.correlate(conv_in[:, c], w[c].astype(np.float64), mode="valid")
        assert np.all(np.abs(out[:, c] - ref) <= ULP * np.abs(ref) + 1e-30)
    np.testing.assert_array_equal(new_state, np.concatenate([state, x])[-(K - 1):])


def test_conv_window_one_hot_taps():
    """Tap K - 1 passes the current token through; tap 0 the token K - 1 back
    (from the carried state for the first K - 1 rows)."""
    g = np.random.default_rng(4)
    K, C, S = 4, 5, 7
    state = bfv(g.standard_normal((K - 1, C)))
    x = bfv(g.standard_normal((S, C)))
    cur = np.zeros((C, K), np.float32)
    cur[:, K - 1] = 1.0
    np.testing.assert_array_equal(om.conv1d_window(state, x, cur)[0], x)
    old = np.zeros((C, K), np.float32)
    old[:, 0] = 1.0
    np.testing.assert_array_equal(om.conv1d_window(state, x, old)[0], np.concatenate([state, x])[:S])


def test_conv_window_streams_across_calls():
    g = np.random.default_rng(5)
    K, C = 4, 8
    state = np.zeros((K - 1, C), np.float32)
    x = bfv(g.standard_normal((11, C)))
    w = bfv(g.standard_normal((C, K)))
    whole, st_w = om.conv1d_window(state, x, w)
    a, st = om.conv1d_window(state, x[:5], w)
    b, st = om.conv1d_window(st, x[5:], w)
    np.testing.assert_array_equal(np.concatenate([a, b]), whole)
    np.testing.assert_array_equal(st, st_w)


# ---------------------------------------------------------------- attention core (causal SDPA)

def test_attention_core_closed_forms():
    g = np.random.default_rng(6)
    S, D, pos0, L = 9, 16, 5, 4
    K = g.standard_normal((S, D))
    V = g.standard_normal((S, D))
    # a zero query averages the keys it may see: query l sees pos0 + l + 1 keys
    o = om.attention_core(np.zeros((L, D)), K, V, pos0, 0.25)
    for l in range(L):
        np.testing.assert_allclose(o[l], V[:pos0 + l + 1].mean(0), rtol=1e-12, atol=1e-12)
    # keys past a query's position do not change its output
    q = g.standard_normal((L, D))
    base = om.attention_core(q, K, V, pos0, 0.25)
    K2, V2 = K.copy(), V.copy()
    K2[pos0 + 1:] += 5.0
    V2[pos0 + 1:] -= 3.0
    np.testing.assert_array_equal(om.attention_core(q, K2, V2, pos0, 0.25)[0], base[0])
    # one key far above the others takes all the weight
    K3 = K.copy()
    K3[2] = 50.0 * q[0] / np.linalg.norm(q[0])
    np.testing.assert_allclose(om.attention_core(q[:1], K3, V, pos0, 1.0)[0], V[2], atol=1e-9)


# ---------------------------------------------------------------- MTP head (engine/mtp.py:58-68)

def qlin(g, N, K, zero_cols=None):
    w = torch.from_numpy(g.integers(0, 2**32, (N, K // 8), dtype=np.uint64).astype(np.uint32).view(np.int32))
    s = (0.5 + g.random((N, K // 64))) / np.sqrt(21.25 * K)
    if zero_cols is not None:
        s[:, zero_cols[0] // 64:zero_cols[1] // 64] = 0.0
    sb = oracle.bf16_bits(s.astype(np.float32))
    bb = oracle.bf16_bits(-8.0 * oracle.bf16_to_f32(sb))
    return SimpleNamespace(w=w, scales=torch.from_numpy(sb.view(np.int16)).view(torch.bfloat16),
                           biases=torch.from_numpy(bb.view(np.int16)).view(torch.bfloat16), N=N)


def ones(g, n):
    return torch.from_numpy(bfv(1.0 + 0.1 * g.standard_normal(n))).to(torch.bfloat16)


def tiny_mtp(seed=0, zero_hidden_half=False, hidden_mode="pre"):
    """A small model + MTP head as the oracle reads them (weights only)."""
    g = np.random.default_rng(seed)
    H, I, D, Hq, Hkv, V = 128, 256, 64, 2, 1, 512
    cfg = SimpleNamespace(hidden_size=H, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D,
                          rotary_dim=16, rope_theta=1e7, rms_norm_eps=1e-6, linear_conv_kernel_dim=4)
    model = SimpleNamespace(cfg=cfg, layers=[], embed=qlin(g, V, H), norm=ones(g, H), lm_head=qlin(g, V, H))
    att = SimpleNamespace(qkv_proj=qlin(g, Hq * 2 * D + 2 * Hkv * D, H), o_proj=qlin(g, H, Hq * D),
                          q_norm=ones(g, D), k_norm=ones(g, D))
    layer = SimpleNamespace(linear=False, mixer=att, ln1=ones(g, H), ln2=ones(g, H),
                            mlp=SimpleNamespace(gate_up=qlin(g, 2 * I, H), down=qlin(g, H, I), hidden=I))
    head = SimpleNamespace(hidden_mode=hidden_mode, fc=qlin(g, H, 2 * H, zero_cols=(H, 2 * H) if zero_hidden_half
                                                                 else None),
                           norm_emb=ones(g, H), norm_hid=ones(g, H), norm_out=ones(g, H), layer=layer)
    return model, head


def run_mtp(model, head, hidden, ids, last_only=False):
    orc = om.OracleModel(model)
    return orc.mtp(head, hidden, ids, orc.new_kv_cache(), last_only=last_only)


def test_mtp_concatenates_embedding_then_hidden():
    """With the fc's second-half columns zero, the head depends on the token only
    ([rms(embed) | rms(h)], embedding first): changing the hidden changes nothing,
    changing the token does."""
    model, head = tiny_mtp(seed=1, zero_hidden_half=True)
    g = np.random.default_rng(2)
    h1, h2 = bfv(g.standard_normal((3, 128))), bfv(5 * g.standard_normal((3, 128)))
    ids = np.array([3, 77, 400])
    l1, x1 = run_mtp(model, head, h1, ids)
    l2, x2 = run_mtp(model, head, h2, ids)
    np.testing.assert_array_equal(l1, l2)
    np.testing.assert_array_equal(x1, x2)
    l3, _ = run_mtp(model, head, h1, np.array([4, 77, 400]))
    assert not np.array_equal(l3[0], l1[0])


def test_mtp_rows_equal_sequential_calls_and_chaining():
    """T rows in one call equal T one-row calls on the same KV cache (causality
    of the head's attention), and last_only keeps the last row; the returned
    hidden is the block output a chained step feeds back."""
    model, head = tiny_mtp(seed=3)
    g = np.random.default_rng(4)
    hid = bfv(g.standard_normal((4, 128)))
    ids = np.array([5, 6, 7, 8])
    full, xf = run_mtp(model, head, hid, ids)
    orc = om.OracleModel(model)
    c = orc.new_kv_cache()
    for t in range(4):
        lt, xt = orc.mtp(head, hid[t:t + 1], ids[t:t + 1], c)
        np.testing.assert_allclose(lt[0], full[t], atol=2 * ULP * np.abs(full).max())
        np.testing.assert_allclose(xt[0], xf[t], atol=2 * ULP * np.abs(xf).max())
    last, _ = run_mtp(model, head, hid, ids, last_only=True)
    np.testing.assert_array_equal(last[0], full[-1])
    # chained step: (block output of the last row, its draft) advances the same cache
    draft = int(np.argmax(full[-1]))
    c2 = orc.new_kv_cache()
    orc.mtp(head, hid, ids, c2)
    l_ch, _ = orc.mtp(head, xf[-1:], np.array([draft]), c2)
    assert l_ch.shape == (1, 512) and c2["k"].shape[1] == 5


def test_mtp_post_mode_normalises_the_hidden_first():
    model, head_pre = tiny_mtp(seed=5)
    _, head_post = tiny_mtp(seed=5, hidden_mode="post")
    g = np.random.default_rng(6)
    hid = bfv(g.standard_normal((2, 128)))
    ids = np.array([9, 10])
    normed = om.rms_norm(hid, om._np(model.norm), 1e-6)
    a, _ = run_mtp(model, head_post, hid, ids)
    b, _ = run_mtp(model, head_pre, normed, ids)
    np.testing.assert_array_equal(a, b)


def test_rms_norm_formula():
    g = np.random.default_rng(7)
    x = bfv(3 * g.standard_normal((4, 64)))
    w = bfv(1 + 0.1 * g.standard_normal(64))
    got = om.rms_norm(x, w, 1e-6)
    ref = w.astype(np.float64) * x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.all(np.abs(got - ref) <= ULP * np.abs(ref) + 1e-30)
