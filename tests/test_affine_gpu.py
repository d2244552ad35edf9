"""Any-width MLX affine quantization on the GPU (per-module overrides,
Config.qparams at engine/model.py:68-71; mixed 4/3-bit models written by
quant/build.py:67-68).

* qvex_qmv_affine vs the float64 oracle, bits 2..8 x groups 32/64/128, with the
  tolerance of the 4-bit kernels: |err| <= 2^-8 |ref| + 2^-14 sum|x| (|s| q + |b|);
* qvex_embed_affine and qvex_affine_widen_w4g64 bit-exact against the oracle's
  unpack (widening is a re-encoding, not an approximation);
* QLinear through every row-count path (packed, chunked, dense GEMM, the
  any-width product) vs the oracle;
* tiny models with overrides: a widening mix (every product still packed, norms
  fused, graphed cycle) and a non-widening mix (separate norm kernels) against
  the numpy forward, and greedy speculative decoding against plain greedy.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle.model import OracleModel
from qvex import kernels, synth
from qvex.model import Config, QEmbedding, QLinear, random_model
from qvex.mtp import random_mtp
from test_model_gpu import f32, logit_tol, prompt, run_decode, start_decoder

DEV = "cuda:0"
WIDTHS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)


def to_dev(a, dtype):
    a = np.ascontiguousarray(a)
    if dtype == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a.view(np.int32)).to(DEV)


def bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def weights(N, K, bits, gs, seed):
    """Codes uniform on 0..2^bits-1, scales ~ U(0.5, 1.5)/sqrt(var K), biases -2^(bits-1) s."""
    g = np.random.default_rng(seed)
    q = g.integers(0, 2 ** bits, size=(N, K), dtype=np.uint8)
    sd = 1.0 / np.sqrt((4 ** bits - 1) / 12 * K)
    s = oracle.bf16_bits((g.uniform(0.5, 1.5, size=(N, K // gs)) * sd).astype(np.float32))
    b = oracle.bf16_bits(-float(2 ** (bits - 1)) * oracle.bf16_to_f32(s))
    return oracle.pack_bits(q, bits), s, b, q


def check(x, w, s, b, bits, gs, y_bits, bf16_weights=False):
    """bf16_weights: the reference uses bf16(s*q + b), the operand of the
    prefill GEMM (qvex_w4g64_packed_gemm), as in tests/test_qgemm_gpu.py."""
    K = x.shape[1]
    if bf16_weights:
        wd = oracle.round_bf16(oracle.dequant_f64(w, s, b, K, bits, gs).astype(np.float32)).astype(np.float64)
        xf = oracle.bf16_to_f32(x).astype(np.float64)
        ref = xf @ wd.T
        err = np.abs(oracle.bf16_to_f32(y_bits).astype(np.float64) - ref)
        tol = 2.0 ** -8 * np.abs(ref) + 2.0 ** -16 * (np.abs(xf) @ np.abs(wd).T)
        print(f"bits={bits} gs={gs} (bf16 weights) worst_ratio={(err / tol).max():.3f}")
        assert np.all(err <= tol), f"max err/tol {(err / tol).max():.3f}"
        return
    ref = oracle.qmv_affine_f64(x, w, s, b, bits, gs)
    q = oracle.unpack_bits(w, K, bits).astype(np.float64)
    sa = np.repeat(np.abs(oracle.bf16_to_f32(s)).astype(np.float64), gs, axis=1)
    ba = np.repeat(np.abs(oracle.bf16_to_f32(b)).astype(np.float64), gs, axis=1)
    cond = np.abs(oracle.bf16_to_f32(x).astype(np.float64)) @ (sa * q + ba).T
    got = oracle.bf16_to_f32(y_bits).astype(np.float64)
    err = np.abs(got - ref)
    tol = 2.0 ** -8 * np.abs(ref) + 2.0 ** -14 * cond
    print(f"bits={bits} gs={gs} max_abs={err.max():.3e} worst_ratio={(err / tol).max():.3f}")
    assert np.all(err <= tol), f"max err/tol {(err / tol).max():.3f}"


@pytest.mark.gpu
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("M", [1, 5, 8])
def test_qmv_affine_vs_oracle(M, bits, gs):
    N, K = 301, 768                      # rows past the last full wave, K a multiple of every group
    w, s, b, _ = weights(N, K, bits, gs, seed=bits * 1000 + gs + M)
    x = synth.qmv_x(M, K, seed=5, tag=bits)
    y = kernels.quantized_matmul(to_dev(x, torch.bfloat16), to_dev(w, torch.int32), to_dev(s, torch.bfloat16),
                                 to_dev(b, torch.bfloat16), group_size=gs, bits=bits)
    torch.cuda.synchronize()
    check(x, w, s, b, bits, gs, bits16(y))


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(3, 64), (8, 128), (5, 32)])
def test_qmv_affine_layer_width(bits, gs):
    N, K = 4096, 4096
    w, s, b, _ = weights(N, K, bits, gs, seed=77 + bits)
    x = synth.qmv_x(4, K, seed=7)
    y = kernels.quantized_matmul(to_dev(x, torch.bfloat16), to_dev(w, torch.int32), to_dev(s, torch.bfloat16),
                                 to_dev(b, torch.bfloat16), group_size=gs, bits=bits)
    torch.cuda.synchronize()
    check(x, w, s, b, bits, gs, bits16(y))


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 64), (5, 128), (6, 64), (8, 32), (4, 128)])
def test_embed_affine_bit_exact(bits, gs):
    V, H = 300, 512
    w, s, b, _ = weights(V, H, bits, gs, seed=bits + gs)
    ids = np.array([0, 17, 299, -3, 305, 17], np.int32)           # out-of-range ids clamp
    e = QEmbedding(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16), gs, bits)
    got = bits16(e(torch.from_numpy(ids).to(DEV)))
    rows = np.clip(ids, 0, V - 1)
    want = oracle.bf16_bits(oracle.dequant_f64(w[rows], s[rows], b[rows], H, bits, gs).astype(np.float32))
    assert np.array_equal(got, want)
    # the generic gather agrees with the widened table's 4-bit gather
    if bits <= 4 and gs % 64 == 0:
        assert e.w4g64() is not None and not e.w.is_cuda
        gen = kernels.embed_affine(torch.from_numpy(ids).to(DEV), to_dev(w, torch.int32), to_dev(s, torch.bfloat16),
                                   to_dev(b, torch.bfloat16), H, gs, bits)
        assert np.array_equal(bits16(gen), want)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(2, 64), (3, 64), (3, 128), (4, 128), (2, 128)])
def test_widen_is_lossless(bits, gs):
    N, K = 37, 1024
    w, s, b, q = weights(N, K, bits, gs, seed=3 * bits + gs)
    w4, s4, b4 = kernels.widen_w4g64(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16),
                                     K, gs, bits)
    torch.cuda.synchronize()
    assert np.array_equal(w4.cpu().numpy().view(np.uint32), oracle.pack_w4(q))
    assert np.array_equal(bits16(s4), np.repeat(s, gs // 64, axis=1))
    assert np.array_equal(bits16(b4), np.repeat(b, gs // 64, axis=1))


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(3, 64), (2, 128), (5, 32), (6, 128), (8, 64)])
@pytest.mark.parametrize("M", [1, 4, 12, 40])
def test_qlinear_any_width(bits, gs, M):
    """Every row-count path of QLinear: packed (1..8), packed chunks (9..15),
    packed GEMM (>= 16) for widened layers; the any-width product otherwise."""
    N, K = 520, 1024
    w, s, b, _ = weights(N, K, bits, gs, seed=bits * gs + M)
    lin = QLinear(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16), gs, bits)
    assert (lin.packed is not None) == (bits <= 4 and gs % 64 == 0)
    lin.offload_mlx()
    x = synth.qmv_x(M, K, seed=13, tag=M)
    y = lin(to_dev(x, torch.bfloat16))
    torch.cuda.synchronize()
    check(x, w, s, b, bits, gs, bits16(y), bf16_weights=lin.packed is not None and M >= QLinear.DENSE_MIN_ROWS)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(3, 64), (4, 64), (5, 32)])
@pytest.mark.parametrize("M", [1, 12])
def test_qlinear_unpackable_k(bits, gs, M):
    """K not a multiple of 256 (no packed copy): every width, 4-bit included,
    runs its MLX-layout product in chunks of 8 rows."""
    N, K = 200, 320
    w, s, b, _ = weights(N, K, bits, gs, seed=5 * bits + M)
    lin = QLinear(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16), gs, bits)
    assert lin.packed is None
    x = synth.qmv_x(M, K, seed=17, tag=M)
    y = lin(to_dev(x, torch.bfloat16))
    torch.cuda.synchronize()
    check(x, w, s, b, bits, gs, bits16(y))


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(3, 64), (6, 32)])
def test_qlinear_swiglu_any_width(bits, gs):
    """The fused gate/up product with SwiGLU: widened (packed SwiGLU kernel) or
    not (product, then qvex_swiglu), against silu(g) * u of the oracle's bf16 g, u."""
    I, K, M = 256, 512, 3
    gw, gsc, gb, _ = weights(I, K, bits, gs, seed=1)
    uw, usc, ub, _ = weights(I, K, bits, gs, seed=2)
    mk = lambda w, s, b: QLinear(to_dev(w, torch.int32), to_dev(s, torch.bfloat16), to_dev(b, torch.bfloat16), gs,
                                 bits, pack=False)
    lin = QLinear.fuse([mk(gw, gsc, gb), mk(uw, usc, ub)], swiglu=True)
    x = synth.qmv_x(M, K, seed=3)
    h = oracle.bf16_to_f32(bits16(lin.swiglu(to_dev(x, torch.bfloat16)))).astype(np.float64)
    g = oracle.round_bf16(oracle.qmv_affine_f64(x, gw, gsc, gb, bits, gs).astype(np.float32)).astype(np.float64)
    u = oracle.round_bf16(oracle.qmv_affine_f64(x, uw, usc, ub, bits, gs).astype(np.float32)).astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    err = np.abs(h - ref)
    # one bf16 step in g or u (their fp32 sums round either way) and the output rounding
    tol = 2.0 ** -6 * (np.abs(ref) + np.abs(g) * np.abs(u)) + 1e-6
    print(f"swiglu bits={bits} max_abs={err.max():.3e} worst_ratio={(err / tol).max():.3f}")
    assert np.all(err <= tol)


WIDENING = {  # a 4/3-bit mix like the reference quantizer's, plus group-128 and 2-bit units
    "model.layers.0.mlp.gate_proj": {"bits": 3}, "model.layers.0.mlp.up_proj": {"bits": 3},
    "model.layers.0.mlp.down_proj": {"bits": 3},
    **{f"model.layers.1.linear_attn.{n}": {"bits": 3} for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a")},
    "model.layers.2.linear_attn.out_proj": {"bits": 2, "group_size": 128},
    **{f"model.layers.3.self_attn.{n}": {"bits": 3, "group_size": 128} for n in ("q_proj", "k_proj", "v_proj")},
    "lm_head": {"bits": 3}, "model.embed_tokens": {"bits": 3},
}
NON_WIDENING = {
    "model.layers.0.mlp.down_proj": {"bits": 5, "group_size": 32},
    "model.layers.2.linear_attn.out_proj": {"bits": 6},
    "model.layers.3.self_attn.o_proj": {"bits": 8, "group_size": 128},
    "lm_head": {"bits": 8}, "model.embed_tokens": {"bits": 5, "group_size": 32},
}


def mixed_model(quant, seed=17):
    cfg = Config.tiny(layers=4, vocab=4096)
    cfg.quant = dict(quant)
    return random_model(cfg, seed=seed, device=DEV, max_context=1024, max_width=8)


@pytest.mark.gpu
@pytest.mark.parametrize("mix", ["widening", "non_widening"])
def test_mixed_model_matches_oracle(mix):
    m = mixed_model(WIDENING if mix == "widening" else NON_WIDENING)
    assert m.all_packed() == (mix == "widening")
    assert m._fused_inputs() == (mix == "widening")
    assert (m.lm_head.bits, m.embed.bits) == ((3, 3) if mix == "widening" else (8, 5))
    V = m.cfg.vocab_size
    ids = prompt(21, V, seed=8)
    cache = m.make_cache()
    logits = m(torch.from_numpy(ids).reshape(1, -1), cache)
    orc = OracleModel(m)
    ol, _ = orc.forward(ids, last_only=True)
    d = np.abs(f32(logits[0]) - ol).max()
    ver = prompt(4, V, seed=9)
    l4 = m(torch.from_numpy(ver).reshape(1, -1), cache, last_only=False)
    ol4, _ = orc.forward(ver, last_only=False)
    d4 = np.abs(f32(l4[0]) - ol4).max()
    print(f"{mix}: prefill max|dlogit|={d:.4f} (tol {logit_tol(ol):.4f}) verify {d4:.4f} (tol {logit_tol(ol4):.4f})")
    assert d <= logit_tol(ol) and d4 <= logit_tol(ol4)


@pytest.mark.gpu
@pytest.mark.parametrize("mix", ["widening", "non_widening"])
def test_mixed_model_greedy_spec_equals_plain(mix):
    m = mixed_model(WIDENING if mix == "widening" else NON_WIDENING, seed=23)
    mtp = random_mtp(m, seed=29, bits=3) if mix == "widening" else random_mtp(m, seed=29, bits=6, group_size=32)
    spec, st = run_decode(m, mtp, 3, 0.0, 16)
    plain, _ = run_decode(m, mtp, 3, 0.0, 16, use_mtp=False)
    print(mix, "cycles", st["cycles"], "accepted", st["accepted"])
    assert spec == plain


@pytest.mark.gpu
@pytest.mark.parametrize("mix", ["widening", "non_widening"])
def test_mixed_model_graphed_cycle_equals_eager(mix):
    """The widening mix keeps the deferred-argmax decode cycle (every product
    packed, 3-bit embedding widened), the non-widening mix the cycle with the
    separate norm kernels: graphed and eager cycles agree in both."""
    from qvex.speculative import GraphedMTPCycle
    if mix == "widening":
        m = mixed_model(WIDENING, seed=31)
        mtp = random_mtp(m, seed=37, bits=3)
        assert m._deferred_argmax() and mtp.all_packed()
    else:
        m = mixed_model(NON_WIDENING, seed=31)
        mtp = random_mtp(m, seed=37, bits=6, group_size=32)
        assert not m._deferred_argmax() and not mtp.all_packed()
    eager = start_decoder(m, mtp, 3, 0.0)
    graphed = GraphedMTPCycle(start_decoder(m, mtp, 3, 0.0))
    te, tg = [], []
    for _ in range(8):
        te += eager.cycle()
        tg += graphed.cycle()
    assert te == tg
    assert [c.offset for c in eager.cache] == [c.offset for c in graphed.dec.cache]
