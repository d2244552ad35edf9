"""ORACLE ONLY (test infrastructure): numpy restatement of the Qwen3.5 verify
forward, following engine/model.py:121-336 and engine/mtp.py:58-68 op by op,
with a bf16 rounding wherever the reference produces a bf16 array.

Weights are read from a qvex model object's tensors (host copies); the oracle
never calls the HIP library. fp32 arithmetic (float64 for the matmul
accumulations, through the C fp64 qmv of liboracle).

Pinning (tests/test_oracle_model.py, CPU): rope against the complex-rotation
form and its invariants (identity at position 0, norm kept, scores depend only
on the position difference, dims past rot_dim untouched, the half-split pairing
of traditional=False); conv1d_window against numpy's correlate and one-hot taps;
rms_norm against a float64 formula; attention_core against a log-sum-exp form;
the MTP head (mtp) against the composition of these pinned parts, written out
separately in the test.
"""

from __future__ import annotations

import numpy as np

from . import (bf16_bits, bf16_to_f32, round_bf16, dequant_f64, gated_delta_f64, qmv_affine_f64,
               qmv_f64)


def _np_bf16(t):
    import torch
    return bf16_to_f32(t.detach().view(torch.int16).cpu().numpy().view(np.uint16))


def _np(t):
    import torch
    if t.dtype == torch.bfloat16:
        return _np_bf16(t)
    return t.detach().cpu().numpy()


def _qweights(q):
    import torch
    w = q.w.detach().cpu().numpy().view(np.uint32)
    s = q.scales.detach().view(torch.int16).cpu().numpy().view(np.uint16)
    b = q.biases.detach().view(torch.int16).cpu().numpy().view(np.uint16)
    return w, s, b


def _width(q):
    return getattr(q, "bits", 4), getattr(q, "group_size", 64)


def embed_rows(e, ids):
    """bf16(s * q + b) of the gathered rows (mx.dequantize on QEmbedding rows)."""
    w, s, b = _qweights(e)
    bits, gs = _width(e)
    ids = np.asarray(ids, np.int64)
    H = w.shape[1] * 32 // bits
    return round_bf16(dequant_f64(w[ids], s[ids], b[ids], H, bits, gs).astype(np.float32))


def qlinear(q, x):
    """y = bf16(x @ dequant(W)^T) (mx.quantized_matmul); x holds bf16 values.
    4-bit group-64: the fp64 sum runs in C (one dequantized weight row at a
    time), so a full-vocabulary lm_head needs no dense copy of the weight; other
    widths dequantize blocks of rows in numpy."""
    w, s, b = _qweights(q)
    bits, gs = _width(q)
    K = w.shape[1] * 32 // bits
    x2 = np.asarray(x, np.float32).reshape(-1, K)
    if (bits, gs) == (4, 64):
        y = qmv_f64(bf16_bits(x2), w, s, b)
    else:
        y = qmv_affine_f64(bf16_bits(x2), w, s, b, bits, gs)
    return round_bf16(y.astype(np.float32)).reshape(*np.shape(x)[:-1], w.shape[0])


def rms_norm(x, w, eps):
    """mx.fast.rms_norm: w * (x * rsqrt(mean(x^2) + eps)), fp32 inside, bf16 out."""
    x = x.astype(np.float32)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + np.float32(eps))
    y = x * inv.astype(np.float32)
    if w is not None:
        y = w * y
    return round_bf16(y.astype(np.float32))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def conv1d_window(state, x, w):
    """Causal depthwise conv over [state; x] (engine/model.py:261-269): mx.conv1d
    with weight [C, K, 1] and groups = C is a cross-correlation, so output row t
    = sum_j conv_in[t + j] * w[:, j]; tap K - 1 multiplies the current token.
    state [K-1, C], x [S, C], w [C, K] -> (bf16 conv output [S, C], new state)."""
    Kw = w.shape[1]
    conv_in = np.concatenate([state, x], axis=0)
    S = x.shape[0]
    acc = np.zeros((S, x.shape[1]), np.float64)
    for j in range(Kw):
        acc += conv_in[j:j + S].astype(np.float64) * w[:, j][None, :]
    return round_bf16(acc.astype(np.float32)), conv_in[-(Kw - 1):].copy()


def attention_core(q, K, V, pos0, scale):
    """Causal softmax attention of L queries at positions pos0.. over S keys
    (mx.fast.scaled_dot_product_attention with mask="causal" when L > 1):
    q [L, D], K, V [S, D] -> [L, D] float64."""
    L, S = q.shape[0], K.shape[0]
    s = (q.astype(np.float64) @ K.T.astype(np.float64)) * scale
    s[np.arange(S)[None, :] > (pos0 + np.arange(L))[:, None]] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return p @ V.astype(np.float64)


def rope(x, pos0, dims, base):
    """mx.fast.rope(traditional=False): rotate (x_i, x_{i+dims/2}) for i < dims/2
    by (pos0 + l) * base^(-2i/dims); x [H, L, D]."""
    H, L, D = x.shape
    half = dims // 2
    inv = base ** (-2.0 * np.arange(half) / dims)
    ang = (pos0 + np.arange(L))[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    y = x.astype(np.float64).copy()
    x1, x2 = x[..., :half].astype(np.float64), x[..., half:dims].astype(np.float64)
    y[..., :half] = x1 * c - x2 * s
    y[..., half:dims] = x1 * s + x2 * c
    return round_bf16(y.astype(np.float32))


class OracleModel:
    """Mirror of engine/model.py Qwen35 with caches held as numpy arrays."""

    def __init__(self, model):
        self.m = model
        self.cfg = model.cfg
        self.reset()

    def reset(self):
        cfg = self.cfg
        self.caches = []
        for l in self.m.layers:
            if l.linear:
                g = l.mixer
                self.caches.append({"conv": np.zeros((cfg.linear_conv_kernel_dim - 1, g.conv_dim), np.float32),
                                    "ssm": np.zeros((1, g.hv, g.dv, g.dk), np.float64)})
            else:
                self.caches.append({"k": np.zeros((cfg.num_key_value_heads, 0, cfg.head_dim), np.float32),
                                    "v": np.zeros((cfg.num_key_value_heads, 0, cfg.head_dim), np.float32)})

    def snapshot(self):
        import copy
        return copy.deepcopy(self.caches)

    def restore(self, snap):
        import copy
        self.caches = copy.deepcopy(snap)

    # -- blocks
    def attention(self, att, x, c):
        cfg = self.cfg
        L = x.shape[0]
        H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        proj = qlinear(att.qkv_proj, x)
        qg = proj[:, :H * 2 * D].reshape(L, H, 2 * D)
        q, gate = qg[..., :D], qg[..., D:]
        k = proj[:, H * 2 * D:H * 2 * D + Hkv * D].reshape(L, Hkv, D)
        v = proj[:, H * 2 * D + Hkv * D:].reshape(L, Hkv, D)
        q = rms_norm(q, _np(att.q_norm), cfg.rms_norm_eps).transpose(1, 0, 2)
        k = rms_norm(k, _np(att.k_norm), cfg.rms_norm_eps).transpose(1, 0, 2)
        v = v.transpose(1, 0, 2)
        pos0 = c["k"].shape[1]
        q = rope(q, pos0, cfg.rotary_dim, cfg.rope_theta)
        k = rope(k, pos0, cfg.rotary_dim, cfg.rope_theta)
        c["k"] = np.concatenate([c["k"], k], axis=1)
        c["v"] = np.concatenate([c["v"], v], axis=1)
        K, V = c["k"], c["v"]
        rep = H // Hkv
        o = np.zeros((H, L, D), np.float64)
        for h in range(H):
            o[h] = attention_core(q[h], K[h // rep], V[h // rep], pos0, 1.0 / np.sqrt(D))
        o = round_bf16(o.astype(np.float32)).transpose(1, 0, 2).reshape(L, H * D)
        og = round_bf16(o * round_bf16(sigmoid(gate.reshape(L, H * D))))
        return qlinear(att.o_proj, og)

    def gdn(self, g, x, c):
        cfg = self.cfg
        S = x.shape[0]
        proj = qlinear(g.in_proj, x)
        qkv = proj[:, :g.conv_dim]
        z = proj[:, g.conv_dim:g.conv_dim + g.value_dim]
        b = proj[:, g.conv_dim + g.value_dim:g.conv_dim + g.value_dim + g.hv]
        a = proj[:, g.conv_dim + g.value_dim + g.hv:]
        conv, c["conv"] = conv1d_window(c["conv"], qkv, _np(g.conv_w))
        conv = round_bf16(conv * round_bf16(sigmoid(conv)))
        q = conv[:, :g.key_dim].reshape(1, S, g.hk, g.dk)
        k = conv[:, g.key_dim:2 * g.key_dim].reshape(1, S, g.hk, g.dk)
        v = conv[:, 2 * g.key_dim:].reshape(1, S, g.hv, g.dv)
        inv = g.dk ** -0.5
        q = round_bf16(np.float32(inv * inv) * rms_norm(q, None, 1e-6))
        k = round_bf16(np.float32(inv) * rms_norm(k, None, 1e-6))
        y, st, _ = gated_delta_f64(q, k, v, a.reshape(1, S, g.hv), b.reshape(1, S, g.hv), _np(g.A_log),
                                   _np(g.dt_bias), c["ssm"], snaps=False)
        c["ssm"] = st
        y = round_bf16(y.astype(np.float32)).reshape(S, g.hv, g.dv)
        n = rms_norm(y, _np(g.norm_w), cfg.rms_norm_eps)
        zf = z.reshape(S, g.hv, g.dv)
        out = round_bf16((zf * sigmoid(zf) * n).astype(np.float32)).reshape(S, -1)
        return qlinear(g.out_proj, out)

    def mlp(self, mlp, x):
        gu = qlinear(mlp.gate_up, x)
        I = mlp.hidden
        gt, up = gu[:, :I], gu[:, I:]
        return qlinear(mlp.down, round_bf16((gt * sigmoid(gt) * up).astype(np.float32)))

    def layer(self, l, x, c):
        eps = self.cfg.rms_norm_eps
        n = rms_norm(x, _np(l.ln1), eps)
        d = self.gdn(l.mixer, n, c) if l.linear else self.attention(l.mixer, n, c)
        h = round_bf16(x + d)
        return round_bf16(h + self.mlp(l.mlp, rms_norm(h, _np(l.ln2), eps)))

    def new_kv_cache(self):
        cfg = self.cfg
        return {"k": np.zeros((cfg.num_key_value_heads, 0, cfg.head_dim), np.float32),
                "v": np.zeros((cfg.num_key_value_heads, 0, cfg.head_dim), np.float32)}

    def mtp(self, head, hidden, next_ids, cache, last_only=True):
        """The MTP head (engine/mtp.py:58-68): hidden [T, H] (main model,
        pre-norm, bf16 values) and next_ids [T] -> (logits [1 or T, V], block
        output x [T, H] before the final norm). x is what a chained draft step
        takes as its hidden (k > 1 drafting). cache: new_kv_cache()."""
        eps = self.cfg.rms_norm_eps
        h = np.asarray(hidden, np.float32)
        if head.hidden_mode == "post":
            h = rms_norm(h, _np(self.m.norm), eps)
        e = rms_norm(embed_rows(self.m.embed, next_ids), _np(head.norm_emb), eps)
        hn = rms_norm(h, _np(head.norm_hid), eps)
        x = qlinear(head.fc, np.concatenate([e, hn], axis=-1))
        x = self.layer(head.layer, x, cache)
        xo = x[-1:] if last_only else x
        return qlinear(self.m.lm_head, rms_norm(xo, _np(head.norm_out), eps)), x

    def forward(self, ids, last_only=True):
        """ids [L] -> (logits [L or 1, V] fp32 of bf16 values, pre-norm hidden [L, H])."""
        m = self.m
        x = embed_rows(m.embed, ids)
        for l, c in zip(m.layers, self.caches):
            x = self.layer(l, x, c)
        h = x
        xn = x[-1:] if last_only else x
        logits = qlinear(m.lm_head, rms_norm(xn, _np(m.norm), self.cfg.rms_norm_eps))
        return logits, h
