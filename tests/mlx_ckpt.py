"""Write a model built in memory back to the MLX checkpoint format that
qvex.loader reads (the reference's key names and layouts, engine/model.py:
342-397 and engine/mtp.py:18-46): test helper, not a converter."""

from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors.torch import save_file


def _q(out: dict, name: str, w: torch.Tensor, s: torch.Tensor, b: torch.Tensor) -> None:
    out[f"{name}.weight"] = w.contiguous().cpu().view(torch.uint32)
    out[f"{name}.scales"] = s.contiguous().cpu()
    out[f"{name}.biases"] = b.contiguous().cpu()


def _split(out: dict, fused, names_rows: list[tuple[str, int]]) -> None:
    r0 = 0
    for name, rows in names_rows:
        _q(out, name, fused.w[r0:r0 + rows], fused.scales[r0:r0 + rows], fused.biases[r0:r0 + rows])
        r0 += rows
    assert r0 == fused.N


def config_json(cfg, overrides: dict | None = None) -> dict:
    text = {k: getattr(cfg, k) for k in (
        "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
        "head_dim", "linear_num_key_heads", "linear_num_value_heads", "linear_key_head_dim",
        "linear_value_head_dim", "linear_conv_kernel_dim", "full_attention_interval", "rms_norm_eps",
        "vocab_size")}
    text["rope_parameters"] = {"rope_theta": cfg.rope_theta, "partial_rotary_factor": cfg.rotary_dim / cfg.head_dim}
    quant = {"group_size": cfg.group_size, "bits": cfg.bits, **(overrides or {})}
    return {"model_type": "qwen3_5", "text_config": text, "quantization": quant}


def export_model(model, out_dir: Path, shards: int = 2, extra: dict | None = None,
                 overrides: dict | None = None) -> None:
    """model -> out_dir/config.json + model-0000i.safetensors with the
    `language_model.` prefix (plus `extra` tensors, e.g. a vision tower)."""
    cfg = model.cfg
    t: dict[str, torch.Tensor] = {}
    H, I = cfg.hidden_size, cfg.intermediate_size
    for i, layer in enumerate(model.layers):
        pre = f"model.layers.{i}"
        t[f"{pre}.input_layernorm.weight"] = layer.ln1.cpu()
        t[f"{pre}.post_attention_layernorm.weight"] = layer.ln2.cpu()
        _split(t, layer.mlp.gate_up, [(f"{pre}.mlp.gate_proj", I), (f"{pre}.mlp.up_proj", I)])
        d = layer.mlp.down
        _q(t, f"{pre}.mlp.down_proj", d.w, d.scales, d.biases)
        m = layer.mixer
        if layer.linear:
            la = f"{pre}.linear_attn"
            _split(t, m.in_proj, [(f"{la}.in_proj_qkv", m.conv_dim), (f"{la}.in_proj_z", m.value_dim),
                                  (f"{la}.in_proj_b", m.hv), (f"{la}.in_proj_a", m.hv)])
            _q(t, f"{la}.out_proj", m.out_proj.w, m.out_proj.scales, m.out_proj.biases)
            t[f"{la}.conv1d.weight"] = m.conv_w.cpu().reshape(m.conv_dim, m.K, 1).contiguous()
            t[f"{la}.A_log"] = m.A_log.cpu()
            t[f"{la}.dt_bias"] = m.dt_bias.cpu()
            t[f"{la}.norm.weight"] = m.norm_w.cpu()
        else:
            sa = f"{pre}.self_attn"
            D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
            _split(t, m.qkv_proj, [(f"{sa}.q_proj", Hq * 2 * D), (f"{sa}.k_proj", Hkv * D),
                                   (f"{sa}.v_proj", Hkv * D)])
            _q(t, f"{sa}.o_proj", m.o_proj.w, m.o_proj.scales, m.o_proj.biases)
            t[f"{sa}.q_norm.weight"] = m.q_norm.cpu()
            t[f"{sa}.k_norm.weight"] = m.k_norm.cpu()
    e = model.embed
    _q(t, "model.embed_tokens", e.w, e.scales, e.biases)
    t["model.norm.weight"] = model.norm.cpu()
    lm = model.lm_head
    _q(t, "lm_head", lm.w, lm.scales, lm.biases)
    keys = sorted(t)
    out_dir.mkdir(parents=True, exist_ok=True)
    for s in range(shards):
        part = {"language_model." + k: t[k] for k in keys[s::shards]}
        if s == 0 and extra:
            part.update(extra)
        save_file(part, str(out_dir / f"model-{s + 1:05d}-of-{shards:05d}.safetensors"))
    (out_dir / "config.json").write_text(json.dumps(config_json(cfg, overrides)))


def export_mtp(mtp, path: Path, group_size: int = 64, bits: int = 4) -> None:
    t: dict[str, torch.Tensor] = {}
    _q(t, "mtp.fc", mtp.fc.w, mtp.fc.scales, mtp.fc.biases)
    t["mtp.pre_fc_norm_embedding.weight"] = mtp.norm_emb.cpu()
    t["mtp.pre_fc_norm_hidden.weight"] = mtp.norm_hid.cpu()
    t["mtp.norm.weight"] = mtp.norm_out.cpu()
    layer, cfg = mtp.layer, mtp.model.cfg
    t["mtp.layers.0.input_layernorm.weight"] = layer.ln1.cpu()
    t["mtp.layers.0.post_attention_layernorm.weight"] = layer.ln2.cpu()
    sa, m = "mtp.layers.0.self_attn", layer.mixer
    D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
    _split(t, m.qkv_proj, [(f"{sa}.q_proj", Hq * 2 * D), (f"{sa}.k_proj", Hkv * D), (f"{sa}.v_proj", Hkv * D)])
    _q(t, f"{sa}.o_proj", m.o_proj.w, m.o_proj.scales, m.o_proj.biases)
    t[f"{sa}.q_norm.weight"] = m.q_norm.cpu()
    t[f"{sa}.k_norm.weight"] = m.k_norm.cpu()
    I = cfg.intermediate_size
    _split(t, layer.mlp.gate_up, [("mtp.layers.0.mlp.gate_proj", I), ("mtp.layers.0.mlp.up_proj", I)])
    d = layer.mlp.down
    _q(t, "mtp.layers.0.mlp.down_proj", d.w, d.scales, d.biases)
    save_file(t, str(path), metadata={"group_size": str(group_size), "bits": str(bits)})
