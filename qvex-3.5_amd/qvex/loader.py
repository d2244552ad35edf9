"""Loading an MLX-format Qwen3.5 checkpoint into the HIP model (the on-disk
format of the reference: engine/model.py:342-397 for the model,
engine/mtp.py:71-73 for the MTP head).

A model directory holds config.json (read by Config.from_file, which follows
engine/model.py:39-67: `text_config` nesting, rope parameters, the
quantization block with per-module overrides) and *.safetensors shards:

* a quantized module `<name>` is `<name>.weight` uint32 [N, K*bits/32] (each
  row a little-endian stream of `bits`-bit codes: for 4 bits, code j of word i
  at bits 4j..4j+3), `<name>.scales` and `<name>.biases` bf16 [N, K/group];
* norms are bf16 [dim]; the GDN conv1d weight is bf16 [conv_dim, K, 1]
  (mx.conv1d's [out, kernel, in/groups]); A_log is read as fp32;
* multimodal checkpoints prefix the language model's keys with
  `language_model.` or `model.language_model.`; every other key (the vision
  tower) is never read.

Tensors are read through safetensors' own loader (no pickle) lazily, one
module at a time, and moved to the device as the layer that uses them is
built. The MTP head lives in a separate file whose metadata carries its
`group_size` and `bits` (written by tools/fetch_mtp.py in the reference).
"""

from __future__ import annotations

from pathlib import Path

import torch
from safetensors import safe_open

from . import _C
from .model import Config, Layer, QEmbedding, QLinear, Qwen35


class _Shards:
    """Name -> tensor over the *.safetensors files of a directory (or one file),
    with the reference's prefix rules (engine/model.py:348-353)."""

    def __init__(self, files: list[Path], strip_language_model: bool = True):
        if not files:
            raise FileNotFoundError("no .safetensors files")
        self._handles = [safe_open(str(f), framework="pt", device="cpu") for f in files]
        self.index: dict[str, tuple[int, str]] = {}
        for i, h in enumerate(self._handles):
            for k in h.keys():
                name = k
                if strip_language_model:
                    if k.startswith("language_model."):
                        name = k[len("language_model."):]
                    elif k.startswith("model.language_model."):
                        name = "model." + k[len("model.language_model."):]
                    else:
                        continue
                self.index[name] = (i, k)

    def metadata(self) -> dict:
        md = {}
        for h in self._handles:
            md.update(h.metadata() or {})
        return md

    def has(self, name: str) -> bool:
        return name in self.index

    def get(self, name: str, device) -> torch.Tensor:
        if name not in self.index:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        i, k = self.index[name]
        t = self._handles[i].get_tensor(k)
        if t.dtype == torch.uint32:
            t = t.view(torch.int32)           # the kernels take the words as int32
        return t.to(device)


def _qlinear(sh: _Shards, prefix: str, group_size: int, bits: int, device) -> QLinear:
    w = sh.get(f"{prefix}.weight", device)
    if w.dtype != torch.int32:
        raise _C.QvexError(f"{prefix}.weight: expected packed uint32 codes, got {w.dtype}")
    return QLinear(w, sh.get(f"{prefix}.scales", device).to(torch.bfloat16),
                   sh.get(f"{prefix}.biases", device).to(torch.bfloat16), group_size, bits)


def _bf16(sh: _Shards, name: str, device) -> torch.Tensor:
    return sh.get(name, device).to(torch.bfloat16).contiguous()


def load_model(model_dir: str | Path, device="cuda", max_context: int = 8192, max_width: int = 8) -> Qwen35:
    """The model of an MLX-format directory (engine/model.py:342-397). Raises on
    an unsanitized checkpoint that still holds MTP tensors, as the reference does,
    and on a quantization the kernels do not implement (bits other than 2, 3, 4,
    5, 6, 8 or groups other than 32, 64, 128). Per-module overrides of the
    config's quantization block (Config.qparams) apply to every linear and to
    the embedding; fused projections must share theirs (QLinear.fuse)."""
    model_dir = Path(model_dir)
    cfg = Config.from_file(model_dir / "config.json")
    sh = _Shards(sorted(model_dir.glob("*.safetensors")))
    if any("mtp." in k for k in sh.index):
        raise ValueError("unsanitized checkpoint (mtp weights present): convert with mlx first")

    def qlin(prefix):
        return _qlinear(sh, prefix, *cfg.qparams(prefix), device)

    layers = []
    for i in range(cfg.num_hidden_layers):
        pre = f"model.layers.{i}"
        p = {
            "input_layernorm": _bf16(sh, f"{pre}.input_layernorm.weight", device),
            "post_attention_layernorm": _bf16(sh, f"{pre}.post_attention_layernorm.weight", device),
            "mlp": {n: qlin(f"{pre}.mlp.{n}") for n in ("gate_proj", "up_proj", "down_proj")},
        }
        if cfg.is_linear(i):
            la = f"{pre}.linear_attn"
            conv = _bf16(sh, f"{la}.conv1d.weight", device)
            p["linear_attn"] = {
                **{n: qlin(f"{la}.{n}") for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj")},
                "conv1d": conv.reshape(conv.shape[0], -1).contiguous(),      # [conv_dim, K, 1] -> [conv_dim, K]
                "A_log": sh.get(f"{la}.A_log", device).float().contiguous(),
                "dt_bias": _bf16(sh, f"{la}.dt_bias", device),
                "norm": _bf16(sh, f"{la}.norm.weight", device),
            }
        else:
            sa = f"{pre}.self_attn"
            p["self_attn"] = {
                **{n: qlin(f"{sa}.{n}") for n in ("q_proj", "k_proj", "v_proj", "o_proj")},
                "q_norm": _bf16(sh, f"{sa}.q_norm.weight", device),
                "k_norm": _bf16(sh, f"{sa}.k_norm.weight", device),
            }
        layers.append(Layer(cfg, i, p))

    e = "model.embed_tokens"
    gs, bits = cfg.qparams(e)
    embed = QEmbedding(sh.get(f"{e}.weight", device), _bf16(sh, f"{e}.scales", device),
                       _bf16(sh, f"{e}.biases", device), gs, bits)
    model = Qwen35(cfg, embed, layers, _bf16(sh, "model.norm.weight", device), qlin("lm_head"),
                   max_context=max_context, max_width=max_width)
    model.offload_mlx()          # one device copy of each weight: the packed one
    return model


def load_mtp(model: Qwen35, path: str | Path, hidden_mode: str = "pre"):
    """The MTP head of a separate safetensors file (engine/mtp.py:71-73):
    group size and bits from the file's metadata (default 64 / 4); the head
    shares the model's embedding and lm_head."""
    from .mtp import MTPHead

    sh = _Shards([Path(path)], strip_language_model=False)
    md = sh.metadata()
    gs, bits = int(md.get("group_size", 64)), int(md.get("bits", 4))
    dev = model.norm.device

    def qlin(prefix):
        return _qlinear(sh, prefix, gs, bits, dev)

    sa, mlp = "mtp.layers.0.self_attn", "mtp.layers.0.mlp"
    w = {
        "fc": qlin("mtp.fc"),
        "norm_emb": _bf16(sh, "mtp.pre_fc_norm_embedding.weight", dev),
        "norm_hid": _bf16(sh, "mtp.pre_fc_norm_hidden.weight", dev),
        "norm_out": _bf16(sh, "mtp.norm.weight", dev),
        "ln1": _bf16(sh, "mtp.layers.0.input_layernorm.weight", dev),
        "ln2": _bf16(sh, "mtp.layers.0.post_attention_layernorm.weight", dev),
        "attn": {**{n: qlin(f"{sa}.{n}") for n in ("q_proj", "k_proj", "v_proj", "o_proj")},
                 "q_norm": _bf16(sh, f"{sa}.q_norm.weight", dev), "k_norm": _bf16(sh, f"{sa}.k_norm.weight", dev)},
        "mlp": {n: qlin(f"{mlp}.{n}") for n in ("gate_proj", "up_proj", "down_proj")},
    }
    head = MTPHead(model, w, gs, bits, hidden_mode)
    head.offload_mlx()
    return head
