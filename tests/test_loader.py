"""MLX checkpoint loading (qvex.loader; engine/model.py:39-67, 342-397 and
engine/mtp.py:71-73). CPU: config parsing, key prefixes, rejected checkpoints.
GPU: a model and an MTP head written in the MLX format and loaded back give
the in-memory model's logits bit for bit."""

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from qvex.loader import _Shards, load_model
from qvex.model import Config

DEV = "cuda:0"


def test_config_from_file_nested_and_overrides(tmp_path):
    raw = {"text_config": {"hidden_size": 512, "intermediate_size": 1024, "num_hidden_layers": 8,
                           "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 128,
                           "linear_num_key_heads": 2, "linear_num_value_heads": 4, "linear_key_head_dim": 128,
                           "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4, "rms_norm_eps": 1e-6,
                           "vocab_size": 4096, "rope_parameters": {"rope_theta": 5e6, "partial_rotary_factor": 0.5}},
           "quantization": {"group_size": 64, "bits": 4,
                            "language_model.model.layers.3.mlp.down_proj": {"bits": 8, "group_size": 32}}}
    (tmp_path / "config.json").write_text(json.dumps(raw))
    c = Config.from_file(tmp_path / "config.json")
    assert (c.hidden_size, c.num_hidden_layers, c.full_attention_interval) == (512, 8, 4)
    assert c.rope_theta == 5e6 and c.rotary_dim == 64
    assert c.qparams("model.layers.3.mlp.down_proj") == (32, 8)
    assert c.qparams("model.layers.2.mlp.down_proj") == (64, 4)
    assert [c.is_linear(i) for i in range(8)] == [True, True, True, False] * 2


def test_config_defaults_without_text_config(tmp_path):
    raw = {"hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 4, "num_attention_heads": 2,
           "num_key_value_heads": 1, "linear_num_key_heads": 1, "linear_num_value_heads": 2,
           "linear_key_head_dim": 128, "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4,
           "rms_norm_eps": 1e-6, "vocab_size": 100, "rope_theta": 1000.0}
    (tmp_path / "config.json").write_text(json.dumps(raw))
    c = Config.from_file(tmp_path / "config.json")
    assert c.head_dim == 128 and c.rotary_dim == 32 and c.rope_theta == 1000.0
    assert (c.group_size, c.bits, c.quant) == (64, 4, {})


def test_shards_prefixes_and_uint32(tmp_path):
    w = torch.from_numpy(np.arange(8, dtype=np.uint32).reshape(2, 4) * 0x11111111)
    save_file({"language_model.model.norm.weight": torch.ones(4, dtype=torch.bfloat16),
               "model.language_model.embed_tokens.weight": w,
               "vision_tower.blocks.0.weight": torch.zeros(3)}, str(tmp_path / "a.safetensors"))
    save_file({"language_model.lm_head.scales": torch.full((2, 1), 0.5, dtype=torch.bfloat16)},
              str(tmp_path / "b.safetensors"))
    sh = _Shards(sorted(tmp_path.glob("*.safetensors")))
    assert sorted(sh.index) == ["lm_head.scales", "model.embed_tokens.weight", "model.norm.weight"]
    t = sh.get("model.embed_tokens.weight", "cpu")
    assert t.dtype == torch.int32 and np.array_equal(t.numpy().view(np.uint32), w.numpy())
    with pytest.raises(KeyError):
        sh.get("vision_tower.blocks.0.weight", "cpu")


def test_load_rejects_unsanitized_mtp_checkpoint(tmp_path):
    from mlx_ckpt import config_json
    (tmp_path / "config.json").write_text(json.dumps(config_json(Config.tiny(layers=4))))
    save_file({"language_model.mtp.fc.weight": torch.zeros((2, 2), dtype=torch.int32)},
              str(tmp_path / "m.safetensors"))
    with pytest.raises(ValueError, match="unsanitized"):
        load_model(tmp_path, device="cpu")


@pytest.fixture(scope="module")
def tiny_pair(tmp_path_factory):
    from qvex.model import random_model
    from qvex.mtp import random_mtp
    from mlx_ckpt import export_model, export_mtp
    d = tmp_path_factory.mktemp("ckpt")
    m = random_model(Config.tiny(layers=4, vocab=2048), seed=31, device=DEV, max_context=512)
    mtp = random_mtp(m, seed=32)
    export_model(m, d / "model", extra={"vision_tower.patch_embed.weight": torch.ones(4, 4)})
    export_mtp(mtp, d / "mtp-4bit.safetensors")
    return m, mtp, d


@pytest.mark.gpu
def test_loaded_model_matches_in_memory(tiny_pair):
    from qvex.loader import load_model
    m, _, d = tiny_pair
    lm = load_model(d / "model", device=DEV, max_context=512)
    ids = torch.from_numpy(np.random.default_rng(3).integers(0, 2048, 40).astype(np.int32)).reshape(1, -1).to(DEV)
    outs = []
    for model in (m, lm):
        c = model.make_cache()
        a = model(ids, c, last_only=False).float()           # prefill (chunked) path
        b = model(ids[:, :4], c, last_only=False).float()    # fused 4-row path
        e = model(ids[:, 4:5], c, last_only=False).float()   # one token
        outs.append((a, b, e))
    torch.cuda.synchronize()
    for x, y in zip(*outs):
        assert torch.equal(x, y)


@pytest.mark.gpu
def test_loaded_mtp_matches_in_memory(tiny_pair):
    from qvex.loader import load_model, load_mtp
    m, mtp, d = tiny_pair
    lm = load_model(d / "model", device=DEV, max_context=512)
    lmtp = load_mtp(lm, d / "mtp-4bit.safetensors")
    H = m.cfg.hidden_size
    g = torch.Generator(device=DEV).manual_seed(4)
    hid = torch.randn((1, 3, H), generator=g, device=DEV).to(torch.bfloat16)
    nxt = torch.tensor([[5, 77, 901]], dtype=torch.int32, device=DEV)
    ra = mtp(hid, nxt, mtp.make_cache(), last_only=False).float()
    rb = lmtp(hid, nxt, lmtp.make_cache(), last_only=False).float()
    torch.cuda.synchronize()
    assert torch.equal(ra, rb)


@pytest.mark.gpu
@pytest.mark.parametrize("override,match", [({"bits": 7}, "7-bit group-64"),
                                            ({"group_size": 16}, "4-bit group-16"),
                                            ({"bits": 3}, "not a 3-bit row")])
def test_load_rejects_unimplemented_quantization(tmp_path, override, match):
    """Widths outside bits 2-8 / groups 32-128, and tensors whose shape does not
    fit the declared width, raise at load."""
    from qvex import _C
    from qvex.model import random_model
    from mlx_ckpt import export_model
    m = random_model(Config.tiny(layers=4, vocab=1024), seed=33, device=DEV, max_context=256)
    export_model(m, tmp_path, shards=1, overrides={"language_model.model.layers.1.mlp.down_proj": override})
    with pytest.raises(_C.QvexError, match=match):
        load_model(tmp_path, device=DEV)


@pytest.mark.gpu
def test_mixed_width_checkpoint_round_trip(tmp_path):
    """A mixed-width model (per-module overrides, engine/model.py:68-71; the
    reference quantizer's 4/3-bit mix plus 5/6/8-bit modules) written with its
    config's overrides and loaded back computes the same logits bit for bit."""
    from qvex.model import random_model
    from mlx_ckpt import export_model
    quant = {"model.layers.0.mlp.down_proj": {"bits": 3},
             **{f"model.layers.1.linear_attn.{n}": {"bits": 3, "group_size": 128}
                for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a")},
             "model.layers.2.linear_attn.out_proj": {"bits": 6, "group_size": 32},
             "lm_head": {"bits": 8}, "model.embed_tokens": {"bits": 3}}
    cfg = Config.tiny(layers=4, vocab=2048)
    cfg.quant = dict(quant)
    m = random_model(cfg, seed=34, device=DEV, max_context=256)
    export_model(m, tmp_path, shards=2, overrides={"language_model." + k: v for k, v in quant.items()})
    lm = load_model(tmp_path, device=DEV, max_context=256)
    assert lm.cfg.quant == quant
    assert (lm.layers[1].mixer.in_proj.bits, lm.layers[1].mixer.in_proj.group_size) == (3, 128)
    assert (lm.lm_head.bits, lm.embed.bits, lm.layers[2].mixer.out_proj.bits) == (8, 3, 6)
    ids = torch.from_numpy(np.random.default_rng(5).integers(0, 2048, 24).astype(np.int32)).reshape(1, -1).to(DEV)
    outs = []
    for model in (m, lm):
        c = model.make_cache()
        outs.append((model(ids, c, last_only=False).float(), model(ids[:, :3], c, last_only=False).float()))
    torch.cuda.synchronize()
    for x, y in zip(*outs):
        assert torch.equal(x, y)
