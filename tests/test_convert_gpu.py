"""Weight conversion on the GPU (the engines convert device tensors at load time, as the reference's `convert` and
loader do on CUDA, foidfinder/cli.py:143-161 and foidfinder/backends/cuda/engine.py:68-70) against the oracle's
conversion on the CPU, and the int8 checkpoint format written and read back.

The rotation product W blockdiag(H) is a float64 FWHT with a fixed butterfly order on both sides, so the device
result must be the oracle's bit for bit: int8 codes, fp32 scales and biases, at the real layer shapes of each model
family (EVA02-L 1024 / 3072 / 2 x 2816 / 2816, PixAI 1024 / 4736, Haruka 768 / 2048)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import haruka as OH
from oracle import model as OM
from oracle import pixai as OP

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def assert_same(got: dict, want: dict, keys):
    for k in keys:
        a, b = got[k].cpu().numpy(), want[k]
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert np.array_equal(a, b), f"{k}: {int((a != b).sum())} of {a.size} entries differ"


def test_eva02_conversion_on_device_matches_oracle(dev):
    from foidfinder_amd.engine import Eva02Config, convert_checkpoint, synthetic_checkpoint

    cfg = Eva02Config(depth=2, tags=64)
    raw = synthetic_checkpoint(cfg, seed=21)
    conv = convert_checkpoint({k: v.to(dev) for k, v in raw.items()}, cfg)
    ocfg = OM.Eva02Config(depth=2, tags=64)
    names = {"qkv": "attn.qkv", "proj": "attn.proj", "fc1": "mlp.fc1", "fc2": "mlp.fc2"}
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        n = {k[len(p):]: v.numpy() for k, v in raw.items() if k.startswith(p)}
        blk = {"qkv_w": n["attn.qkv.weight"], "qkv_b": n["attn.qkv.bias"], "proj_w": n["attn.proj.weight"],
               "proj_b": n["attn.proj.bias"], "fc1_w": n["mlp.fc1.weight"], "fc1_b": n["mlp.fc1.bias"],
               "fc2_w": n["mlp.fc2.weight"], "fc2_b": n["mlp.fc2.bias"], "norm1_w": n["norm1.weight"],
               "norm1_b": n["norm1.bias"], "norm2_w": n["norm2.weight"], "norm2_b": n["norm2.bias"],
               "mlp_norm_w": n["mlp.norm.weight"], "mlp_norm_b": n["mlp.norm.bias"]}
        want = OM.convert_block(blk, ocfg)
        remapped = {p + names[k.split(".")[0]] + "." + k.split(".")[1]: v for k, v in want.items() if "." in k}
        assert_same(conv, remapped, remapped)
    assert conv["blocks.0.mlp.fc1.qweight"].shape == (2 * cfg.hidden_pad, cfg.dim)


def test_pixai_conversion_on_device_matches_oracle(dev):
    from foidfinder_amd.pixai import PixAIConfig, convert_checkpoint, synthetic_checkpoint

    kw = dict(img_size=112, win=4, pretrain_grid=4, depth=2, global_blocks=(1,), tags=64)  # PixAI's hidden 4736
    cfg, ocfg = PixAIConfig(**kw), OP.PixAIConfig(**kw)
    raw = synthetic_checkpoint(cfg, seed=22)
    conv = convert_checkpoint({k: v.to(dev) for k, v in raw.items()}, cfg)
    want = OP.convert_checkpoint({k: v.numpy() for k, v in raw.items()}, ocfg)
    assert set(conv) == set(want)
    assert_same(conv, want, want)
    assert conv["blocks.0.mlp.fc2.qweight"].shape == (1024, 4736)


def test_haruka_conversion_on_device_matches_oracle(dev):
    from foidfinder_amd.haruka import HarukaConfig, convert_checkpoint, synthetic_checkpoint

    kw = dict(img_size=112, depth=2, tags=64)  # Haruka's d 768 and hidden 2048
    cfg, ocfg = HarukaConfig(**kw), OH.HarukaConfig(**kw)
    raw = synthetic_checkpoint(cfg, seed=23)
    conv = convert_checkpoint({k: v.to(dev) for k, v in raw.items()}, cfg)
    want = OH.convert_checkpoint({k: v.numpy() for k, v in raw.items()}, ocfg)
    assert set(conv) == set(want)
    assert_same(conv, want, want)


def test_pixai_int8_dir_round_trip(dev, tmp_path):
    """An official PixAI directory converted on the GPU into the reference's int8 format (engine.py:44-62) loads
    without conversion and predicts exactly what converting on load predicts."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    from foidfinder_amd.pixai import PixAIConfig, load_pixai_dir, synthetic_checkpoint, write_int8_dir

    kw = dict(img_size=112, win=4, pretrain_grid=4, depth=2, global_blocks=(1,), hidden=256, tags=64)
    cfg = PixAIConfig(**kw)
    src, out = tmp_path / "official", tmp_path / "int8"
    src.mkdir()
    save_file(synthetic_checkpoint(cfg, seed=24), str(src / "model.safetensors"))
    (src / "config.json").write_text(json.dumps(
        {"num_classes": cfg.tags, "foidfinder_rocm": {"img_size": 112, "win": 4, "global_blocks": [1]}}))
    write_int8_dir(src, out, device=dev)
    with safe_open(str(out / "model.safetensors"), "pt") as f:
        assert f.metadata() == {"format": "foidfinder-pixai-int8-v1"}
        assert f.get_tensor("blocks.0.attn.qkv.qweight").dtype == torch.int8
        assert f.get_tensor("blocks.1.mlp.fc2.wscale").dtype == torch.float32
    assert json.loads((out / "config.json").read_text()) == json.loads((src / "config.json").read_text())
    eng_a, _ = load_pixai_dir(src, device=dev)
    eng_b, _ = load_pixai_dir(out, device=dev)
    img = torch.from_numpy(np.random.default_rng(25).uniform(-1, 1, (2, 112, 112, 3)).astype(np.float16)).to(dev)
    assert torch.equal(eng_a.eager(img), eng_b.eager(img))
