"""Host-side logic on the CPU: weight conversion against the oracle, RoPE tables, configuration checks, the backend
registry and bench.py's single-GPU contract."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from foidfinder_amd import engine as E
from oracle import model as OM

ROOT = Path(__file__).resolve().parents[1]


def test_hadamard_matches_oracle():
    for n in (2, 128, 1024):
        np.testing.assert_array_equal(E.hadamard(n).numpy(), OM.hadamard(n))


def test_quantize_rows_matches_oracle(rng):
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    q, s = E.quantize_rows_int8(torch.from_numpy(w))
    q0, s0 = OM.quantize_rows_int8(w)
    np.testing.assert_array_equal(q.numpy(), q0)
    np.testing.assert_array_equal(s.numpy(), s0)


def test_convert_checkpoint_matches_oracle_conversion():
    cfg = E.Eva02Config(img_size=56, depth=2, tags=32)
    raw = E.synthetic_checkpoint(cfg, seed=2)
    conv = E.convert_checkpoint(raw, cfg)
    ocfg = OM.Eva02Config(img_size=56, depth=2, tags=32)
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        blk = {
            "qkv_w": raw[p + "attn.qkv.weight"].numpy(), "qkv_b": raw[p + "attn.qkv.bias"].numpy(),
            "proj_w": raw[p + "attn.proj.weight"].numpy(), "proj_b": raw[p + "attn.proj.bias"].numpy(),
            "fc1_w": raw[p + "mlp.fc1.weight"].numpy(), "fc1_b": raw[p + "mlp.fc1.bias"].numpy(),
            "fc2_w": raw[p + "mlp.fc2.weight"].numpy(), "fc2_b": raw[p + "mlp.fc2.bias"].numpy(),
        }
        for n in ("norm1", "norm2"):
            blk[n + "_w"], blk[n + "_b"] = raw[p + n + ".weight"].numpy(), raw[p + n + ".bias"].numpy()
        blk["mlp_norm_w"], blk["mlp_norm_b"] = raw[p + "mlp.norm.weight"].numpy(), raw[p + "mlp.norm.bias"].numpy()
        want = OM.convert_block(blk, ocfg)
        names = {"qkv": "attn.qkv", "proj": "attn.proj", "fc1": "mlp.fc1", "fc2": "mlp.fc2"}
        for short, long in names.items():
            for f in ("qweight", "wscale", "bias"):
                np.testing.assert_array_equal(conv[p + long + "." + f].numpy(), want[f"{short}.{f}"], err_msg=long + f)


def test_weight_rotation_matches_oracle_bit_for_bit(rng):
    for block, k in ((1024, 1024), (128, 2816)):
        w = (rng.standard_normal((40, k)) * 0.02).astype(np.float32)
        np.testing.assert_array_equal(E.rotate_rows64(torch.from_numpy(w), block).numpy(), OM.rotate_rows64(w, block))


def test_rope_tables_match_oracle():
    for grid in (2, 8, 32):
        c, s = E.eva02_rope_tables(grid, 16)
        c0, s0 = OM.eva02_rope_tables(grid, 16)
        np.testing.assert_array_equal(c.numpy(), c0)
        np.testing.assert_array_equal(s.numpy(), s0)


def test_config_validation():
    with pytest.raises(ValueError):
        E.Eva02Config(dim=768, heads=12).validate()
    with pytest.raises(ValueError):
        E.Eva02Config(hidden_pad=2800).validate()
    E.Eva02Config().validate()
    cfg = E.Eva02Config()
    assert cfg.tokens == 1025 and cfg.grid == 32
    ops = cfg.gemm_ops(32)
    assert sum(ops.values()) == pytest.approx(19.81e12, rel=2e-3)  # per batch-32 forward, unpadded dims
    assert cfg.attention_flops(32) == pytest.approx(3.305e12, rel=2e-3)


def test_backend_registry_without_gpu():
    from foidfinder_amd import backends

    assert backends.NAMES == ("mlx", "cuda", "rocm")
    with pytest.raises(ValueError, match="unknown backend"):
        backends.load("bogus", Path("."))
    with pytest.raises(RuntimeError):
        backends.load("cuda", Path("."))
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="no AMD GPU"):
            backends.load("rocm", Path("."))
        with pytest.raises(RuntimeError, match="no supported accelerator"):
            backends.detect()


def test_model_dir_round_trip(tmp_path):
    cfg = E.Eva02Config(img_size=56, depth=1, tags=8)
    state = E.convert_checkpoint(E.synthetic_checkpoint(cfg, seed=1), cfg)
    E.save_model_dir(tmp_path, state, cfg, [f"t{i}" for i in range(8)], ["general"] * 7 + ["rating"],
                     {"general": 0.35, "rating": 0.5})
    cfg_json = (tmp_path / "config.json").read_text()
    assert '"architecture": "eva02-int8"' in cfg_json
    from safetensors.torch import load_file

    back = load_file(str(tmp_path / "model.safetensors"))
    assert set(back) == set(state)
    assert torch.equal(back["blocks.0.mlp.fc1.qweight"], state["blocks.0.mlp.fc1.qweight"])


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
