"""PixAI Tagger v1.0 host logic and its oracle, on the CPU: window layout, axial RoPE tables, window-ordered
patchify, stem, attention-pool head, checkpoint conversion, and the int8 forward against the float forward."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pixai as OP

torch = pytest.importorskip("torch")


def small_cfgs():
    from foidfinder_amd.pixai import PixAIConfig

    kw = dict(img_size=112, win=4, pretrain_grid=4, depth=2, global_blocks=(1,), hidden=256, tags=64)
    return PixAIConfig(**kw), OP.PixAIConfig(**kw)


def test_window_perm_layout():
    from foidfinder_amd.pixai import PixAIConfig, window_perm

    for cfg in (PixAIConfig(), small_cfgs()[0]):
        ocfg = OP.PixAIConfig(img_size=cfg.img_size, win=cfg.win, pretrain_grid=cfg.pretrain_grid)
        perm = window_perm(cfg).numpy()
        assert np.array_equal(perm, OP.window_perm(ocfg))
        assert np.array_equal(np.sort(perm), np.arange(cfg.tokens))  # a bijection onto the grid
        g, w, n = cfg.grid, cfg.win, cfg.win_tokens
        for wr in range(cfg.windows):  # window (wr, wc) starts at its top-left grid cell
            for wc in range(cfg.windows):
                assert perm[(wr * cfg.windows + wc) * n] == wr * w * g + wc * w
        steps = np.diff(perm.reshape(-1, w), axis=1)
        assert (steps == 1).all()  # one column per step inside a window row


def test_axial_rope_tables():
    from foidfinder_amd.pixai import axial_rope

    for end, scale in ((24, 1.0), (72, 24 / 72), (4, 1.0), (8, 0.5)):
        cos, sin = axial_rope(end, scale)
        want_c, want_s = OP.axial_rope64(end, scale)
        assert cos.dtype == torch.float32 and cos.shape == (end * end, 32)
        # fp32 angle products: a few ulps of angles up to ~24 rad
        assert np.abs(cos.numpy() - want_c).max() < 8e-6 and np.abs(sin.numpy() - want_s).max() < 8e-6
    cos, sin = axial_rope(24, 1.0)
    assert (cos[0] == 1).all() and (sin[0] == 0).all()  # position (0, 0): identity
    assert abs(float(sin[1, 0]) - np.sin(1.0)) < 1e-7  # column 1, pair 0: 1 rad
    assert abs(float(sin[24, 16]) - np.sin(1.0)) < 1e-7  # row 1, pair 16: 1 rad
    assert float(sin[1, 16]) == 0.0  # row 0: no rotation in the row pairs


def test_oracle_rope_closed_forms():
    c, s = OP.axial_rope64(24, 1.0)
    assert np.allclose(c[0], 1) and np.allclose(s[0], 0)
    assert np.isclose(s[1, 0], np.sin(1.0)) and np.isclose(s[24, 16], np.sin(1.0)) and s[1, 16] == 0
    assert np.isclose(s[2, 1], np.sin(2.0 * 10000.0 ** (-4.0 / 64)))


def test_patchify_window_order():
    from foidfinder_amd.pixai import PixAIInt8

    cfg, ocfg = small_cfgs()
    rng = np.random.default_rng(0)
    img = rng.standard_normal((2, cfg.img_size, cfg.img_size, 3)).astype(np.float16)
    got = PixAIInt8.patchify(type("E", (), {"cfg": cfg})(), torch.from_numpy(img)).numpy()
    want = OP.patchify(img, ocfg).reshape(-1, 14 * 14 * 3)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # patches that encode their grid cell come out in window_perm order
    g, p = cfg.grid, cfg.patch
    cells = np.arange(g * g, dtype=np.float32).reshape(g, g)
    img = np.repeat(np.repeat(cells, p, 0), p, 1)[None, :, :, None].repeat(3, axis=3)
    tokens = OP.patchify(img, ocfg)[0]
    assert np.array_equal(tokens[:, 0], OP.window_perm(ocfg).astype(np.float32))
    assert (tokens == tokens[:, :1]).all()


def test_oracle_stem_is_a_strided_convolution():
    _, ocfg = small_cfgs()
    rng = np.random.default_rng(1)
    d, p = ocfg.dim, ocfg.patch
    state = {
        "patch_embed.proj.weight": rng.standard_normal((d, 3, p, p)).astype(np.float32) * 0.02,
        "pos_embed": np.zeros((1, 1 + ocfg.pretrain_grid**2, d), np.float32),
        "ln_pre.weight": np.ones(d, np.float32),
        "ln_pre.bias": np.zeros(d, np.float32),
    }
    img = rng.uniform(-1, 1, (1, ocfg.img_size, ocfg.img_size, 3)).astype(np.float32)
    x = OP.stem(img, state, ocfg).astype(np.float64)
    # token 5 in window order: grid cell perm[5]; its embedding by a direct convolution sum, then LayerNorm
    cell = OP.window_perm(ocfg)[5]
    r, c = divmod(int(cell), ocfg.grid)
    patch = img[0, r * p : (r + 1) * p, c * p : (c + 1) * p, :]  # [kh, kw, ch]
    w = state["patch_embed.proj.weight"].astype(np.float64)
    e = np.array([sum(w[o, ch, kh, kw] * patch[kh, kw, ch] for ch in range(3) for kh in range(p) for kw in range(p))
                  for o in range(8)])
    full = np.einsum("ocij,ijc->o", w, patch.astype(np.float64))
    assert np.allclose(full[:8], e)
    ln = (full - full.mean()) / np.sqrt(full.var() + ocfg.eps)
    assert np.abs(x[5] - ln).max() < 4e-3


def test_oracle_pool_head_against_torch_sdpa():
    _, ocfg = small_cfgs()
    rng = np.random.default_rng(2)
    d, L = ocfg.dim, ocfg.tokens
    s = {
        "head_pool.norm.weight": 1 + 0.02 * rng.standard_normal(d),
        "head_pool.norm.bias": 0.02 * rng.standard_normal(d),
        "head_pool.pos_embed": 0.02 * rng.standard_normal((L, d)),
        "head_pool.q": 0.5 * rng.standard_normal((1, 1, d)),
        "head_pool.kv.weight": 0.02 * rng.standard_normal((2 * d, d)),
        "head_pool.kv.bias": 0.02 * rng.standard_normal(2 * d),
        "head_pool.proj.weight": 0.02 * rng.standard_normal((d, d)),
        "head_pool.proj.bias": 0.02 * rng.standard_normal(d),
        "head.weight": 0.05 * rng.standard_normal((ocfg.tags, d)),
        "head.bias": 0.02 * rng.standard_normal(ocfg.tags),
    }
    x = rng.standard_normal((2 * L, d))
    got = OP.pool_head(x, s, ocfg)
    t = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in s.items()}
    perm = torch.from_numpy(OP.window_perm(ocfg))
    F = torch.nn.functional
    h = F.layer_norm(torch.from_numpy(x).view(2, L, d), (d,), t["head_pool.norm.weight"], t["head_pool.norm.bias"],
                     ocfg.eps) + t["head_pool.pos_embed"][perm]
    k, v = F.linear(h, t["head_pool.kv.weight"], t["head_pool.kv.bias"]).view(2, L, 2, 16, 64).permute(2, 0, 3, 1, 4)
    q = t["head_pool.q"].view(1, 16, 1, 64).expand(2, 16, 1, 64)
    o = F.scaled_dot_product_attention(q, k.contiguous(), v.contiguous()).reshape(2, d)
    want = F.linear(F.linear(o, t["head_pool.proj.weight"], t["head_pool.proj.bias"]), t["head.weight"], t["head.bias"])
    assert np.abs(got - want.numpy()).max() < 1e-9


def test_convert_checkpoint_matches_oracle():
    from foidfinder_amd.pixai import config_from_state, convert_checkpoint, synthetic_checkpoint

    cfg, ocfg = small_cfgs()
    raw = synthetic_checkpoint(cfg, seed=3)
    assert config_from_state(raw, img_size=112, win=4, global_blocks=(1,)) == cfg
    conv = convert_checkpoint(raw, cfg)
    want = OP.convert_checkpoint({k: v.numpy() for k, v in raw.items()}, ocfg)
    assert set(conv) == set(want)
    for k in conv:
        a, b = conv[k].numpy(), want[k]
        assert a.dtype == b.dtype and np.array_equal(a, b), k
    assert conv["blocks.1.mlp.fc2.qweight"].shape == (1024, cfg.hidden)


def test_oracle_int8_forward_within_float_budget():
    from foidfinder_amd.pixai import convert_checkpoint, synthetic_checkpoint

    cfg, ocfg = small_cfgs()
    raw = synthetic_checkpoint(cfg, seed=4)
    conv = {k: v.numpy() for k, v in convert_checkpoint(raw, cfg).items()}
    rng = np.random.default_rng(5)
    img = rng.uniform(-1, 1, (2, cfg.img_size, cfg.img_size, 3)).astype(np.float32)
    p8 = OP.forward_int8(img, conv, ocfg)
    pf = OP.forward_float(img, {k: v.numpy() for k, v in raw.items()}, ocfg)
    assert np.isfinite(p8).all() and p8.shape == (2, cfg.tags)
    err = np.abs(p8 - pf)
    assert err.max() < 0.05 and err.mean() < 0.01, (err.max(), err.mean())


@pytest.mark.parametrize(("h", "w", "nh", "nw"), [(900, 1200, 84, 112), (37, 100, 41, 112), (20, 30, 75, 112),
                                                (1200, 1200, 112, 112), (5, 3000, 1, 112), (1008, 700, 1008, 700)])
def test_bilinear_aa_matrix_is_torch_antialiased_bilinear(h, w, nh, nw):
    """The oracle's filter rows against torch's own interpolate(bilinear, antialias=True) on the CPU in float64 (the
    function PixAI's preprocessing calls through torchvision, foidfinder/backends/cuda/preprocess.py:27-28):
    downscales by 1 to 27, enlargements, a one-row output and the identity."""
    import torch.nn.functional as F

    from oracle import resample as ORS

    x = np.random.default_rng(h * w).random((h, w, 3))
    got = F.interpolate(torch.from_numpy(x).permute(2, 0, 1)[None], size=(nh, nw), mode="bilinear",
                        align_corners=False, antialias=True)[0].permute(1, 2, 0).numpy()
    want = ORS.resize_2d(x, ORS.bilinear_aa_matrix(h, nh), ORS.bilinear_aa_matrix(w, nw))
    assert np.abs(got - want).max() < 1e-12
    assert np.allclose(ORS.bilinear_aa_matrix(h, nh).sum(1), 1.0)


def test_write_int8_dir_format(tmp_path):
    """The converted PixAI directory (the reference's `foidfinder convert` output, cli.py:143-161): format metadata,
    the reference's key set (engine.py:49-62) and the oracle's codes; a second conversion is refused."""
    import json

    from safetensors import safe_open
    from safetensors.torch import save_file

    from foidfinder_amd.pixai import synthetic_checkpoint, write_int8_dir

    cfg, ocfg = small_cfgs()
    raw = synthetic_checkpoint(cfg, seed=31)
    src, out = tmp_path / "official", tmp_path / "int8"
    src.mkdir()
    save_file(raw, str(src / "model.safetensors"))
    (src / "config.json").write_text(json.dumps(
        {"num_classes": cfg.tags, "foidfinder_rocm": {"img_size": 112, "win": 4, "global_blocks": [1]}}))
    write_int8_dir(src, out, device="cpu")
    want = OP.convert_checkpoint({k: v.numpy() for k, v in raw.items()}, ocfg)
    with safe_open(str(out / "model.safetensors"), "np") as f:
        assert f.metadata() == {"format": "foidfinder-pixai-int8-v1"}
        assert set(f.keys()) == set(want)
        for k in want:
            assert np.array_equal(f.get_tensor(k), want[k]), k
    with pytest.raises(RuntimeError, match="already in the int8 format"):
        write_int8_dir(out, tmp_path / "again", device="cpu")
