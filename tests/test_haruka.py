"""Haruka Tagger host logic and its oracle, on the CPU: config, weight conversion, the compressed checkpoint format,
the stem, the tree-pool head against the model card's formulation, and the int8 forward against the float forward."""

from __future__ import annotations

import gzip
import json

import numpy as np
import pytest

from oracle import haruka as OH
from oracle import model as OM

torch = pytest.importorskip("torch")


def small_cfgs(**kw):
    from foidfinder_amd.haruka import HarukaConfig

    kw = {**dict(img_size=112, depth=2, hidden=256, tags=64), **kw}
    return HarukaConfig(**kw), OH.HarukaConfig(**kw)


def np_state(sd):
    return {k: v.numpy() for k, v in sd.items()}


def test_config_from_model_entry():
    from foidfinder_amd.haruka import HarukaConfig

    # config.json "model" entry as written by foidfinder/haruka.py:13-27, 101-110
    model = {"name": "Haruka Tagger", "architecture": "haruka-eva02-tree", "img_size": 448, "patch_size": 14,
             "dim": 768, "heads": 12, "depth": 12, "mlp_hidden": 2048, "pool_heads": 16, "coarse_queries": 6,
             "leaf_queries": 18, "leaf_dim": 64, "rope_ref_grid": 16}
    cfg = HarukaConfig.from_model(model, tags=98782)
    assert cfg == HarukaConfig()
    cfg.validate()
    assert cfg.tokens == 1025 and cfg.grid == 32
    assert HarukaConfig.from_model(model, tags=10, depth=2).depth == 2
    with pytest.raises(ValueError):
        HarukaConfig(dim=700).validate()


def test_synthetic_checkpoint_has_the_folded_layout():
    from foidfinder_amd.haruka import synthetic_checkpoint

    cfg, _ = small_cfgs()
    sd = synthetic_checkpoint(cfg)
    d, h, g = cfg.dim, cfg.hidden, cfg.grid
    # names and shapes of foidfinder/haruka.py:fold
    want = {"patch_w": (d, 14 * 14 * 3), "patch_b": (g * g, d), "cls": (1, d), "norm.weight": (d,),
            "pool.kv.weight": (2 * d, d), "pool.q_coarse": (6, d), "pool.q_coarse_bias": (6,), "pool.q_child": (18, d),
            "pool.q_child_bias": (18,), "pool.leaf.weight": (18, d, 64), "pool.leaf.bias": (18, 64),
            "head.weight": (64, 18 * 64), "blocks.1.qkv.weight": (3 * d, d), "blocks.1.fc1.weight": (2 * h, d),
            "blocks.1.fc2.weight": (d, h), "blocks.1.mlp_norm.weight": (h,)}
    for k, shape in want.items():
        assert tuple(sd[k].shape) == shape, k
    for n in ("norm", "trunk_norm", "child_q_norm", "leaf_norm"):
        assert f"pool.{n}.bias" in sd
    assert (sd["blocks.0.qkv.bias"][d : 2 * d] == 0).all()  # EVA02 has no k bias (foidfinder/haruka.py:55-57)


def test_convert_checkpoint_matches_oracle():
    from foidfinder_amd.haruka import convert_checkpoint, synthetic_checkpoint

    cfg, ocfg = small_cfgs()
    raw = synthetic_checkpoint(cfg, seed=3)
    conv = convert_checkpoint(raw, cfg)
    want = OH.convert_checkpoint(np_state(raw), ocfg)
    assert set(conv) == set(want)
    for k in conv:
        a, b = conv[k].numpy(), want[k]
        assert a.dtype == b.dtype and np.array_equal(a, b), k
    # fc1 rows interleave gate j and value j, so the dequantized rotated rows are the original rows times H128
    w = raw["blocks.0.fc1.weight"].double().numpy()
    deq = conv["blocks.0.fc1.qweight"].double().numpy() * conv["blocks.0.fc1.wscale"].double().numpy()[:, None]
    back = (deq.reshape(2 * cfg.hidden, -1, 128) @ OM.hadamard(128)).reshape(deq.shape)  # H128 is its own inverse
    assert np.abs(back[0::2] - w[: cfg.hidden]).max() < 2e-3 and np.abs(back[1::2] - w[cfg.hidden :]).max() < 2e-3


def zigzag_planes(codes: np.ndarray) -> list[bytes]:
    """The download format's encoding, written from its description (foidfinder/haruka_quant.py:1-15): zigzag the
    codes (0, -1, 1, -2, ... -> 0, 1, 2, 3, ...), split into as many byte planes as the largest needs, gzip each."""
    c = codes.astype(np.int64).ravel()
    z = np.where(c >= 0, 2 * c, -2 * c - 1).astype(np.uint64)
    n = max(1, (int(z.max()).bit_length() + 7) // 8)
    return [gzip.compress(((z >> np.uint64(8 * i)) & np.uint64(0xFF)).astype(np.uint8).tobytes()) for i in range(n)]


def test_decode_planes_known_answers_and_round_trip():
    from foidfinder_amd.haruka import decode_planes

    # hand-computed: codes 0, -1, 1, -128, 200 -> zigzag 0, 1, 2, 255, 400 = 0x0190 -> low bytes / high bytes
    lo = bytes([0, 1, 2, 255, 0x90])
    hi = bytes([0, 0, 0, 0, 0x01])
    got = decode_planes([gzip.compress(lo), gzip.compress(hi)], (1, 5))
    assert got.tolist() == [[0, -1, 1, -128, 200]]
    # signs, zero, a zero row and codes needing a second plane (the reference's round-trip case shape)
    codes = np.random.default_rng(0).integers(-300, 301, (5, 128)).astype(np.int32)
    codes[0, :4] = [0, -1, 1, -128]
    codes[1] = 0
    planes = zigzag_planes(codes)
    assert len(planes) == 2
    assert np.array_equal(decode_planes(planes, codes.shape), codes)
    small = np.array([[3, -3, 0, 127]], np.int32)  # |zigzag| < 256: one plane
    assert len(zigzag_planes(small)) == 1 and np.array_equal(decode_planes(zigzag_planes(small), (1, 4)), small)


def test_load_compressed_rebuilds_code_times_row_step(tmp_path):
    from safetensors.numpy import save_file

    from foidfinder_amd.haruka import load_compressed

    rng = np.random.default_rng(1)
    codes = rng.integers(-200, 201, (6, 40)).astype(np.int32)
    step = (rng.uniform(1e-4, 1e-3, 6)).astype(np.float16)
    planes = zigzag_planes(codes)
    tensors = {"head.weight.step": step, "cls": rng.standard_normal((1, 8)).astype(np.float16)}
    for i, p in enumerate(planes):
        tensors[f"head.weight.plane{i}"] = np.frombuffer(p, np.uint8)
    save_file(tensors, str(tmp_path / "model.safetensors"))
    out = load_compressed(tmp_path, {"head.weight": {"shape": [6, 40], "planes": len(planes)}})
    assert set(out) == {"head.weight", "cls"}
    assert np.array_equal(out["head.weight"].numpy(), codes.astype(np.float32) * step.astype(np.float32)[:, None])
    assert np.array_equal(out["cls"].numpy(), tensors["cls"])


def test_oracle_stem_is_a_strided_convolution():
    _, ocfg = small_cfgs()
    rng = np.random.default_rng(2)
    d, p, g = ocfg.dim, ocfg.patch, ocfg.grid
    state = {"patch_w": rng.standard_normal((d, p * p * 3)) * 1e-4, "patch_b": rng.standard_normal((g * g, d)) * 0.02,
             "cls": rng.standard_normal((1, d)) * 0.02}
    img = rng.integers(0, 256, (1, ocfg.img_size, ocfg.img_size, 3)).astype(np.float32)
    x = OH.stem(img, state, ocfg).astype(np.float64).reshape(ocfg.tokens, d)
    assert np.array_equal(x[0], state["cls"][0].astype(np.float16).astype(np.float64))
    r, c = 3, 5  # token 1 + r*g + c is the patch at grid row r, column c
    patch = img[0, r * p : (r + 1) * p, c * p : (c + 1) * p, :]
    w = state["patch_w"].reshape(d, p, p, 3)
    direct = np.array([sum(w[o, kh, kw, ch] * patch[kh, kw, ch] for kh in range(p) for kw in range(p)
                           for ch in range(3)) for o in range(6)]) + state["patch_b"][r * g + c, :6]
    assert np.abs(x[1 + r * g + c, :6] - direct).max() < 1e-3 * max(1.0, np.abs(direct).max())


def model_card_pool(xn, s, cfg):
    """The model card's MHAttnPool (tests/test_haruka.py:65-116 of the reference) in float64 torch, on unfolded
    parameters: explicit 1/sqrt(head_dim) on the logits, child queries broadcast as [coarse, branches], leaves by
    einsum."""
    F = torch.nn.functional
    t = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in s.items()}
    B, N, D = xn.shape
    Hp, C, Q = cfg.pool_heads, cfg.coarse, cfg.leaves
    hd, br = D // Hp, Q // C
    scale = hd**-0.5
    kw, vw = t["pool.kv.weight"][:D] / scale, t["pool.kv.weight"][D:]  # unfold the key scale
    kb, vb = t["pool.kv.bias"][:D] / scale, t["pool.kv.bias"][D:]

    def ln(x, n):
        return F.layer_norm(x, (D,), t[f"pool.{n}.weight"], t[f"pool.{n}.bias"], cfg.eps)

    x = ln(torch.from_numpy(xn), "norm")
    k = F.linear(x, kw, kb).view(B, N, Hp, hd).transpose(1, 2)
    v = F.linear(x, vw, vb).view(B, N, Hp, hd).transpose(1, 2)
    q_c = t["pool.q_coarse"].view(1, C, D).expand(B, C, D).reshape(B, C, Hp, hd).transpose(1, 2)
    lc = (q_c @ k.transpose(-2, -1)) * scale
    ac = torch.softmax(lc, dim=-2) * torch.sigmoid(lc + t["pool.q_coarse_bias"].view(1, 1, C, 1))
    z_coarse = ln((ac @ v).transpose(1, 2).reshape(B, C, D), "trunk_norm")
    q_leaf = ln((z_coarse.unsqueeze(2) + t["pool.q_child"].view(1, C, br, D)).reshape(B, Q, D), "child_q_norm")
    ll = (q_leaf.reshape(B, Q, Hp, hd).transpose(1, 2) @ k.transpose(-2, -1)) * scale
    al = torch.softmax(ll, dim=-2) * torch.sigmoid(ll + t["pool.q_child_bias"].view(1, 1, Q, 1))
    z_child = (al @ v).transpose(1, 2).reshape(B, C, br, D)
    z_tree = ln((z_coarse.unsqueeze(2) + z_child).reshape(B, Q, D), "leaf_norm")
    mass = al.sum(-1).mean(1).unsqueeze(-1)
    leaf = torch.einsum("bqd,qdf->bqf", z_tree * (mass / (mass + 4.0)), t["pool.leaf.weight"]) + t["pool.leaf.bias"]
    return F.linear(leaf.reshape(B, -1), t["head.weight"], t["head.bias"]).numpy()


def test_oracle_pool_head_matches_the_model_card_form():
    from foidfinder_amd.haruka import synthetic_checkpoint

    cfg, ocfg = small_cfgs()
    s = np_state(synthetic_checkpoint(cfg, seed=4))
    xn = np.random.default_rng(5).standard_normal((2, ocfg.tokens, ocfg.dim))
    got = OH.pool_head(xn, s, ocfg)
    want = model_card_pool(xn, {k: v for k, v in s.items() if k.startswith(("pool.", "head."))}, ocfg)
    assert got.shape == (2, ocfg.tags)
    assert np.abs(got - want).max() < 1e-9 * max(1.0, np.abs(want).max())
    # the query biases reach the output (so the comparison above covers the sigmoid gate too)
    s2 = dict(s)
    s2["pool.q_coarse_bias"] = s["pool.q_coarse_bias"] + 1.0
    assert np.abs(OH.pool_head(xn, s2, ocfg) - got).max() > 1e-3


def test_oracle_int8_forward_within_float_budget():
    from foidfinder_amd.haruka import convert_checkpoint, synthetic_checkpoint

    cfg, ocfg = small_cfgs()
    raw = synthetic_checkpoint(cfg, seed=6)
    conv = np_state(convert_checkpoint(raw, cfg))
    img = np.random.default_rng(7).integers(0, 256, (2, cfg.img_size, cfg.img_size, 3)).astype(np.float32)
    p8 = OH.forward_int8(img, conv, ocfg)
    pf = OH.forward_float(img, np_state(raw), ocfg)
    assert np.isfinite(p8).all() and p8.shape == (2, cfg.tags)
    err = np.abs(p8 - pf)
    assert err.max() < 0.05 and err.mean() < 0.01, (err.max(), err.mean())


def test_model_dir_config_is_recognized(tmp_path):
    """load_haruka_dir refuses a directory of another architecture before touching the GPU."""
    from foidfinder_amd.haruka import load_haruka_dir

    (tmp_path / "config.json").write_text(json.dumps({"model": {"architecture": "eva02-int8"}, "tags": []}))
    with pytest.raises(RuntimeError, match="not a Haruka model"):
        load_haruka_dir(tmp_path)


RESIZE_CASES = [(850, 1200), (448, 900), (3, 5000), (5000, 3), (100, 37), (448, 300), (1, 1), (1200, 900),
                (640, 2000), (900, 449), (9, 900), (9, 910), (10, 1001)]
# the reference's cases (tests/test_haruka.py:36-47), a few more, and both sides of Pillow 12's pass-order boundary


def pillow_letterbox(rgb, s=448):
    """The model card's letterbox by Pillow itself (the reference's tests/test_haruka.py:19-34)."""
    from PIL import Image

    h, w = rgb.shape[:2]
    if (w, h) == (s, s):
        return rgb
    r = min(s / w, s / h)
    nw, nh = max(1, int(w * r)), max(1, int(h * r))
    canvas = Image.new("RGB", (s, s), (255, 255, 255))
    canvas.paste(Image.fromarray(rgb).resize((nw, nh), Image.Resampling.BICUBIC), ((s - nw) // 2, (s - nh) // 2))
    return np.asarray(canvas)


@pytest.mark.parametrize(("w", "h"), RESIZE_CASES)
def test_oracle_letterbox_is_bit_exact_with_pillow(w, h):
    from foidfinder_amd.backends.rocm.preprocess import PILLOW_MAJOR

    from oracle import resample as ORS

    rgb = np.random.default_rng(w * h).integers(0, 256, (h, w, 3), dtype=np.uint8)
    assert np.array_equal(ORS.letterbox(rgb, 448, PILLOW_MAJOR), pillow_letterbox(rgb))


def test_pass_order_rules():
    import importlib

    P = importlib.import_module("foidfinder_amd.backends.rocm.preprocess")  # the module, not the function it exports

    from oracle import resample as ORS

    for w, h in RESIZE_CASES:
        r = min(448 / w, 448 / h)
        nw, nh = max(1, int(w * r)), max(1, int(h * r))
        assert P.vertical_first(w, h, nw, nh) == ORS.vertical_first(w, h, nw, nh, 13)  # the served rule: Pillow 13
    # the reference's rule for Pillow 13 (its resize_pad): (448, 900) shrinks the height over twice as much
    assert ORS.vertical_first(448, 900, 223, 448, 13) and not ORS.vertical_first(850, 1200, 317, 448, 13)


def test_bicubic_taps_match_the_oracle():
    from foidfinder_amd.backends.rocm.preprocess import bicubic_taps

    from oracle import resample as ORS

    for n_in, n_out in ((850, 448), (1200, 448), (3, 1), (5000, 448), (37, 165), (100, 448), (1, 448), (448, 448),
                        (900, 449), (7, 3)):
        kk, b = bicubic_taps(n_in, n_out)
        kk_o, b_o = ORS.coeffs(n_in, n_out)
        assert np.array_equal(kk, kk_o) and np.array_equal(b, b_o), (n_in, n_out)
        assert (b[:, 0] >= 0).all() and (b.sum(1) <= n_in).all() and (b[:, 1] <= kk.shape[1]).all()
        # each row of taps sums to 1 in 22-bit fixed point, within the rounding of its taps
        assert (np.abs(kk.sum(1).astype(np.int64) - (1 << 22)) <= kk.shape[1]).all()


def test_bicubic_taps_match_the_pillow_known_answers():
    """The reference's own Pillow tap tables (web/src/engine/engine.test.ts:8-34), kept as a fixture."""
    from pathlib import Path

    from foidfinder_amd.backends.rocm.preprocess import bicubic_taps

    from oracle import resample as ORS

    cases = json.loads((Path(__file__).parent / "golden" / "pillow_bicubic_taps.json").read_text())["cases"]
    assert len(cases) == 5
    for key, want in cases.items():
        n_in, n_out = map(int, key.split("->"))
        for kk, b in (bicubic_taps(n_in, n_out), ORS.coeffs(n_in, n_out)):
            flat = kk.astype(np.int64).ravel()
            assert kk.shape[1] == want["ksize"], key
            assert kk[0].tolist() == want["row0"], key
            assert int((flat * np.arange(1, flat.size + 1)).sum()) == want["checksum"], key
            assert int(b.astype(np.int64).sum()) == want["boundsSum"], key
            assert b[0].tolist() == want["first"] and b[-1].tolist() == want["last"], key
