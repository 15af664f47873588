"""The PixAI int8 engine on the GPU against the CPU oracle, same converted weights, on a model of PixAI's structure
at a small size (112 px, 2 x 2 windows of 4 x 4 tokens, one windowed and one global block).

Bars, as for the EVA02 engine (tests/test_engine_gpu.py): (1) wiring bit-exact under teacher forcing at the
attention and GELU outputs (qkv and every block output reproduced bit for bit; the GELU output within 2e-3 of the
oracle's tanh GELU), with each block's attention within 4e-3 of float64 attention over the right span (window or
grid); (2) end to end within 1.5x the int8 noise budget; (3) graph replay equal to eager.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import pixai as OP

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def cfgs(depth=2):
    from foidfinder_amd.pixai import PixAIConfig

    kw = dict(img_size=112, win=4, pretrain_grid=4, depth=depth, global_blocks=(1,), hidden=256, tags=64)
    return PixAIConfig(**kw), OP.PixAIConfig(**kw)


def model(cfg, seed=0):
    from foidfinder_amd.pixai import convert_checkpoint, synthetic_checkpoint

    raw = synthetic_checkpoint(cfg, seed=seed)
    return raw, convert_checkpoint(raw, cfg)


def images(n, cfg, seed):
    return np.random.default_rng(seed).uniform(-1, 1, (n, cfg.img_size, cfg.img_size, 3)).astype(np.float16)


def test_pixai_wiring_bit_exact(dev):
    from foidfinder_amd.pixai import PixAIInt8

    cfg, ocfg = cfgs(depth=3)
    _, state = model(cfg)
    eng = PixAIInt8(state, cfg, device=dev)
    img = images(2, cfg, seed=1)
    trace = {}
    logits = eng.eager(torch.from_numpy(img).to(dev), trace).cpu().numpy()
    st = {k: v.numpy() for k, v in state.items()}
    rope = {"win": tuple(t.cpu().numpy() for t in eng.rope_win), "glob": tuple(t.cpu().numpy() for t in eng.rope_glob)}
    x = trace["stem"].cpu().numpy()
    want_stem = OP.stem(img, st, ocfg).astype(np.float32)
    assert np.abs(x.astype(np.float32) - want_stem).max() <= 4e-3 * max(1.0, np.abs(want_stem).max()), "stem"
    worst_attn = 0.0
    for i in range(cfg.depth):
        glob = i in cfg.global_blocks
        seq = cfg.tokens if glob else cfg.win_tokens
        rec = {}
        o_eng, h_eng = trace[f"attn{i}"].cpu().numpy(), trace[f"h{i}"].cpu().numpy()
        x_new = OP.block_int8(x, st, i, ocfg, rope["glob" if glob else "win"], seq, attention_out=o_eng,
                              hidden_out=h_eng, record=rec)
        qkv_eng = trace[f"qkv{i}"].cpu().numpy()
        assert np.array_equal(rec["qkv"].view(np.uint16), qkv_eng.view(np.uint16)), f"block {i}: qkv differs"
        h_err = np.abs(h_eng.astype(np.float32) - rec["h"].astype(np.float32)).max()
        assert h_err <= 2e-3, f"block {i}: GELU output off by {h_err}"
        x_eng = trace[f"x{i}"].cpu().numpy()
        assert np.array_equal(x_new.view(np.uint16), x_eng.view(np.uint16)), f"block {i}: block output differs"
        o_want = OA.attention(qkv_eng, seq, out_dtype=np.float64)
        worst_attn = max(worst_attn, float(np.abs(o_eng.astype(np.float64) - o_want).max()))
        x = x_eng
    assert worst_attn < 4e-3, f"attention max abs err {worst_attn}"
    want = OP.pool_head(x, st, ocfg)
    p, pw = 1 / (1 + np.exp(-logits.astype(np.float64))), 1 / (1 + np.exp(-want))
    assert np.abs(p - pw).max() < 3e-3, "pool head"


def test_pixai_end_to_end_within_int8_noise(dev):
    from foidfinder_amd.pixai import PixAIInt8

    cfg, ocfg = cfgs(depth=2)
    raw, state = model(cfg, seed=2)
    img = images(2, cfg, seed=3)
    eng = PixAIInt8(state, cfg, device=dev)
    logits = eng.eager(torch.from_numpy(img).to(dev)).cpu().numpy().astype(np.float64)
    assert np.isfinite(logits).all()
    p = 1 / (1 + np.exp(-logits))
    p8 = OP.forward_int8(img, {k: v.numpy() for k, v in state.items()}, ocfg)
    pf = OP.forward_float(img, {k: v.numpy() for k, v in raw.items()}, ocfg)
    err, budget = np.abs(p - p8), np.abs(p8 - pf)
    print(f"engine vs oracle int8: max {err.max():.3e} mean {err.mean():.3e}; "
          f"oracle int8 vs float: max {budget.max():.3e} mean {budget.mean():.3e}", flush=True)
    assert err.max() <= 1.5 * budget.max() and err.mean() <= 1.5 * budget.mean()


def test_pixai_graph_replay_matches_eager(dev):
    from foidfinder_amd.pixai import PixAIInt8

    cfg, _ = cfgs(depth=2)
    eng = PixAIInt8(model(cfg, seed=4)[1], cfg, device=dev)
    a = torch.from_numpy(images(2, cfg, seed=5)).to(dev)
    b = torch.from_numpy(images(2, cfg, seed=6)).to(dev)
    ea, eb = eng.eager(a), eng.eager(b)
    for i in range(4):
        x = a if i % 2 == 0 else b
        got = eng(x)
        torch.cuda.synchronize()
        want = ea if i % 2 == 0 else eb
        assert torch.equal(got, want), f"replay {i} differs from eager"
        eng.eager(b)
        torch.cuda.synchronize()


def test_pixai_full_size_block_runs(dev):
    """One block pair (windowed, then global) at PixAI's real size, 1008 px, batch 1: 5184 tokens in 9 windows of
    576, the grid RoPE and 5184-token attention, hidden 4736 (37 blocks of 128); qkv bit-exact with the oracle on
    the engine's own inputs, finite logits."""
    from foidfinder_amd.pixai import PixAIConfig, PixAIInt8, convert_checkpoint, synthetic_checkpoint

    cfg = PixAIConfig(depth=2, global_blocks=(1,), tags=256)
    ocfg = OP.PixAIConfig(depth=2, global_blocks=(1,), tags=256)
    state = convert_checkpoint(synthetic_checkpoint(cfg, seed=7), cfg)
    eng = PixAIInt8(state, cfg, device=dev)
    img = images(1, cfg, seed=8)
    trace = {}
    logits = eng.eager(torch.from_numpy(img).to(dev), trace)
    assert torch.isfinite(logits).all()
    st = {k: v.numpy() for k, v in state.items()}
    x = trace["stem"].cpu().numpy()
    for i, span in ((0, "win"), (1, "glob")):
        rope = tuple(t.cpu().numpy() for t in (eng.rope_win if span == "win" else eng.rope_glob))
        rec = {}
        seq = cfg.win_tokens if span == "win" else cfg.tokens
        x_new = OP.block_int8(x, st, i, ocfg, rope, seq, attention_out=trace[f"attn{i}"].cpu().numpy(),
                              hidden_out=trace[f"h{i}"].cpu().numpy(), record=rec)
        assert np.array_equal(rec["qkv"].view(np.uint16), trace[f"qkv{i}"].cpu().numpy().view(np.uint16))
        assert np.array_equal(x_new.view(np.uint16), trace[f"x{i}"].cpu().numpy().view(np.uint16))
        x = trace[f"x{i}"].cpu().numpy()


def test_rocm_backend_serves_a_pixai_model_dir(dev, tmp_path):
    """The reference's model-directory contract (config.json + model.safetensors with official weights, converted
    on load): backends.load("rocm", dir).predict(image) -> probabilities; tag directories of an unknown
    architecture are refused."""
    import json

    from PIL import Image
    from safetensors.torch import save_file

    from foidfinder_amd import backends
    from foidfinder_amd.pixai import synthetic_checkpoint

    cfg, _ = cfgs(depth=2)
    save_file(synthetic_checkpoint(cfg, seed=9), str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(
        {"num_classes": cfg.tags, "foidfinder_rocm": {"img_size": 112, "win": 4, "global_blocks": [1]}}))
    be = backends.load("rocm", tmp_path)
    assert be.name == "rocm" and be.size == 112
    rng = np.random.default_rng(10)
    img = Image.fromarray(rng.integers(0, 256, (90, 140, 3), dtype=np.uint8))
    p = be.predict(img)
    assert p.shape == (cfg.tags,) and p.dtype == np.float32 and ((p > 0) & (p < 1)).all()
    pb = be.predict_batch([img, img.convert("L").convert("RGB"), img])
    assert pb.shape == (3, cfg.tags) and np.array_equal(pb[0], pb[2])
    assert np.abs(pb[0] - p).max() < 0.05  # batch 1 and 3 differ only through the fp16 stem GEMM's blocking
    other = tmp_path / "other"
    other.mkdir()
    (other / "config.json").write_text(json.dumps({"model": {"architecture": "vit-x"}, "categories": ["general"],
                                                   "tags": ["a"]}))
    with pytest.raises(RuntimeError, match="unsupported model architecture"):
        backends.load("rocm", other)


PREPROCESS_CASES = [(900, 1200), (1200, 900), (448, 900), (300, 1500), (37, 100), (60, 45), (112, 112), (3, 400)]


@pytest.mark.parametrize(("h", "w"), PREPROCESS_CASES)
def test_preprocess_matches_the_letterbox_restatement(dev, h, w):
    """backends/rocm/preprocess.py:preprocess (PixAI's letterbox on the GPU) against the float64 restatement of the
    reference's recipe (foidfinder/backends/cuda/preprocess.py:16-32: white compositing, antialiased bilinear resize
    of the longer side to the input size, [-1, 1] normalization, -1 padding): downscales, wide and tall images, an
    enlargement, the identity size and a 3-pixel-high strip. The bar: every pixel within half an fp16 ulp of the
    float64 value plus 2e-5 (the GPU's float32 weights and sums), the padding exactly -1."""
    from PIL import Image

    from foidfinder_amd.backends.rocm.preprocess import preprocess
    from oracle import resample as ORS

    size = 112
    rgb = np.random.default_rng(h * 7 + w).integers(0, 256, (h, w, 3), dtype=np.uint8)
    got = preprocess([Image.fromarray(rgb)], size, device=dev)[0].float().cpu().numpy().astype(np.float64)
    want = ORS.letterbox_pixai(rgb, size)
    bound = 0.5 * np.spacing(np.abs(want).astype(np.float16)).astype(np.float64) + 2e-5
    assert (np.abs(got - want) <= bound).all(), np.abs(got - want).max()
    assert np.array_equal(got[want == -1.0], want[want == -1.0])


def test_preprocess_constant_and_transparent_images(dev):
    """A constant image stays that constant (the filter rows sum to one); a transparent one becomes white (+1); a
    grey image with half-transparent pixels is composited onto white first, as the reference's rgb_on_white."""
    from PIL import Image

    from foidfinder_amd.backends.rocm.preprocess import preprocess

    grey = Image.fromarray(np.full((90, 140, 3), 100, np.uint8))
    clear = Image.fromarray(np.zeros((50, 50, 4), np.uint8), "RGBA")
    half = np.zeros((40, 40, 4), np.uint8)
    half[..., :3], half[..., 3] = 0, 128
    out = preprocess([grey, clear, Image.fromarray(half, "RGBA")], 112, device=dev).float().cpu().numpy()
    nh = int(90 * 112 / 140)
    top = (112 - nh) // 2
    v = np.float16(100 / 255 * 2 - 1)
    assert np.abs(out[0, top : top + nh] - v).max() <= 1e-3 and (out[0, :top] == -1).all()
    assert (out[1] == 1.0).all()
    comp = np.asarray(Image.alpha_composite(Image.new("RGBA", (40, 40), (255,) * 4), Image.fromarray(half, "RGBA")))
    assert np.abs(out[2] - np.float16(comp[0, 0, 0] / 255 * 2 - 1)).max() <= 1e-3
