"""The Haruka int8 engine on the GPU against the CPU oracle, same converted weights, on a model of Haruka's structure
at a small size (112 px: 1 cls + 8 x 8 tokens, d 768, hidden 256, 64 tags).

Bars, as for the EVA02 engine (tests/test_engine_gpu.py): (1) wiring bit-exact under teacher forcing at the
attention and SwiGLU outputs (qkv and every block output reproduced bit for bit; the SwiGLU output within 2e-3 of
the oracle's), with each block's attention within 4e-3 of float64 attention; the tree-pool head on the engine's
final stream within 3e-3 in probability; (2) end to end within 1.5x the int8 noise budget; (3) graph replay equal to
eager.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import attention as OA
from oracle import haruka as OH
from oracle import model as OM

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def cfgs(depth=2, **kw):
    from foidfinder_amd.haruka import HarukaConfig

    kw = {**dict(img_size=112, depth=depth, hidden=256, tags=64), **kw}
    return HarukaConfig(**kw), OH.HarukaConfig(**kw)


def model(cfg, seed=0):
    from foidfinder_amd.haruka import convert_checkpoint, synthetic_checkpoint

    raw = synthetic_checkpoint(cfg, seed=seed)
    return raw, convert_checkpoint(raw, cfg)


def pixels(n, cfg, seed):
    return np.random.default_rng(seed).integers(0, 256, (n, cfg.img_size, cfg.img_size, 3), dtype=np.uint8)


def test_haruka_wiring_bit_exact(dev):
    from foidfinder_amd.haruka import HarukaInt8

    cfg, ocfg = cfgs(depth=3)
    _, state = model(cfg)
    eng = HarukaInt8(state, cfg, device=dev)
    img = pixels(2, cfg, seed=1)
    trace = {}
    logits = eng.eager(torch.from_numpy(img).to(dev), trace).cpu().numpy()
    st = {k: v.numpy() for k, v in state.items()}
    rope = tuple(t.cpu().numpy() for t in eng.rope)
    want_rope = OM.eva02_rope_tables(cfg.grid, cfg.rope_ref)
    assert all(np.array_equal(a, b) for a, b in zip(rope, want_rope)), "rope tables"
    x = trace["stem"].cpu().numpy()
    want_stem = OH.stem(img, st, ocfg).astype(np.float32)
    assert np.abs(x.astype(np.float32) - want_stem).max() <= 4e-3 * max(1.0, np.abs(want_stem).max()), "stem"
    worst_attn = 0.0
    for i in range(cfg.depth):
        rec = {}
        o_eng, h_eng = trace[f"attn{i}"].cpu().numpy(), trace[f"h{i}"].cpu().numpy()
        x_new = OH.block_int8(x, st, i, ocfg, rope, attention_out=o_eng, hidden_out=h_eng, record=rec)
        qkv_eng = trace[f"qkv{i}"].cpu().numpy()
        assert np.array_equal(rec["qkv"].view(np.uint16), qkv_eng.view(np.uint16)), f"block {i}: qkv differs"
        h_err = np.abs(h_eng.astype(np.float32) - rec["h"].astype(np.float32)).max()
        assert h_err <= 2e-3, f"block {i}: SwiGLU output off by {h_err}"
        x_eng = trace[f"x{i}"].cpu().numpy()
        assert np.array_equal(x_new.view(np.uint16), x_eng.view(np.uint16)), f"block {i}: block output differs"
        o_want = OA.attention(qkv_eng, cfg.tokens, out_dtype=np.float64)
        worst_attn = max(worst_attn, float(np.abs(o_eng.astype(np.float64) - o_want).max()))
        x = x_eng
    assert worst_attn < 4e-3, f"attention max abs err {worst_attn}"
    want = OH.head(x, st, ocfg)
    p, pw = 1 / (1 + np.exp(-logits.astype(np.float64))), 1 / (1 + np.exp(-want))
    assert np.abs(p - pw).max() < 3e-3, f"tree-pool head off by {np.abs(p - pw).max()}"


def test_haruka_end_to_end_within_int8_noise(dev):
    from foidfinder_amd.haruka import HarukaInt8

    cfg, ocfg = cfgs(depth=2)
    raw, state = model(cfg, seed=2)
    img = pixels(2, cfg, seed=3)
    eng = HarukaInt8(state, cfg, device=dev)
    logits = eng.eager(torch.from_numpy(img).to(dev)).cpu().numpy().astype(np.float64)
    assert np.isfinite(logits).all()
    p = 1 / (1 + np.exp(-logits))
    p8 = OH.forward_int8(img, {k: v.numpy() for k, v in state.items()}, ocfg)
    pf = OH.forward_float(img, {k: v.numpy() for k, v in raw.items()}, ocfg)
    err, budget = np.abs(p - p8), np.abs(p8 - pf)
    print(f"engine vs oracle int8: max {err.max():.3e} mean {err.mean():.3e}; "
          f"oracle int8 vs float: max {budget.max():.3e} mean {budget.mean():.3e}", flush=True)
    assert err.max() <= 1.5 * budget.max() and err.mean() <= 1.5 * budget.mean()


def test_haruka_graph_replay_matches_eager(dev):
    from foidfinder_amd.haruka import HarukaInt8

    cfg, _ = cfgs(depth=2)
    eng = HarukaInt8(model(cfg, seed=4)[1], cfg, device=dev)
    a = torch.from_numpy(pixels(3, cfg, seed=5)).to(dev)
    b = torch.from_numpy(pixels(3, cfg, seed=6)).to(dev)
    ea, eb = eng.eager(a), eng.eager(b)
    for i in range(4):
        x = a if i % 2 == 0 else b
        got = eng(x)
        torch.cuda.synchronize()
        want = ea if i % 2 == 0 else eb
        assert torch.equal(got, want), f"replay {i} differs from eager"
        eng.eager(b)
        torch.cuda.synchronize()


def test_haruka_full_size_block_runs(dev):
    """Two blocks at Haruka's real size, 448 px, batch 1: 1025 tokens, d 768 (6 rotation blocks of 128), 12 heads,
    hidden 2048; qkv and block outputs bit-exact with the oracle on the engine's own inputs, finite logits."""
    from foidfinder_amd.haruka import HarukaConfig, HarukaInt8, convert_checkpoint, synthetic_checkpoint

    cfg = HarukaConfig(depth=2, tags=256)
    ocfg = OH.HarukaConfig(depth=2, tags=256)
    state = convert_checkpoint(synthetic_checkpoint(cfg, seed=7), cfg)
    eng = HarukaInt8(state, cfg, device=dev)
    img = pixels(1, cfg, seed=8)
    trace = {}
    logits = eng.eager(torch.from_numpy(img).to(dev), trace)
    assert torch.isfinite(logits).all()
    st = {k: v.numpy() for k, v in state.items()}
    rope = tuple(t.cpu().numpy() for t in eng.rope)
    x = trace["stem"].cpu().numpy()
    for i in range(cfg.depth):
        rec = {}
        x_new = OH.block_int8(x, st, i, ocfg, rope, attention_out=trace[f"attn{i}"].cpu().numpy(),
                              hidden_out=trace[f"h{i}"].cpu().numpy(), record=rec)
        assert np.array_equal(rec["qkv"].view(np.uint16), trace[f"qkv{i}"].cpu().numpy().view(np.uint16))
        assert np.array_equal(x_new.view(np.uint16), trace[f"x{i}"].cpu().numpy().view(np.uint16))
        x = trace[f"x{i}"].cpu().numpy()


def write_folded_dir(path, cfg, seed):
    """A Haruka model directory as foidfinder/haruka.py:convert writes it: fp16 folded tensors + config.json."""
    from safetensors.torch import save_file

    from foidfinder_amd.haruka import synthetic_checkpoint

    sd = synthetic_checkpoint(cfg, seed=seed)
    save_file({k: v.half().contiguous() for k, v in sd.items()}, str(path / "model.safetensors"))
    model = {"name": "Haruka Tagger", "architecture": "haruka-eva02-tree", "img_size": cfg.img_size,
             "patch_size": cfg.patch, "dim": cfg.dim, "heads": cfg.heads, "depth": cfg.depth,
             "mlp_hidden": cfg.hidden, "pool_heads": cfg.pool_heads, "coarse_queries": cfg.coarse,
             "leaf_queries": cfg.leaves, "leaf_dim": cfg.leaf_dim, "rope_ref_grid": cfg.rope_ref}
    tags = [f"t{i}" for i in range(cfg.tags)]
    (path / "config.json").write_text(json.dumps({"model": model, "tags": tags, "categories": ["general"] * cfg.tags,
                                                  "thresholds": {"general": 0.35}}))
    return sd, model, tags


def test_rocm_backend_serves_haruka_model_dirs(dev, tmp_path):
    """Folded (foidfinder/haruka.py:convert) and compressed (foidfinder/haruka_quant.py) Haruka directories load
    through backends.load("rocm", dir); predict(image) -> float32 probabilities [num_tags] after the model card's
    letterbox; the compressed directory, rebuilt from the same codes, predicts what its folded twin predicts."""
    import gzip

    from PIL import Image
    from safetensors.numpy import save_file

    from foidfinder_amd import backends

    cfg, _ = cfgs(depth=2)
    folded = tmp_path / "folded"
    folded.mkdir()
    sd, model_entry, tags = write_folded_dir(folded, cfg, seed=9)
    be = backends.load("rocm", folded)
    assert be.name == "rocm" and be.size == cfg.img_size
    rng = np.random.default_rng(10)
    img = Image.fromarray(rng.integers(0, 256, (90, 140, 3), dtype=np.uint8))
    p = be.predict(img)
    assert p.shape == (cfg.tags,) and p.dtype == np.float32 and ((p > 0) & (p < 1)).all()
    pb = be.predict_batch([img, img.convert("L").convert("RGB"), img])
    assert pb.shape == (3, cfg.tags) and np.array_equal(pb[0], pb[2])

    # compressed twin: the head and block-0 qkv as row steps x codes; the same matrices go into a folded twin
    comp, twin = tmp_path / "compressed", tmp_path / "twin"
    comp.mkdir()
    twin.mkdir()
    tensors, layers, twin_sd = {}, {}, {k: v.half() for k, v in sd.items()}
    for k in ("head.weight", "blocks.0.qkv.weight"):
        w = sd[k].double().numpy()
        step = (np.sqrt((w**2).mean(1)) / 32).astype(np.float16)
        codes = np.rint(w / step.astype(np.float64)[:, None]).astype(np.int64)
        z = np.where(codes >= 0, 2 * codes, -2 * codes - 1).astype(np.uint64)
        n = max(1, (int(z.max()).bit_length() + 7) // 8)
        for i in range(n):
            tensors[f"{k}.plane{i}"] = np.frombuffer(
                gzip.compress(((z >> np.uint64(8 * i)) & np.uint64(0xFF)).astype(np.uint8).tobytes()), np.uint8)
        tensors[k + ".step"] = step
        layers[k] = {"shape": list(w.shape), "planes": n}
        twin_sd[k] = torch.from_numpy((codes * step.astype(np.float32)[:, None].astype(np.float64)).astype(np.float32))
    for k, v in sd.items():
        if k not in layers:
            tensors[k] = v.half().numpy()
    save_file(tensors, str(comp / "model.safetensors"), {"format": "foidfinder-haruka-rowstep1"})
    config = {"model": model_entry, "quantization": {"format": "foidfinder-haruka-rowstep1", "layers": layers},
              "tags": tags, "categories": ["general"] * cfg.tags, "thresholds": {"general": 0.35}}
    (comp / "config.json").write_text(json.dumps(config))
    from safetensors.torch import save_file as save_torch

    save_torch({k: v.contiguous() for k, v in twin_sd.items()}, str(twin / "model.safetensors"))
    (twin / "config.json").write_text(json.dumps({k: v for k, v in config.items() if k != "quantization"}))
    pc = backends.load("rocm", comp).predict(img)
    pt = backends.load("rocm", twin).predict(img)
    assert np.array_equal(pc, pt)


RESIZE_CASES = [(850, 1200), (448, 900), (3, 5000), (5000, 3), (100, 37), (448, 300), (1, 1), (1200, 900), (640, 2000),
                (900, 449), (9, 900), (9, 910), (10, 1001), (448, 448)]


@pytest.mark.parametrize(("w", "h"), RESIZE_CASES)
def test_gpu_letterbox_is_bit_exact_with_pillow(dev, w, h):
    """The Haruka letterbox on the GPU (ff_resample_u8, two passes) against the oracle's letterbox in the pass order of
    Pillow 13, the version the reference pins: the reference's cases (tests/test_haruka.py:36-55), both sides of the
    pass-order boundaries, and an image already at the input size. Where the installed Pillow orders the passes the
    same way, also against Pillow's own Image.resize(BICUBIC) pasted on white (the oracle's passes are pinned against
    Pillow in both orders by the CPU tests)."""
    from PIL import Image

    from foidfinder_amd.backends.rocm.preprocess import PILLOW_MAJOR, letterbox_gpu
    from oracle import resample as ORS

    s = 448
    rgb = np.random.default_rng(w * h).integers(0, 256, (h, w, 3), dtype=np.uint8)
    out = torch.full((s, s, 3), 7, dtype=torch.uint8, device=dev)
    letterbox_gpu(rgb, s, out)
    got = out.cpu().numpy()
    assert np.array_equal(got, ORS.letterbox(rgb, s, 13))
    r = min(s / w, s / h)
    nw, nh = max(1, int(w * r)), max(1, int(h * r))
    if (w, h) == (s, s):
        assert np.array_equal(got, rgb)
    elif ORS.vertical_first(w, h, nw, nh, 13) == ORS.vertical_first(w, h, nw, nh, PILLOW_MAJOR):
        canvas = Image.new("RGB", (s, s), (255, 255, 255))
        canvas.paste(Image.fromarray(rgb).resize((nw, nh), Image.Resampling.BICUBIC), ((s - nw) // 2, (s - nh) // 2))
        assert np.array_equal(got, np.asarray(canvas))


def test_preprocess_haruka_batch(dev):
    """A batch of mixed images: every slot is its own letterbox; transparency is composited onto white."""
    from PIL import Image

    from foidfinder_amd.backends.rocm.preprocess import letterbox_gpu, preprocess_haruka

    rng = np.random.default_rng(11)
    a = Image.fromarray(rng.integers(0, 256, (90, 40, 3), dtype=np.uint8))
    b = Image.fromarray(np.zeros((64, 64, 4), np.uint8), "RGBA")  # fully transparent -> white
    c = Image.fromarray(rng.integers(0, 256, (30, 200), dtype=np.uint8), "L").convert("RGB")
    out = preprocess_haruka([a, b, c], 112, device=dev)
    assert out.shape == (3, 112, 112, 3) and out.dtype == torch.uint8
    assert (out[1] == 255).all()
    for i, im in ((0, a), (2, c)):
        one = torch.empty(112, 112, 3, dtype=torch.uint8, device=dev)
        letterbox_gpu(np.asarray(im), 112, one)
        assert torch.equal(out[i], one)


@pytest.mark.timeout(600)
def test_haruka_config5_full_shape(dev):
    """Haruka at the benchmark's shape: EVA02-B/14-448, 12 blocks, tree pool, 98 782 tags, batch 64 of raw pixels
    (the reference's model, foidfinder/haruka.py:13-27). Properties that hold at any size: finite logits; the graph
    replay equals the eager forward bit for bit; permuting the batch permutes the logits bit for bit (blocks work per
    token or per sequence, and the pool and head GEMMs see the same shapes). And the pool head plus the 98 782-column
    head, on the engine's own final stream of one image, within 3e-3 in probability of the oracle's float64 head."""
    from foidfinder_amd.haruka import HarukaConfig, HarukaInt8, convert_checkpoint, synthetic_checkpoint

    cfg, ocfg = HarukaConfig(), OH.HarukaConfig()
    state = convert_checkpoint(synthetic_checkpoint(cfg, seed=12), cfg)
    eng = HarukaInt8(state, cfg, device=dev)
    img = torch.from_numpy(pixels(64, cfg, seed=13)).to(dev)
    print("haruka batch 64: graph", flush=True)
    full = eng(img).clone()
    torch.cuda.synchronize()
    assert full.shape == (64, 98782) and torch.isfinite(full).all()
    print("haruka batch 64: eager with trace", flush=True)
    trace = {}
    assert torch.equal(eng.eager(img, trace), full), "graph replay differs from eager at batch 64"
    perm = torch.randperm(64, generator=torch.Generator().manual_seed(1)).to(dev)
    shuffled = eng(img[perm].contiguous()).clone()
    torch.cuda.synchronize()
    assert torch.equal(shuffled, full[perm]), "permuting the batch does not permute the logits"
    x0 = trace[f"x{cfg.depth - 1}"][: cfg.tokens].cpu().numpy()
    del trace
    st = {k: v.numpy() for k, v in state.items() if not k.startswith("blocks.")}
    want = OH.head(x0, st, ocfg)[0]
    p, pw = 1 / (1 + np.exp(-full[0].double().cpu().numpy())), 1 / (1 + np.exp(-want))
    assert np.abs(p - pw).max() < 3e-3, f"pool head + head off by {np.abs(p - pw).max()}"
