"""The EVA02 int8 engine on the GPU against the CPU oracle, same converted weights.

Why three bars. Every block kernel is bit-exact with the oracle on identical inputs (tests/test_kernels_gpu.py),
except attention, whose fp32 MFMA sums cannot be restated bit for bit on the CPU. Attention mixes all tokens, and
every rotate+quant downstream turns a last-bit change into occasional one-step code flips. So a single ulp of
difference grows, within a block or two, to the size of the int8 quantization noise itself (the oracle's own int8
forward differs from the unquantized float forward by the same amount). Hence:

  1. wiring, bit-exact: the oracle takes the engine's stem output and per-block attention outputs (teacher forcing)
     and must reproduce every qkv and every block output bit for bit;
  2. attention per block: within 4e-3 absolute of float64 attention on the engine's own qkv;
  3. end to end: |p_engine - p_oracle_int8| within 1.5x the int8 noise budget |p_oracle_int8 - p_float|
     (max and mean over tags and images), with the logits finite.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import model as OM

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def engine_cfg(depth=2, img=112, tags=512):
    from foidfinder_amd.engine import Eva02Config

    return Eva02Config(img_size=img, depth=depth, tags=tags)


def oracle_cfg(cfg):
    return OM.Eva02Config(img_size=cfg.img_size, depth=cfg.depth, tags=cfg.tags)


def raw_and_converted(cfg, seed=0):
    from foidfinder_amd.engine import convert_checkpoint, synthetic_checkpoint

    raw = synthetic_checkpoint(cfg, seed=seed)
    return raw, convert_checkpoint(raw, cfg)


def float_weights(raw, cfg) -> OM.FloatWeights:
    n = {k: v.numpy() for k, v in raw.items()}
    w = OM.FloatWeights(cfg=cfg, patch_w=n["patch_embed.weight"], patch_b=n["patch_embed.bias"], cls=n["cls_token"],
                        pos=n["pos_embed"], norm_w=n["norm.weight"], norm_b=n["norm.bias"], head_w=n["head.weight"],
                        head_b=n["head.bias"])
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        w.blocks.append({
            "norm1_w": n[p + "norm1.weight"], "norm1_b": n[p + "norm1.bias"], "qkv_w": n[p + "attn.qkv.weight"],
            "qkv_b": n[p + "attn.qkv.bias"], "proj_w": n[p + "attn.proj.weight"], "proj_b": n[p + "attn.proj.bias"],
            "norm2_w": n[p + "norm2.weight"], "norm2_b": n[p + "norm2.bias"], "fc1_w": n[p + "mlp.fc1.weight"],
            "fc1_b": n[p + "mlp.fc1.bias"], "mlp_norm_w": n[p + "mlp.norm.weight"], "mlp_norm_b": n[p + "mlp.norm.bias"],
            "fc2_w": n[p + "mlp.fc2.weight"], "fc2_b": n[p + "mlp.fc2.bias"],
        })
    return w


def check_wiring(eng, state, cfg, images, dev):
    trace = {}
    logits = eng.eager(torch.from_numpy(images).to(dev), trace).cpu().numpy()
    np_state = {k: v.cpu().numpy() for k, v in state.items()}
    ocfg = oracle_cfg(cfg)
    blocks = OM.blocks_from_state(np_state, cfg.depth)
    rope = (eng.rope[0].cpu().numpy(), eng.rope[1].cpu().numpy())  # the kernel's inputs, pinned on the CPU
    x = trace["stem"].cpu().numpy()
    want_stem = OM.stem(images, OM.float_weights_from_state(np_state, ocfg))
    assert np.abs(x.astype(np.float32) - want_stem.astype(np.float32)).max() <= 2e-3 * max(1.0, np.abs(want_stem).max())
    worst_attn = 0.0
    for i, qb in enumerate(blocks):
        rec = {}
        o_eng = trace[f"attn{i}"].cpu().numpy()
        h_eng = trace[f"h{i}"].cpu().numpy()
        x_new = OM.block_int8(x, qb, ocfg, rope, attention_out=o_eng, hidden_out=h_eng, record=rec)
        h_want = rec["h"].astype(np.float32)
        ulp = np.maximum(np.spacing(np.abs(rec["h"])), np.spacing(np.abs(h_eng))).astype(np.float32)
        assert (np.abs(h_eng.astype(np.float32) - h_want) <= ulp).all(), f"block {i}: SwiGLU output beyond one ulp"
        qkv_eng = trace[f"qkv{i}"].cpu().numpy()
        assert np.array_equal(rec["qkv"].view(np.uint16), qkv_eng.view(np.uint16)), f"block {i}: qkv differs"
        x_eng = trace[f"x{i}"].cpu().numpy()
        assert np.array_equal(x_new.view(np.uint16), x_eng.view(np.uint16)), f"block {i}: block output differs"
        worst_attn = max(worst_attn, float(np.abs(o_eng.astype(np.float64) - OA.attention(qkv_eng, cfg.tokens, out_dtype=np.float64)).max()))
        x = x_eng
    assert worst_attn < 4e-3, f"attention max abs err {worst_attn}"
    head_p = OM.head(x, OM.float_weights_from_state(np_state, ocfg))
    p = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    assert np.abs(p - head_p).max() < 2e-3, "head"
    return logits


def test_engine_wiring_bit_exact(dev):
    from foidfinder_amd.engine import Eva02Int8

    cfg = engine_cfg(depth=3)
    _, state = raw_and_converted(cfg)
    images = OM.synthetic_images(3, cfg.img_size, seed=5)
    check_wiring(Eva02Int8(state, cfg, device=dev), state, cfg, images, dev)


def test_engine_end_to_end_within_int8_noise(dev):
    from foidfinder_amd.engine import Eva02Int8

    cfg = engine_cfg(depth=2)
    raw, state = raw_and_converted(cfg)
    images = OM.synthetic_images(3, cfg.img_size, seed=5)
    eng = Eva02Int8(state, cfg, device=dev)
    logits = eng.eager(torch.from_numpy(images).to(dev)).cpu().numpy().astype(np.float64)
    assert np.isfinite(logits).all()
    p = 1.0 / (1.0 + np.exp(-logits))
    p_int8 = OM.forward_int8_state(images, {k: v.numpy() for k, v in state.items()}, oracle_cfg(cfg))
    p_float = OM.forward_float(images, float_weights(raw, oracle_cfg(cfg)))
    err, budget = np.abs(p - p_int8), np.abs(p_int8 - p_float)
    print(f"engine vs oracle int8: max {err.max():.3e} mean {err.mean():.3e}; "
          f"oracle int8 vs float: max {budget.max():.3e} mean {budget.mean():.3e}", flush=True)
    assert err.max() <= 1.5 * budget.max() and err.mean() <= 1.5 * budget.mean()


def test_graph_replay_matches_eager(dev):
    from foidfinder_amd.engine import Eva02Int8

    cfg = engine_cfg(depth=3)
    eng = Eva02Int8(raw_and_converted(cfg, seed=1)[1], cfg, device=dev)
    images = torch.from_numpy(OM.synthetic_images(2, cfg.img_size, seed=6)).to(dev)
    other = torch.from_numpy(OM.synthetic_images(2, cfg.img_size, seed=7)).to(dev)
    eager = eng.eager(images)
    eager_other = eng.eager(other)
    for i in range(4):  # replays interleaved with eager work and synchronizations
        x = images if i % 2 == 0 else other
        got = eng(x)
        torch.cuda.synchronize()
        want = eager if i % 2 == 0 else eager_other
        assert torch.equal(got, want), f"replay {i} differs from eager: {(got - want).abs().max().item()}"
        eng.eager(other)
        torch.cuda.synchronize()


def test_engine_full_eva02_l_wiring(dev):
    """EVA02-L/14-448, all 24 blocks, 1025 tokens (the throughput metric's model) at batch 1, teacher-forced."""
    from foidfinder_amd.engine import Eva02Config, Eva02Int8

    cfg = Eva02Config()
    _, state = raw_and_converted(cfg, seed=3)
    images = OM.synthetic_images(1, cfg.img_size, seed=8)
    check_wiring(Eva02Int8(state, cfg, device=dev), state, cfg, images, dev)


def test_full_size_batch_32_is_permutation_equivariant(dev):
    """The benchmark's configuration itself (EVA02-L/14-448, batch 32) through properties that hold at any size:
    every block kernel works row by row (GEMMs exact in int32, rotations per token) or sequence by sequence
    (attention), and the stem and head GEMMs see the same shapes, so permuting the batch permutes the logits bit for
    bit; and the graph replay equals the eager forward bit for bit. (A batch of 1 against a batch of 32 is not
    compared: the third-party stem and head GEMMs pick their algorithm by M, which may round differently.)"""
    from foidfinder_amd.engine import Eva02Config, Eva02Int8

    cfg = Eva02Config()
    _, state = raw_and_converted(cfg, seed=4)
    eng = Eva02Int8(state, cfg, device=dev)
    images = torch.from_numpy(OM.synthetic_images(32, cfg.img_size, seed=9)).to(dev)
    full = eng(images).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(full).all()
    assert torch.equal(eng.eager(images), full), "graph replay differs from eager at batch 32"
    perm = torch.randperm(32, generator=torch.Generator().manual_seed(0)).to(dev)
    shuffled = eng(images[perm].contiguous()).clone()
    torch.cuda.synchronize()
    assert torch.equal(shuffled, full[perm]), "permuting the batch does not permute the logits"
