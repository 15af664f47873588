"""The EVA02 int8 engine on the GPU against the CPU oracle, same converted weights.

Why these bars. Every block kernel is bit-exact with the oracle on identical inputs (tests/test_kernels_gpu.py),
except attention, whose fp32 MFMA sums cannot be restated bit for bit on the CPU. Attention mixes all tokens, and
every rotate+quant downstream turns a last-bit change into occasional one-step code flips. So a single ulp of
difference grows, within a block or two, to the size of the int8 quantization noise itself (the oracle's own int8
forward differs from the unquantized float forward by the same amount). Hence:

  1. wiring, bit-exact: the oracle takes the engine's stem output and per-block attention outputs (teacher forcing)
     and must reproduce every qkv and every block output bit for bit;
  2. attention per block: within 4e-3 absolute of float64 attention on the engine's own qkv;
  3. end to end on a small model (2 blocks, 112 px): |p_engine - p_oracle_int8| within 1.5x the int8 noise budget
     |p_oracle_int8 - p_float| (max and mean over tags and images), with the logits finite;
  4. end to end at the benchmark's model (24 blocks, 1025 tokens) against stated bars (E2E_REL_MAX, E2E_MEAN_DP and
     E2E_RMS_REL_X): max |dp| and max |dlogit| within a stated multiple of the int8 noise measured on the same images
     (the int8 oracle against the float forward), mean |dp|, the reference's decision-stability rule, the same top-1
     tag and gap-filtered top-k, against both the int8 oracle and the float forward.
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


def test_full_size_logits_do_not_depend_on_gemm_variants(dev):
    """EVA02-L/14-448 at batch 1 (1025 tokens, 24 blocks): every GEMM tile variant is bit-exact in int32 and
    applies the same epilogue arithmetic, so the logits are bit-identical whichever variants the autotune picks.
    Checked with the autotune's own picks (graph replay) against each variant forced on all four GEMMs (eager)."""
    from foidfinder_amd import kernels as K
    from foidfinder_amd.engine import GEMMS, Eva02Config, Eva02Int8

    cfg = Eva02Config()
    _, state = raw_and_converted(cfg, seed=5)
    eng = Eva02Int8(state, cfg, device=dev)
    images = torch.from_numpy(OM.synthetic_images(1, cfg.img_size, seed=10)).to(dev)
    tuned = eng(images).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(tuned).all()
    picks = {name: eng.variants[(name, 1)] for name in GEMMS}
    for v in range(1, K.lib().ff_gemm_s8_variants() + 1):
        for name in GEMMS:
            eng.variants[(name, 1)] = v
        forced = eng.eager(images)
        assert torch.equal(forced, tuned), (f"variant {v} on every GEMM differs from the autotuned picks {picks}: "
                                            f"{(forced - tuned).abs().max().item()}")


# The stated end-to-end bars at the benchmark's model (EVA02-L/14-448, 24 blocks, 1025 tokens), without teacher
# forcing, against each reference: max |dp| and max |dlogit| over all tags and images at most E2E_REL_MAX times the
# int8 noise (the same maxima of the int8 oracle against the float forward, on the same images), mean |dp| at most
# E2E_MEAN_DP. Reasoning and measurements are in the docstring of the test.
E2E_REL_MAX = {"int8 oracle": 1.1, "float": 1.25}
E2E_MEAN_DP = 0.005
E2E_RMS_REL_X = 0.12  # rms(x_engine - x_oracle) / rms(x_oracle) for the residual stream after the last block
E2E_IMAGES = 6  # seeded images through the full-depth end-to-end comparison


def decision_flips(p, p_ref):
    """The reference's decision-stability rule (tests/test_cuda_engine.py:55-57): a tag the reference scores above
    0.65 must stay above 0.5, one below 0.35 must stay below 0.5. Returns the number of violations."""
    return int(((p_ref > 0.65) & (p <= 0.5)).sum() + ((p_ref < 0.35) & (p >= 0.5)).sum())


def gap_filtered_topk(logits, ref, kmax=50):
    """Per image, every k <= kmax whose reference logit gap between rank k and rank k + 1 exceeds twice that image's
    largest logit error: the engine's top-k set must be the reference's. Returns (checked k count, mismatches)."""
    checked, bad = 0, []
    for i in range(ref.shape[0]):
        err = np.abs(logits[i] - ref[i]).max()
        order = np.argsort(-ref[i])
        srt = ref[i][order]
        mine = np.argsort(-logits[i])
        for k in range(1, kmax + 1):
            if srt[k - 1] - srt[k] > 2 * err:
                checked += 1
                if set(mine[:k]) != set(order[:k]):
                    bad.append((i, k))
    return checked, bad


@pytest.mark.timeout(900)
def test_full_depth_eva02_l_end_to_end(dev):
    """EVA02-L/14-448 (24 blocks, 1025 tokens) on E2E_IMAGES seeded images through the served path (graph replay), against the
    int8 oracle forward and against the float64 forward of the same weights, with no teacher forcing.

    Why these bars. Every block kernel is bit-exact with the oracle on identical inputs except attention (fp32 MFMA
    sums, hardware exp2, p rounded to fp16 for the PV product), whose fp16 outputs differ from float64 attention by a
    few ulps. The next rotate+quant maps values of ~38 code steps to codes, so a relative change of ~1e-3 moves a few
    percent of the codes by one step; such flips recur in every block, and the engine and the int8 oracle drift apart
    like two int8 models with independent rounding. Measured at this seed: rms relative difference of the residual
    stream 1.2 % after block 1 and 8.2 % after block 24, against 2.0 % and 10.0 % between the int8 oracle and the
    float forward (the int8 noise itself). On the 6 images the int8 oracle itself differs from the float forward by
    max |dp| 0.158 (per image 0.116, 0.148, 0.139, 0.109, 0.158, 0.128) and max |dlogit| 0.995, with head weights
    N(0, 0.05) over LayerNorm outputs: sigmoid outputs cannot agree to 2e-3, and the reference's own bar for its int8
    engine against the fp32 model on its real checkpoint, max |dp| < 0.15 (tests/test_cuda_engine.py:54), is below
    this synthetic model's int8 noise. The engine measured max |dp| 0.138 and max |dlogit| 0.759 against the int8
    oracle (0.87 and 0.76 of the noise), 0.147 and 0.984 against the float forward (0.93 and 0.99). The bars: max
    |dp| and max |dlogit| at most 1.1 times the noise against the int8 oracle and 1.25 times against the float
    forward (E2E_REL_MAX: the engine is one more int8 model whose maxima over a few images scatter like the
    oracle's); mean |dp| <= 0.005 (measured 0.0024 and 0.0028; the reference's 1e-4 is for its real checkpoint,
    where nearly every tag sits at p ~ 0); the reference's decision-stability rule (tests/test_cuda_engine.py:55-57)
    with no violation; the same top-1 tag; and identical top-k for every k <= 50 where the reference's logit gap
    between ranks k and k + 1 exceeds twice the image's largest logit error (checked for at least one k). The head's bias is spread like a trained tagger's output:
    N(-6, 2^2) for most tags (confidently absent, with a tail near 0.5 for the decision rule) and 12 confident tags
    2.5 logits apart, so that ties do not decide the top-k."""
    from foidfinder_amd.engine import Eva02Config, Eva02Int8, convert_checkpoint, synthetic_checkpoint

    cfg = Eva02Config()
    raw = synthetic_checkpoint(cfg, seed=3)
    g = torch.Generator().manual_seed(11)
    bias = -6.0 + 2.0 * torch.randn(cfg.tags, generator=g)  # most tags confidently absent, a tail near 0.5
    present = torch.randperm(cfg.tags, generator=g)[:12]
    bias[present] = 4.0 + 2.5 * torch.arange(12, dtype=torch.float32)  # a few confident tags, 2.5 logits apart
    raw["head.bias"] = bias
    state = convert_checkpoint(raw, cfg)
    eng = Eva02Int8(state, cfg, device=dev)
    images = OM.synthetic_images(E2E_IMAGES, cfg.img_size, seed=8)
    print(f"full-depth end to end: engine forward (graph, batch {E2E_IMAGES})", flush=True)
    served = eng(torch.from_numpy(images).to(dev)).cpu().numpy().astype(np.float64)
    trace = {}
    eager = eng.eager(torch.from_numpy(images).to(dev), trace).cpu().numpy().astype(np.float64)
    assert np.array_equal(served, eager), "graph replay differs from the eager forward"
    x_eng = trace[f"x{cfg.depth - 1}"].cpu().numpy()

    np_state = {k: v.numpy() for k, v in state.items()}
    ocfg = oracle_cfg(cfg)
    fw = OM.float_weights_from_state(np_state, ocfg)
    qblocks = OM.blocks_from_state(np_state, cfg.depth)
    fweights = float_weights(raw, ocfg)
    from concurrent.futures import ThreadPoolExecutor

    def job(arg):
        kind, i = arg
        one = images[i : i + 1]
        out = OM.forward_int8_x(one, fw, qblocks) if kind == "int8" else OM.forward_float_x(one, fweights)
        print(f"full-depth end to end: oracle {kind} forward of image {i} done", flush=True)
        return out

    print("full-depth end to end: oracle int8 and float64 forwards", flush=True)
    n = E2E_IMAGES
    with ThreadPoolExecutor(4) as ex:
        xs = list(ex.map(job, [("int8", i) for i in range(n)] + [("float", i) for i in range(n)]))
    x_int8, x_float = np.concatenate(xs[:n]), np.concatenate(xs[n:])
    ref_int8, ref_float = OM.head_logits(x_int8, fw), OM.head_logits(x_float, fweights)

    rms = lambda d, r: float(np.sqrt((d.astype(np.float64) ** 2).mean() / (r.astype(np.float64) ** 2).mean()))
    drift = rms(x_eng.astype(np.float64) - x_int8, x_int8)
    noise = rms(x_int8.astype(np.float64) - x_float, x_float)
    sig = lambda z: 1.0 / (1.0 + np.exp(-z))
    p = sig(served)
    report = [f"residual stream after block 24: engine vs int8 oracle rms rel {drift:.4f}, "
              f"int8 oracle vs float {noise:.4f}; int8 noise (int8 oracle vs float): max|dp| "
              f"{np.abs(sig(ref_int8) - sig(ref_float)).max():.4f} max|dlogit| {np.abs(ref_int8 - ref_float).max():.4f}"]
    for name, ref in (("int8 oracle", ref_int8), ("float", ref_float)):
        dp, dl = np.abs(p - sig(ref)), np.abs(served - ref)
        checked, bad = gap_filtered_topk(served, ref)
        report.append(f"vs {name}: max|dp| {dp.max():.4f} mean {dp.mean():.5f}; max|dlogit| {dl.max():.4f} "
                      f"mean {dl.mean():.4f}; per image max|dp| {np.round(dp.max(1), 4).tolist()} max|dlogit| "
                      f"{np.round(dl.max(1), 3).tolist()}; decision flips {decision_flips(p, sig(ref))}; top-1 "
                      f"{[int(np.argmax(served[i]) == np.argmax(ref[i])) for i in range(n)]}; gap-filtered top-k "
                      f"checked {checked}, mismatched {bad}")
    print("\n".join(report), flush=True)
    assert drift <= E2E_RMS_REL_X, report[0]
    noise_dp = np.abs(sig(ref_int8) - sig(ref_float)).max()
    noise_dl = np.abs(ref_int8 - ref_float).max()
    for name, ref in (("int8 oracle", ref_int8), ("float", ref_float)):
        rel = E2E_REL_MAX[name]
        dp, dl = np.abs(p - sig(ref)), np.abs(served - ref)
        assert dp.max() <= rel * noise_dp and dp.mean() <= E2E_MEAN_DP, report
        assert dl.max() <= rel * noise_dl, report
        assert decision_flips(p, sig(ref)) == 0, report
        assert all(np.argmax(served[i]) == np.argmax(ref[i]) for i in range(n)), report
        checked, bad = gap_filtered_topk(served, ref)
        assert checked > 0 and not bad, report
