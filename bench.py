"""Throughput of the int8 EVA02-L/14-448 tagger forward on one MI355X, batch 32, HIP-graph replay.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--batch 32] [--no-cpu-baseline]
                    [--model eva02|pixai|haruka]

A step is one forward over a batch of synthetic images (uniform [-1, 1], NHWC fp16, already in HBM) through the
captured graph: patch-embed GEMM, 24 int8 blocks (3x rotate+quant 1024, rotate+quant h128 + LayerNorm, 4 int8 GEMMs
with fused epilogues, flash attention), final LayerNorm, 1024 -> 30877 tag GEMM. Weights are random-init (seeded).

Prints one JSON line: images/s (whole job), per-kernel times measured live with HIP events on the launch stream,
the roofline of the dominant kernel, and the CPU baseline on the host's cores (PyTorch fp32 float forward at batch 2,
the single W8A8 linear, and the numpy oracle's int8 forward of one image).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s
PEAK_FP16_TFLOPS = 2500.0  # dense fp16 MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "images/sec @448px int8 ViT-L batch 32; int8 GEMM TOPS and % of MFMA peak"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-images", type=int, default=1, help="images in the CPU baseline sample")
    p.add_argument("--model", choices=("eva02", "pixai", "haruka"), default="eva02",
                   help="eva02: the headline EVA02-L/14-448 batch-32 line (default); pixai: PixAI Tagger v1.0 at "
                        "1008 px, the reference's served model (latency at --batch, default 1); haruka: Haruka "
                        "Tagger, EVA02-B/14-448 + tree pool + 98782-tag head (--batch default 64)")
    args = p.parse_args()
    if "--batch" not in sys.argv:
        args.batch = {"pixai": 1, "haruka": 64}.get(args.model, args.batch)
    return args


def timed(fn, stream, iters=20, warm=3) -> float:
    """Average duration (us) of fn's launches, HIP events recorded on the stream the kernels run on."""
    import torch

    for _ in range(warm):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record(stream)
    for _ in range(iters):
        fn()
    e.record(stream)
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters * 1e3


def in_forward_order(seq, stream, reps: int = 2) -> dict:
    """Average duration (us) per kernel name of `seq`, the (name, launch) pairs of one forward's blocks in forward
    order, each timed between HIP events recorded on the stream the kernels run on, one event after every launch
    (an event adds ~2 us to the launch it follows). Timed in sequence, not each kernel on its own: repeated launches
    of one kernel find its operands in the caches, and a rotation then runs up to ~15 % faster than inside the
    forward. The first pass over `seq` is a warm-up."""
    import torch

    for _, fn in seq:
        fn()
    acc: dict[str, list[float]] = {}
    for _ in range(reps):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(len(seq) + 1)]
        torch.cuda.synchronize()
        evs[0].record(stream)
        for i, (_, fn) in enumerate(seq):
            fn()
            evs[i + 1].record(stream)
        torch.cuda.synchronize()
        for i, (name, _) in enumerate(seq):
            acc.setdefault(name, []).append(evs[i].elapsed_time(evs[i + 1]) * 1e3)
    return {name: sum(v) / len(v) for name, v in acc.items()}


def kernel_row(us: float, bound: str, work: int, per_fwd: int) -> dict:
    if bound == "hbm":
        ach, peak, unit = work / us / 1e3, PEAK_HBM_GBS, "GB/s"
    elif bound == "mfma_int8":
        ach, peak, unit = work / us / 1e6, PEAK_INT8_TOPS, "TOP/s"
    else:
        ach, peak, unit = work / us / 1e6, PEAK_FP16_TFLOPS, "TFLOP/s"
    return {"us": round(us, 2), "launches_per_step": per_fwd, "work_per_launch": work, "achieved": round(ach, 1),
            "unit": unit, "peak": peak, "frac": round(ach / peak, 4), "bound": "hbm" if bound == "hbm" else "mfma"}


def kernel_table(eng, B: int, buf) -> dict:
    """The block kernels of a whole forward (every layer's weights) run in forward order on the graph's buffers,
    each launch timed (in_forward_order); algorithmic work per launch and roofline per kernel."""
    import torch

    from foidfinder_amd.kernels import EPI_QKV_ROPE, EPI_RESIDUAL, EPI_SWIGLU

    cfg, k = eng.cfg, eng.k
    M, d, h, hp, L, eps = B * cfg.tokens, cfg.dim, cfg.hidden, cfg.hidden_pad, cfg.tokens, cfg.eps
    v = {n: eng.variants.get((n, B), 0) for n in ("qkv", "proj", "fc1", "fc2")}
    x, a8, rs = buf["x"], buf["a8"], buf["rs"]
    meta = {
        "rot_q8_1024_ln": ("hbm", M * d * 2 + M * d + 4 * M + 8 * d, 2 * cfg.depth),
        "rot_q8_1024": ("hbm", M * d * 3 + 4 * M, cfg.depth),
        "rot_q8_h128_ln": ("hbm", M * hp * 3 + 4 * M + 8 * h, cfg.depth),
        "gemm_qkv": ("mfma_int8", 2 * M * 3 * d * d, cfg.depth),
        "gemm_proj": ("mfma_int8", 2 * M * d * d, cfg.depth),
        "gemm_fc1": ("mfma_int8", 2 * M * 2 * h * d, cfg.depth),
        "gemm_fc2": ("mfma_int8", 2 * M * d * h, cfg.depth),
        "attention": ("mfma_fp16", 4 * B * cfg.heads * L * L * 64, cfg.depth),
    }

    def block(lw):  # Eva02Int8._forward's block, kernel by kernel
        return [("rot_q8_1024_ln", lambda: k.rot_q8_1024(x, *lw["n1"], a8, rs, eps)),
                ("gemm_qkv", lambda: eng._gemm(a8, lw["qkv"], rs, EPI_QKV_ROPE, v["qkv"], buf["qkv"], eng.rope)),
                ("attention", lambda: k.attention(buf["qkv"], buf["o16"], L)),
                ("rot_q8_1024", lambda: k.rot_q8_1024(buf["o16"], None, None, a8, rs, eps)),
                ("gemm_proj", lambda: eng._gemm(a8, lw["proj"], rs, EPI_RESIDUAL, v["proj"], x)),
                ("rot_q8_1024_ln", lambda: k.rot_q8_1024(x, *lw["n2"], a8, rs, eps)),
                ("gemm_fc1", lambda: eng._gemm(a8, lw["fc1"], rs, EPI_SWIGLU, v["fc1"], buf["h16"])),
                ("rot_q8_h128_ln", lambda: k.rot_q8_h128(buf["h16"], buf["h8"], rs, *lw["nm"], h, eps)),
                ("gemm_fc2", lambda: eng._gemm(buf["h8"], lw["fc2"], rs, EPI_RESIDUAL, v["fc2"], x))]

    us = in_forward_order([job for lw in eng.layers for job in block(lw)], torch.cuda.current_stream())
    return {name: kernel_row(us[name], *meta[name]) for name in meta}


def cpu_threads() -> int:
    """Host threads for the CPU baseline: every core this process may use, capped by OMP_NUM_THREADS when set (a
    shared host gives each GPU job a share of its cores and says so there)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() else n


def cpu_info() -> dict:
    """lscpu's model name and sockets x cores per socket (x threads per core)."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return {"model": info.get("Model name"),
            "sockets_x_cores": f"{info.get('Socket(s)')} x {info.get('Core(s) per socket')} "
                               f"(x {info.get('Thread(s) per core')} threads)"}


def median_time(fn, runs: int = 3) -> float:
    """1 untimed warm-up, then the median wall time of `runs` calls (s)."""
    fn()
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(raw, state, cfg, n_images: int) -> dict:
    """The CPU baseline on this host's cores, three legs:

    - value: the EVA02-L/14-448 float forward in PyTorch fp32 on the CPU, in the op order of the reference's PyTorch
      model (foidfinder/backends/cuda/reference.py:109-131, adapted to EVA02), batch 2, 1 warm-up + median of 3;
    - w8a8_linear: the plumbing config's single W8A8 linear (1025 x 1024 -> 3072: rotation, per-token int8, exact
      int8 product, dequant + bias) in PyTorch on the CPU, 1 warm-up + median of 3;
    - int8_oracle: the numpy oracle's int8-semantics forward of `n_images` image(s), one run (it restates the GPU
      kernels' arithmetic, float64 BLAS for the exact int32 GEMMs).
    The reference's own int8 path is CUDA and has no CPU counterpart."""
    import numpy as np
    import torch

    from foidfinder_amd.engine import eva02_rope_tables
    from oracle import float_torch as FT
    from oracle import model as OM

    threads = cpu_threads()
    torch.set_num_threads(threads)
    cpu_raw = {k: v.detach().float().cpu() for k, v in raw.items()}
    rope = eva02_rope_tables(cfg.grid, cfg.rope_ref)
    fb = 2
    imgs = torch.from_numpy(OM.synthetic_images(fb, cfg.img_size, seed=11)).float()
    t_float = median_time(lambda: FT.forward_float(imgs, cpu_raw, cfg.depth, cfg.heads, cfg.patch, cfg.hidden, rope,
                                                   cfg.eps))
    x, qw, ws, b = OM.w8a8_linear_inputs()
    xt, qwt, wst, bt = (torch.from_numpy(a) for a in (x, qw, ws, b))
    t_lin = median_time(lambda: FT.w8a8_linear(xt, qwt, wst, bt))
    lin_ops = 2 * x.shape[0] * qw.shape[0] * qw.shape[1]
    np_state = {k: v.detach().cpu().numpy() for k, v in state.items()}
    ocfg = OM.Eva02Config(img_size=cfg.img_size, depth=cfg.depth, tags=cfg.tags)
    images = OM.synthetic_images(n_images, cfg.img_size, seed=11)
    t = time.perf_counter()
    OM.forward_int8_state(images, np_state, ocfg)
    t_int8 = time.perf_counter() - t
    return {"value": round(fb / t_float, 4), "unit": "images/s", "cores": threads, "kind": "port",
            "sample": f"EVA02-L/14-448 float forward, PyTorch fp32 on the CPU, batch {fb}, 1 warm-up + median of 3 "
                      f"({t_float:.2f} s per batch)",
            "torch_threads": torch.get_num_threads(), "cpu": cpu_info(),
            "w8a8_linear": {"value": round(lin_ops / t_lin / 1e9, 2), "unit": "GOP/s", "ms": round(1e3 * t_lin, 2),
                            "sample": "1025 x 1024 fp16 -> 3072, rotation + per-token int8 + exact int8 product + "
                                      "dequant + bias, PyTorch CPU, 1 warm-up + median of 3"},
            "int8_oracle": {"value": round(n_images / t_int8, 4), "unit": "images/s",
                            "sample": f"{n_images} image(s) through the numpy int8-semantics forward, one run, "
                                      f"{t_int8:.1f} s"}}


def bench_pixai(args) -> None:
    """PixAI Tagger v1.0 at 1008 px (32 blocks, 5184 tokens, windowed + 4 global attention blocks), random-init
    weights: graph-replay time per batch, and the backend's end-to-end predict (GPU letterbox preprocessing of a
    1200 x 900 image, forward, sigmoid, copy to the host) at batch 1. The reference publishes 19.8 ms per image for
    its int8 engine with preprocessing at batch 1 on an RTX 4090 (README.md:173): context, other hardware."""
    import numpy as np
    import torch
    from PIL import Image

    from foidfinder_amd.backends.rocm.preprocess import preprocess
    from foidfinder_amd.pixai import PixAIConfig, PixAIInt8, convert_checkpoint, synthetic_checkpoint

    dev = torch.device("cuda:0")
    cfg = PixAIConfig()
    B = args.batch
    raw = synthetic_checkpoint(cfg, seed=args.seed)
    state = convert_checkpoint({k: v.to(dev) for k, v in raw.items()}, cfg)
    del raw
    eng = PixAIInt8(state, cfg, device=dev)
    g = torch.Generator(device="cpu").manual_seed(args.seed + 1)
    images = (torch.rand(B, cfg.img_size, cfg.img_size, 3, generator=g) * 2 - 1).half().to(dev)
    assert torch.isfinite(eng(images)).all()
    for _ in range(args.warmup):
        eng.replay(B)
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        eng.replay(B)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    ms = elapsed / args.steps * 1e3
    # end to end through the backend's path at batch 1: preprocess + forward + sigmoid + host copy
    img = Image.fromarray(np.random.default_rng(args.seed).integers(0, 256, (900, 1200, 3), dtype=np.uint8))
    e2e = []
    for i in range(args.warmup + args.steps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        torch.sigmoid(eng(preprocess([img], cfg.img_size))).cpu().numpy()
        if i >= args.warmup:
            e2e.append(time.perf_counter() - t)
    gemm_ops = sum(cfg.gemm_ops(B).values())
    line = {
        "metric": "images/sec @1008px int8 PixAI Tagger v1.0 (graph replay)",
        "value": round(B * args.steps / elapsed, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "ms_per_image_e2e_batch1": round(1e3 * float(np.median(e2e)), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "reference_published": {"ms_per_image": 19.8, "hardware": "RTX 4090", "includes": "preprocessing, batch 1"},
        "dtype": "int8",
        "data": "synthetic: random-init weights (seeded), images uniform [-1, 1]; e2e: one 1200x900 RGB image",
        "config": {"workload": "PixAI Tagger v1.0 int8 W8A8 forward, 1008 px, hipGraph replay", "batch": B,
                   "tokens": cfg.tokens, "window_tokens": cfg.win_tokens, "depth": cfg.depth,
                   "global_blocks": list(cfg.global_blocks), "hidden": cfg.hidden, "parallelism": "single GPU"},
        "gemm_variants": {name: eng.variants.get((name, B), 0) for name in ("qkv", "proj", "fc1", "fc2")},
        "work_per_step": {"gemm_int8_ops": gemm_ops, "attention_flops": cfg.attention_flops(B)},
    }
    print(json.dumps(line), flush=True)


def bench_haruka(args) -> None:
    """Haruka Tagger (EVA02-B/14 at 448 px, 12 int8 blocks of d 768, tree pool, 1152 -> 98782 head), random-init
    weights in the reference's folded format, converted to int8 on load: graph-replay time per batch (raw uint8
    pixels already in HBM), each block kernel and the pool head timed alone on the graph's buffers, and the
    backend's end-to-end predict of one 1200 x 900 image (model-card letterbox on the host, forward, sigmoid, copy
    back) at batch 1. The reference serves Haruka on Apple GPUs only and publishes no number for it."""
    import numpy as np
    import torch
    from PIL import Image

    from foidfinder_amd.backends.rocm.preprocess import preprocess_haruka
    from foidfinder_amd.haruka import HarukaConfig, HarukaInt8, convert_checkpoint, synthetic_checkpoint
    from foidfinder_amd.kernels import EPI_QKV_ROPE, EPI_RESIDUAL, EPI_SWIGLU

    dev = torch.device("cuda:0")
    cfg = HarukaConfig()
    B = args.batch
    t0 = time.perf_counter()
    raw = synthetic_checkpoint(cfg, seed=args.seed)
    state = convert_checkpoint({k: v.to(dev) for k, v in raw.items()}, cfg)
    del raw
    eng = HarukaInt8(state, cfg, device=dev)
    g = torch.Generator(device="cpu").manual_seed(args.seed + 1)
    images = torch.randint(0, 256, (B, cfg.img_size, cfg.img_size, 3), generator=g, dtype=torch.uint8).to(dev)
    assert torch.isfinite(eng(images)).all()
    torch.cuda.synchronize()
    print(f"setup {time.perf_counter() - t0:.1f}s; variants { {k[0]: v for k, v in eng.variants.items()} }",
          file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        eng.replay(B)
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        eng.replay(B)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    ms = elapsed / args.steps * 1e3
    ips = B * args.steps / elapsed
    print(f"{ips:.1f} images/s, {ms:.2f} ms per batch of {B}", file=sys.stderr, flush=True)

    buf = eng._graphs[B][3]
    k, st = eng.k, torch.cuda.current_stream()
    M, d, h, L, eps = B * cfg.tokens, cfg.dim, cfg.hidden, cfg.tokens, cfg.eps
    v = {n: eng.variants.get((n, B), 0) for n in ("qkv", "proj", "fc1", "fc2")}
    x, a8, rs = buf["x"], buf["a8"], buf["rs"]
    meta = {
        "rot_q8_h128_ln_768": ("hbm", M * d * 3 + 4 * M + 8 * d, 2 * cfg.depth),
        "rot_q8_h128_768": ("hbm", M * d * 3 + 4 * M, cfg.depth),
        "rot_q8_h128_ln_2048": ("hbm", M * h * 3 + 4 * M + 8 * h, cfg.depth),
        "gemm_qkv": ("mfma_int8", 2 * M * 3 * d * d, cfg.depth),
        "gemm_proj": ("mfma_int8", 2 * M * d * d, cfg.depth),
        "gemm_fc1": ("mfma_int8", 2 * M * 2 * h * d, cfg.depth),
        "gemm_fc2": ("mfma_int8", 2 * M * d * h, cfg.depth),
        "attention": ("mfma_fp16", 4 * B * cfg.heads * L * L * 64, cfg.depth),
    }

    def block(lw):  # HarukaInt8._forward's block, kernel by kernel
        return [("rot_q8_h128_ln_768", lambda: k.rot_q8_h128(x, a8, rs, *lw["n1"], d, eps)),
                ("gemm_qkv", lambda: eng._gemm(a8, lw["qkv"], rs, EPI_QKV_ROPE, v["qkv"], buf["qkv"], eng.rope)),
                ("attention", lambda: k.attention(buf["qkv"], buf["o16"], L)),
                ("rot_q8_h128_768", lambda: k.rot_q8_h128(buf["o16"], a8, rs)),
                ("gemm_proj", lambda: eng._gemm(a8, lw["proj"], rs, EPI_RESIDUAL, v["proj"], x)),
                ("rot_q8_h128_ln_768", lambda: k.rot_q8_h128(x, a8, rs, *lw["n2"], d, eps)),
                ("gemm_fc1", lambda: eng._gemm(a8, lw["fc1"], rs, EPI_SWIGLU, v["fc1"], buf["h16"])),
                ("rot_q8_h128_ln_2048", lambda: k.rot_q8_h128(buf["h16"], buf["h8"], rs, *lw["nm"], h, eps)),
                ("gemm_fc2", lambda: eng._gemm(buf["h8"], lw["fc2"], rs, EPI_RESIDUAL, v["fc2"], x))]

    us = in_forward_order([job for lw in eng.layers for job in block(lw)], st)
    kern = {name: kernel_row(us[name], *m) for name, m in meta.items()}
    # the pool head (the head GEMM's fp16 weights dominate its bytes), eager: its ~40 launches time on their own
    kern["pool_head"] = kernel_row(timed(lambda: eng.pool_head(x.view(B, L, d)), st), "hbm",
                                   cfg.tags * cfg.leaves * cfg.leaf_dim * 2, 1)
    for n, r in kern.items():
        print(f"  {n:20s} {r['us']:8.1f} us x{r['launches_per_step']:3d}  {r['achieved']:8.1f} {r['unit']}"
              f"  ({100 * r['frac']:.1f}% of peak)", file=sys.stderr, flush=True)
    per_step = {n: r["us"] * r["launches_per_step"] for n, r in kern.items()}
    dom = max(per_step, key=per_step.get)
    gemm = [n for n in kern if n.startswith("gemm_")]
    gemm_tops = sum(kern[n]["work_per_launch"] * kern[n]["launches_per_step"] for n in gemm) / sum(
        per_step[n] for n in gemm) / 1e6
    img = Image.fromarray(np.random.default_rng(args.seed).integers(0, 256, (900, 1200, 3), dtype=np.uint8))
    e2e = []
    for i in range(args.warmup + args.steps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        torch.sigmoid(eng(preprocess_haruka([img], cfg.img_size))).cpu().numpy()
        if i >= args.warmup:
            e2e.append(time.perf_counter() - t)
    line = {
        "metric": "images/sec @448px int8 Haruka Tagger (EVA02-B/14 + tree pool, 98782 tags)",
        "value": round(ips, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "ms_per_image_e2e_batch1": round(1e3 * float(np.median(e2e)), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: random-init weights (seeded, folded format), raw pixels uniform 0..255 (uint8); "
                "e2e: one 1200x900 RGB image",
        "config": {"workload": "Haruka Tagger int8 W8A8 forward, 448 px, hipGraph replay", "batch": B,
                   "seq_len": cfg.tokens, "dim": cfg.dim, "depth": cfg.depth, "heads": cfg.heads,
                   "mlp_hidden": cfg.hidden, "pool": f"{cfg.coarse} coarse + {cfg.leaves} leaf queries, "
                   f"{cfg.pool_heads} heads", "tags": cfg.tags, "parallelism": "single GPU"},
        "gemm_tops": round(gemm_tops, 1),
        "gemm_frac_of_int8_peak": round(gemm_tops / PEAK_INT8_TOPS, 4),
        "roofline": {"kernel": dom, **{f: kern[dom][f] for f in ("bound", "achieved", "peak", "frac")},
                     "unit": "GB/s" if kern[dom]["unit"] == "GB/s" else "TFLOP/s"},
        "kernels": kern,
        "kernel_timing": "block kernels of one forward in forward order, 2 passes, a HIP event after each launch "
                         "(~2 us per event included); pool_head eager, 20 calls",
        "gemm_variants": v,
        "work_per_step": {"gemm_int8_ops": sum(cfg.gemm_ops(B).values()), "attention_flops": cfg.attention_flops(B)},
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the tagger forward is data-parallel "
              "over images and every figure here is one GPU's", file=sys.stderr)
        sys.exit(2)
    if args.model == "pixai":
        bench_pixai(args)
        return
    if args.model == "haruka":
        bench_haruka(args)
        return
    import torch

    from foidfinder_amd.engine import Eva02Config, Eva02Int8, convert_checkpoint, synthetic_checkpoint

    torch.manual_seed(args.seed)
    dev = torch.device("cuda:0")
    cfg = Eva02Config()
    B = args.batch
    t0 = time.perf_counter()
    raw = synthetic_checkpoint(cfg, seed=args.seed)
    state = convert_checkpoint({k: v.to(dev) for k, v in raw.items()}, cfg)
    eng = Eva02Int8(state, cfg, device=dev)
    g = torch.Generator(device="cpu").manual_seed(args.seed + 1)
    images = (torch.rand(B, cfg.img_size, cfg.img_size, 3, generator=g) * 2 - 1).half().to(dev)
    logits = eng(images)  # autotune + capture
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    print(f"setup {setup_s:.1f}s (weights, conversion, autotune, graph capture); variants "
          f"{ {k[0]: v for k, v in eng.variants.items()} }", file=sys.stderr, flush=True)
    assert torch.isfinite(logits).all()

    for _ in range(args.warmup):
        eng.replay(B)
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        eng.replay(B)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    ms = elapsed / args.steps * 1e3
    ips = B * args.steps / elapsed
    print(f"{ips:.1f} images/s, {ms:.2f} ms per batch of {B}", file=sys.stderr, flush=True)

    buf = eng._graphs[B][3]
    kern = kernel_table(eng, B, buf)
    per_step = {n: r["us"] * r["launches_per_step"] for n, r in kern.items()}
    dom = max(per_step, key=per_step.get)
    dk = kern[dom]
    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get(dom)
    gemm_names = [n for n in kern if n.startswith("gemm_")]
    gemm_ops = sum(kern[n]["work_per_launch"] * kern[n]["launches_per_step"] for n in gemm_names)
    gemm_us = sum(per_step[n] for n in gemm_names)
    gemm_tops = gemm_ops / gemm_us / 1e6
    for n, r in kern.items():
        print(f"  {n:16s} {r['us']:8.1f} us x{r['launches_per_step']:3d}  {r['achieved']:8.1f} {r['unit']}"
              f"  ({100 * r['frac']:.1f}% of peak)", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(raw, state, cfg, args.cpu_images)
    line = {
        "metric": METRIC,
        "value": round(ips, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: random-init weights (seeded), images uniform [-1, 1]",
        "config": {"workload": "EVA02-L/14-448 int8 W8A8 tagger forward, batch 32, hipGraph replay",
                   "batch": B, "seq_len": cfg.tokens, "dim": cfg.dim, "depth": cfg.depth, "heads": cfg.heads,
                   "mlp_hidden": cfg.hidden, "tags": cfg.tags, "parallelism": "single GPU"},
        "gemm_tops": round(gemm_tops, 1),
        "gemm_frac_of_int8_peak": round(gemm_tops / PEAK_INT8_TOPS, 4),
        "roofline": {"kernel": dom, "bound": dk["bound"], "achieved": dk["achieved"], "peak": dk["peak"],
                     # the roofline object's unit is "GB/s" or "TFLOP/s"; int8 rates are tera-ops (2 per multiply-add)
                     "unit": "GB/s" if dk["unit"] == "GB/s" else "TFLOP/s", "frac": dk["frac"], "traffic": traffic},
        "kernels": kern,
        "kernel_timing": "one forward's block kernels in forward order, 2 passes, a HIP event after each launch "
                         "(~2 us per event included)",
        "gemm_variants": {name: eng.variants.get((name, B), 0) for name in ("qkv", "proj", "fc1", "fc2")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
