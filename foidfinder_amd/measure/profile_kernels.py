"""Launches each block kernel at the batch-32 EVA02-L/14-448 shapes, plus a plain copy of known size, for hardware
counter runs (one counter set per run; `--only` narrows the launches to some of them):

    rocprofv3 --pmc FETCH_SIZE -d <dir> -o fetch -- python -m foidfinder_amd.measure.profile_kernels
    rocprofv3 --pmc WRITE_SIZE -d <dir> -o write -- python -m foidfinder_amd.measure.profile_kernels

The copy (torch's elementwise copy of COPY_BYTES) calibrates the counters: HBM bytes of a kernel =
counter_kib * 1024 * COPY_BYTES / copy_counter_bytes. Inputs are random, outputs scratch; nothing is checked here.
"""

from __future__ import annotations

import argparse

import torch

from ..engine import Eva02Config, eva02_rope_tables
from ..kernels import EPI_QKV_ROPE, EPI_RESIDUAL, EPI_SWIGLU, kernels, pad_norm

COPY_BYTES = 1 << 30


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--variants", default="qkv=4,proj=4,fc1=4,fc2=4",
                    help="GEMM tile variant per GEMM, as the engine's autotune picked them (bench.py prints them)")
    ap.add_argument("--only", default="", help="comma-separated subset of: rot,gemm,attention,copy (default: all)")
    args = ap.parse_args()
    only = set(args.only.split(",")) if args.only else {"rot", "gemm", "attention", "copy"}
    var = {kv.split("=")[0]: int(kv.split("=")[1]) for kv in args.variants.split(",")}
    k = kernels()
    dev = torch.device("cuda:0")
    cfg = Eva02Config()
    M, d, h, hp = args.batch * cfg.tokens, cfg.dim, cfg.hidden, cfg.hidden_pad
    g = torch.Generator(device=dev).manual_seed(0)

    def i8(*s):
        return torch.randint(-127, 128, s, dtype=torch.int8, device=dev, generator=g)

    x = torch.randn(M, d, device=dev, generator=g).half()
    o16 = torch.randn(M, d, device=dev, generator=g).half()
    h16 = torch.randn(M, hp, device=dev, generator=g).half()
    h16[:, h:] = 0
    qkv = (torch.randn(M, 3 * d, device=dev, generator=g) * 0.3).half()
    a8, h8 = i8(M, d), i8(M, hp)
    rs = torch.rand(M, device=dev, generator=g) * 1e-2
    ones = lambda n: torch.ones(n, device=dev)  # noqa: E731
    zeros = lambda n: torch.zeros(n, device=dev)  # noqa: E731
    w = {"qkv": i8(3 * d, d), "proj": i8(d, d), "fc1": i8(2 * hp, d), "fc2": i8(d, hp)}
    cs = {n: torch.rand(t.size(0), device=dev, generator=g) * 1e-3 for n, t in w.items()}
    cos, sin = (t.to(dev) for t in eva02_rope_tables(cfg.grid, cfg.rope_ref))
    out_qkv = torch.empty(M, 3 * d, device=dev, dtype=torch.half)
    xr = x.clone()
    hout = torch.empty(M, hp, device=dev, dtype=torch.half)
    src = torch.empty(COPY_BYTES // 2, device=dev, dtype=torch.half)
    dst = torch.empty_like(src)
    for _ in range(args.reps):
        if "rot" in only:
            k.rot_q8_1024(x, ones(d), zeros(d), a8, rs, cfg.eps)
            k.rot_q8_1024(o16, None, None, a8, rs, cfg.eps)
            k.rot_q8_h128(h16, h8, rs, *pad_norm(ones(h), zeros(h), hp), h, cfg.eps)
        if "gemm" in only:
            k.gemm_s8(a8, w["qkv"], rs, cs["qkv"], zeros(3 * d), out_qkv, EPI_QKV_ROPE, var["qkv"], cos, sin, 0.18)
            k.gemm_s8(a8, w["proj"], rs, cs["proj"], zeros(d), xr, EPI_RESIDUAL, var["proj"], None, None, 1.0)
            k.gemm_s8(a8, w["fc1"], rs, cs["fc1"], zeros(2 * hp), hout, EPI_SWIGLU, var["fc1"], None, None, 1.0)
            k.gemm_s8(h8, w["fc2"], rs, cs["fc2"], zeros(d), xr, EPI_RESIDUAL, var["fc2"], None, None, 1.0)
        if "attention" in only:
            k.attention(qkv, o16, cfg.tokens)
        if "copy" in only:
            dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile_kernels: {sorted(only)} x {args.reps} at batch {args.batch} (M = {M}), GEMM variants {var}; copy of "
          f"{COPY_BYTES} bytes", flush=True)


if __name__ == "__main__":
    main()
