"""Times the hot path's kernels beside the platform libraries that could stand in for them, at the batch-32
EVA02-L/14-448 shapes (M = 32 800 tokens):

  * each block GEMM: ff_gemm_s8 with its fused epilogue; ff_gemm_s8 with the plain int32 output (no epilogue);
    torch._int_mm (hipBLASLt int8 -> int32); and torch.matmul in fp16 (hipBLASLt), the same GEMM in the precision
    the quantization replaces;
  * attention over 1025 tokens, 32 x 16 heads of 64: ff_attention and torch's scaled_dot_product_attention (fp16,
    whichever fused backend torch picks on this platform).

    python -m foidfinder_amd.measure.compare_libs [--batch 32] [--iters 20]

Times are per launch, from torch.cuda events around `iters` back-to-back launches on the current stream (every
function here launches on it). Operands are random; nothing is checked (the tests do that).
"""

from __future__ import annotations

import argparse

import torch
import torch.nn.functional as F

from ..engine import Eva02Config, eva02_rope_tables
from ..kernels import EPI_I32, EPI_QKV_ROPE, EPI_RESIDUAL, EPI_SWIGLU, kernels

INT8_PEAK, FP16_PEAK = 5.0e15, 2.5e15  # MI355X dense MFMA, ops/s


def time_us(fn, iters: int) -> float:
    fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(iters):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / iters


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--variant", type=int, default=4, help="ff_gemm_s8 tile variant (the engine's autotune pick)")
    args = ap.parse_args()
    k = kernels()
    dev = torch.device("cuda:0")
    cfg = Eva02Config()
    M, d, hp = args.batch * cfg.tokens, cfg.dim, cfg.hidden_pad
    g = torch.Generator(device=dev).manual_seed(0)

    def i8(*s):
        return torch.randint(-127, 128, s, dtype=torch.int8, device=dev, generator=g)

    cos, sin = (t.to(dev) for t in eva02_rope_tables(cfg.grid, cfg.rope_ref))
    rows = []
    # (name, N, K, epilogue, ops with the unpadded dims)
    for name, N, K, epi, n_real, k_real in (("qkv", 3 * d, d, EPI_QKV_ROPE, 3 * d, d),
                                            ("proj", d, d, EPI_RESIDUAL, d, d),
                                            ("fc1", 2 * hp, d, EPI_SWIGLU, 2 * cfg.hidden, d),
                                            ("fc2", d, hp, EPI_RESIDUAL, d, cfg.hidden)):
        A, W = i8(M, K), i8(N, K)
        rs = torch.rand(M, device=dev, generator=g) * 1e-2
        cs = torch.rand(N, device=dev, generator=g) * 1e-3
        bias = torch.zeros(N, device=dev)
        out = torch.zeros(M, N // 2 if epi == EPI_SWIGLU else N, device=dev, dtype=torch.half)
        o32 = torch.empty(M, N, device=dev, dtype=torch.int32)
        fused = time_us(lambda: k.gemm_s8(A, W, rs, cs, bias, out, epi, args.variant,
                                          cos if epi == EPI_QKV_ROPE else None,
                                          sin if epi == EPI_QKV_ROPE else None, 0.18), args.iters)
        plain = time_us(lambda: k.gemm_s8(A, W, rs, cs, bias, o32, EPI_I32, args.variant, None, None, 1.0),
                        args.iters)
        Wt = W.t()  # [K, N] column-major view: the layout hipBLASLt's int8 "TN" GEMM takes without a copy
        try:
            blas = time_us(lambda: torch._int_mm(A, Wt), args.iters)
        except RuntimeError as e:  # an unsupported shape or layout on this build
            blas = float("nan")
            print(f"torch._int_mm {name}: {e}".splitlines()[0], flush=True)
        del o32
        Ah, Wh = A.half(), W.half()
        fp16 = time_us(lambda: torch.matmul(Ah, Wh.t()), args.iters)
        del Ah, Wh
        ops = 2.0 * M * n_real * k_real
        rows.append((f"gemm_{name} [{M} x {N} x {K}]", ops, (fused, plain, blas, fp16)))
        torch.cuda.empty_cache()

    B, H, L = args.batch, cfg.heads, cfg.tokens
    qkv = (torch.randn(B * L, 3 * d, device=dev, generator=g) * 0.3).half()
    o16 = torch.empty(B * L, d, device=dev, dtype=torch.half)
    ours = time_us(lambda: k.attention(qkv, o16, L), args.iters)
    q, kk, v = (t.view(B, L, H, 64).transpose(1, 2).contiguous() for t in qkv.split(d, dim=1))
    sdpa = time_us(lambda: F.scaled_dot_product_attention(q, kk, v), args.iters)
    att_flops = 4.0 * B * H * L * L * 64

    print(f"| kernel | ops per launch | ff, fused epilogue | ff, int32 out | torch._int_mm (int8) | torch fp16 matmul |")
    print("|---|---:|---:|---:|---:|---:|")
    for label, ops, ts in rows:
        cells = []
        for t, peak in zip(ts, (INT8_PEAK, INT8_PEAK, INT8_PEAK, FP16_PEAK)):
            cells.append("n/a" if t != t else f"{t:.1f} us ({ops / (t * 1e-6) / 1e12:.0f} T, {ops / (t * 1e-6) / peak:.1%})")
        print(f"| {label} | {ops / 1e9:.1f} G | " + " | ".join(cells) + " |")
    print()
    print("| kernel | flops per launch | ff_attention | torch scaled_dot_product_attention (fp16) |")
    print("|---|---:|---:|---:|")
    cells = [f"{t:.1f} us ({att_flops / (t * 1e-6) / 1e12:.0f} TFLOP/s, {att_flops / (t * 1e-6) / FP16_PEAK:.1%})"
             for t in (ours, sdpa)]
    print(f"| attention [{B} x {H} heads x {L} tokens x 64] | {att_flops / 1e9:.1f} G | " + " | ".join(cells) + " |")
    print(f"(per launch; batch {args.batch}, {args.iters} launches per timing, ff_gemm_s8 variant {args.variant})",
          flush=True)


if __name__ == "__main__":
    main()
