"""CPU oracle for foidfinder's int8 ViT hot path.

TEST INFRASTRUCTURE ONLY. This package restates, in numpy, the arithmetic of the reference's int8 path
(foidfinder/backends/cuda/csrc/kernels.cu, gemm.cuh, attention.cuh and foidfinder/backends/cuda/engine.py) so the
HIP kernels can be checked against it on identical inputs. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the checker or the timed CPU baseline. The product
path (`foidfinder_amd`) never imports it and has no CPU fallback.

Modules:
  rotq8      Walsh-Hadamard rotation + per-token int8 quantization (1024-point and block-128, optional LayerNorm)
  gemm       exact int8 x int8 -> int32 GEMM and the fp16 epilogues (QKV+RoPE, residual, GELU, SwiGLU, bias)
  attention  non-causal softmax attention over packed qkv rows, float64
  model      Hadamard matrix, weight quantization/conversion, EVA02 RoPE tables, synthetic EVA02-L/14-448 weights,
             and the int8-semantics forward of the whole tagger
  pixai      PixAI Tagger v1.0 (the reference's served model): window layout, axial RoPE, stem, attention-pool head,
             the int8-semantics and float forwards
  haruka     Haruka Tagger (EVA02-B + slot-sigmoid tree pool): weight conversion, stem, tree-pool head, the
             int8-semantics and float forwards

Pinning (what checks each function beyond restating it) is listed per function in `PINNED`; tests/test_oracle.py
runs those checks.
"""

PINNED = {
    "model.hadamard": "closed form (-1)^popcount(i&j)/sqrt(n), H H = I, H e0 = 1/sqrt(n)",
    "model.quantize_rows_int8": "brute-force per-element search of the nearest code on small matrices; ties",
    "model.rotate_rows64": "equals W @ blockdiag(H) formed as a float64 product, to float64 rounding (blocks 1024 and "
    "128); a planted wrong-sign butterfly fails it",
    "model.eva02_rope_tables": "cls row identity; every entry within 4e-6 of cos/sin of float64 angles (a planted "
    "row/column swap fails); one entry recomputed step by step in the reference's float32 recipe",
    "rotq8.fwht_rows": "equals x @ H (float64) to fp32 rounding; stage order only changes rounding (Parseval)",
    "rotq8.rot_q8_1024": "dequantized codes reconstruct x @ H within half a code; zero row, one-hot row, "
    "RNE ties; LayerNorm variant vs float64 LayerNorm",
    "rotq8.rot_q8_h128": "block-diagonal H128 closed form; padded columns stay zero; LN over real columns only",
    "gemm.gemm_s8_i32": "exact: int64 brute force on small shapes, float64 BLAS bound |acc| < 2^53",
    "gemm.fma32": "equals exact rational arithmetic rounded once (random operands); a constructed halfway case "
    "where a tiny addend decides the rounding (a float64-then-float32 computation gets it wrong)",
    "gemm.dequant": "each element equals the rational (acc*rs) * cs + bias rounded once",
    "gemm.exp_cw": "relative error below 3e-7 against float64 exp over [-80, 80]",
    "gemm.epilogue": "closed forms: RoPE at cls row is the identity, pair rotation preserves norm, SwiGLU of "
    "zero-padded columns is zero, residual adds in fp16",
    "attention.attention": "identical keys -> mean of V; one dominant logit -> that V row; shift invariance",
    "model.forward_int8": "agrees with the float forward (no quantization) within the int8 error budget",
    "pixai.window_perm": "bijection onto the grid; position 0 of window (wr, wc) is grid cell (wr*win, wc*win); "
    "consecutive positions step one column inside a window row",
    "pixai.axial_rope64": "row 0 is the identity; explicit angles (column 1 -> 1 rad for pair 0, row 1 for pair 16)",
    "pixai.patchify": "an image whose patch values encode their grid cell comes out in window_perm order",
    "pixai.stem": "patch GEMM equals a direct 14x14 stride-14 convolution loop on one patch",
    "pixai.pool_head": "one-token pooling is the single value row projected; uniform keys -> mean of values",
    "pixai.forward_int8": "agrees with the float forward (no quantization) within the int8 error budget",
    "haruka.convert_checkpoint": "dequantized fc1 rows times H128 give back the gate and value rows, interleaved",
    "haruka.stem": "token 0 is cls; a patch token equals a direct 14x14 convolution sum plus its bias",
    "haruka.pool_head": "equals the model card's MHAttnPool (unfolded key scale, child queries broadcast per coarse "
    "query, einsum leaves) in float64 torch",
    "haruka.forward_int8": "agrees with the float forward (no quantization) within the int8 error budget",
}
