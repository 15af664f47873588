"""Walsh-Hadamard rotation + per-token symmetric int8 quantization, restated in numpy float32.

Every operation below is a single IEEE float32 operation (numpy keeps float32 for float32 operands), with no
fused multiply-add, so the results are reproducible bit for bit by a kernel that performs the same operations in
the same order.

Reference: foidfinder/backends/cuda/csrc/kernels.cu:13-160 and common.cuh:45-48, 58-67.
"""

from __future__ import annotations

import numpy as np

from .gemm import fma32

F32 = np.float32
INV_SQRT_128 = F32(0.08838834764831845)  # kernels.cu:138, rounded to fp32 once
EPS_SCALE = F32(1e-12)  # kernels.cu:97
STAGES_1024 = (0, 1, 2, 8, 9, 3, 4, 5, 6, 7)  # kernels.cu:15-44: column bits e (0-2), j (8-9), lane (3-7)


def butterfly(v: np.ndarray, bit: int) -> np.ndarray:
    """One FWHT stage over column bit `bit` of the last axis: (a, b) -> (a + b, a - b), a the lower index."""
    n = v.shape[-1]
    w = v.reshape(*v.shape[:-1], n >> (bit + 1), 2, 1 << bit)
    a, b = w[..., 0, :], w[..., 1, :]
    return np.stack([a + b, a - b], axis=-2).reshape(v.shape)


def fwht_rows(v: np.ndarray, order: tuple[int, ...]) -> np.ndarray:
    """Unnormalized Sylvester FWHT of each row, stages applied in the given bit order."""
    v = np.ascontiguousarray(v, dtype=F32)
    for bit in order:
        v = butterfly(v, bit)
    return v


def quant_rows(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row absmax int8 (kernels.cu:93-107, common.cuh:45-48).

    scale = max(amax, 1e-12) / 127 (IEEE division); inv = 1 / scale; code = clamp(rne(v * inv), -127, 127)."""
    amax = np.abs(v).max(axis=-1)
    scale = np.maximum(amax, EPS_SCALE) / F32(127.0)
    inv = F32(1.0) / scale
    q = np.clip(np.rint(v * inv[:, None]), -127, 127).astype(np.int8)
    return q, scale.astype(F32)


def _xor_tree(s: np.ndarray, masks: tuple[int, ...]) -> np.ndarray:
    """Butterfly all-reduce over the last (lane) axis; every lane ends with the same value."""
    lanes = np.arange(s.shape[-1])
    for m in masks:
        s = s + s[..., lanes ^ m]
    return s[..., 0]


def layer_norm_1024(v: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float) -> np.ndarray:
    """LayerNorm over 1024 columns with the reference's reduction order (kernels.cu:69-91).

    Lane L of the 32-lane group owns columns j*256 + L*8 + e and sums them sequentially in (j, e) order; the 32
    partial sums are then combined by the xor tree 16, 8, 4, 2, 1 (common.cuh:58-62). The variance repeats this on
    (v - mean)^2, accumulated as fma(d, d, sq). rstd = 1 / sqrt(var + eps) with IEEE sqrt and division (the
    reference's rsqrtf is an approximate instruction; this restatement fixes the correctly rounded form). Output
    fma((v - mean) * rstd, gamma, beta). The two fused multiply-adds are where the reference's compiler contracts
    `sq += d * d` and `d * rstd * g + b` (kernels.cu:80-91); every other operation rounds on its own."""
    T = v.shape[0]
    lanes = v.reshape(T, 4, 32, 8).transpose(0, 2, 1, 3).reshape(T, 32, 32)  # [row, lane, i = j*8 + e]
    s = np.zeros((T, 32), F32)
    for i in range(32):
        s = s + lanes[:, :, i]
    mean = _xor_tree(s, (16, 8, 4, 2, 1)) * F32(1.0 / 1024.0)
    d = v - mean[:, None]
    dl = d.reshape(T, 4, 32, 8).transpose(0, 2, 1, 3).reshape(T, 32, 32)
    sq = np.zeros((T, 32), F32)
    for i in range(32):
        sq = fma32(dl[:, :, i], dl[:, :, i], sq)
    var = _xor_tree(sq, (16, 8, 4, 2, 1)) * F32(1.0 / 1024.0)
    rstd = F32(1.0) / np.sqrt(var + F32(eps))
    return fma32(d * rstd[:, None], gamma.astype(F32)[None, :], beta.astype(F32)[None, :])


def rot_q8_1024(
    x: np.ndarray, gamma: np.ndarray | None = None, beta: np.ndarray | None = None, eps: float = 1e-5
) -> tuple[np.ndarray, np.ndarray]:
    """x fp16 [T, 1024] -> (int8 codes [T, 1024], fp32 row scale [T]).

    [LayerNorm] -> 1024-point FWHT with stages over column bits 0,1,2,8,9,3,4,5,6,7 -> x 1/32 -> per-row int8.
    Reference: rot_q8_1024_kernel, kernels.cu:49-108 (FWHT kernels.cu:13-47); eps is 1e-5 there (kernels.cu:80)."""
    assert x.ndim == 2 and x.shape[1] == 1024
    v = x.astype(np.float16).astype(F32)
    if gamma is not None:
        v = layer_norm_1024(v, gamma, beta, eps)
    v = fwht_rows(v, STAGES_1024) * F32(0.03125)
    return quant_rows(v)


def h128_groups(C: int) -> int:
    """16-lane groups per row in the block-128 kernel: 2 (a 32-lane half-wave per row) when the row's block count is
    even but not a multiple of 4 (768 = 6 blocks, 2816 = 22; at most 12 blocks per group), else 4 (a wave per row)."""
    nb = C // 128
    return 2 if nb % 2 == 0 and nb % 4 and nb // 2 <= 12 else 4


def layer_norm_h128(v: np.ndarray, c_real: int, gamma: np.ndarray, beta: np.ndarray, eps: float) -> np.ndarray:
    """LayerNorm over the first c_real of C columns (the rest are zero padding and stay zero).

    Reduction order of the HIP kernel that fuses this norm into the block-128 rotation (G = h128_groups(C) groups of
    16 lanes per row): lane 16g + l owns, for i = 0, 1, ..., the columns (G i + g)*128 + 8*gray(l) + e (e = 0..7,
    gray(l) = l ^ (l >> 1)) and sums the real ones sequentially in (i, e) order; the 16 G partial sums are combined by
    the xor tree over lanes 32 (G = 4 only), 16, 15, 7, 3, 1. mean = sum / c_real and var = sumsq / c_real are IEEE
    divisions; rstd = 1 / sqrt(var + eps).
    As in layer_norm_1024, the squares accumulate as fma(d, d, sq) and the output is fma(d * rstd, gamma, beta).
    (The reference has no such fused norm: its CUDA path is PixAI's GELU MLP. The op order follows the EVA02 SwiGLU +
    LayerNorm of foidfinder/backends/mlx/kernels.py:31-72.)"""
    T, C = v.shape
    nb = C // 128
    G = h128_groups(C)
    ni = (nb + G - 1) // G
    real = np.arange(C) < c_real
    cols = np.full((16 * G, ni * 8), -1, np.int64)  # [lane, i*8 + e] -> column (-1: outside the row)
    for lane in range(16 * G):
        g, l16 = lane >> 4, lane & 15
        gl = l16 ^ (l16 >> 1)
        for i in range(ni):
            b = G * i + g
            if b < nb:
                cols[lane, i * 8 : i * 8 + 8] = b * 128 + 8 * gl + np.arange(8)
    valid = (cols >= 0) & real[np.maximum(cols, 0)]
    safe = np.maximum(cols, 0)
    gathered = np.where(valid[None], v[:, safe], F32(0.0))  # [T, 64, ni*8]
    s = np.zeros((T, 16 * G), F32)
    for k in range(ni * 8):
        s = s + gathered[:, :, k]
    masks = (32, 16, 15, 7, 3, 1) if G == 4 else (16, 15, 7, 3, 1)
    mean = _xor_tree(s, masks) / F32(c_real)
    d = np.where(real[None, :], v - mean[:, None], F32(0.0)).astype(F32)
    dg = np.where(valid[None], d[:, safe], F32(0.0))
    sq = np.zeros((T, 16 * G), F32)
    for k in range(ni * 8):
        sq = fma32(dg[:, :, k], dg[:, :, k], sq)
    var = _xor_tree(sq, masks) / F32(c_real)
    rstd = F32(1.0) / np.sqrt(var + F32(eps))
    g_full = np.zeros(C, F32)
    b_full = np.zeros(C, F32)
    g_full[:c_real] = gamma
    b_full[:c_real] = beta
    y = fma32(d * rstd[:, None], g_full[None, :], b_full[None, :])
    return np.where(real[None, :], y, F32(0.0)).astype(F32)


def rot_q8_h128(
    x: np.ndarray,
    c_real: int | None = None,
    gamma: np.ndarray | None = None,
    beta: np.ndarray | None = None,
    eps: float = 1e-6,
) -> tuple[np.ndarray, np.ndarray]:
    """x fp16 [T, C] (C a multiple of 128) -> (int8 [T, C], fp32 row scale [T]).

    [LayerNorm over the first c_real columns] -> block-diagonal 128-point FWHT (stages over column bits 0..6 in
    ascending order) -> x fp32(1/sqrt(128)) -> absmax over the whole row -> int8.
    Reference: rot_q8_h128_kernel, kernels.cu:112-160."""
    assert x.ndim == 2 and x.shape[1] % 128 == 0
    T, C = x.shape
    v = x.astype(np.float16).astype(F32)
    if gamma is not None:
        v = layer_norm_h128(v, C if c_real is None else c_real, gamma, beta, eps)
    blocks = fwht_rows(v.reshape(T * (C // 128), 128), (0, 1, 2, 3, 4, 5, 6)).reshape(T, C)
    return quant_rows(blocks * INV_SQRT_128)
