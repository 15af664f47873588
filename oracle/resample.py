"""Pillow's 8-bit bicubic resampling in numpy: the letterbox of the Haruka model card, restated.

Test infrastructure (like every module of this package): only the tests use it, as the checker of the GPU resize
kernel; the tests also hold it against Pillow itself.

The algorithm (Pillow's libImaging/Resample.c, as the reference restates it in
foidfinder/backends/mlx/kernels.py:75-186): per output index i along an axis, center = (i + 0.5) * scale, the taps
are the input indices in [trunc(center - support + 0.5), trunc(center + support + 0.5)) clipped to the input, with
weights filter((j - center + 0.5) / filterscale) (bicubic, a = -0.5, support 2 * max(scale, 1)) divided by their
sequential sum and rounded half away from zero to 22-bit fixed point. A pass sums code * weight over the taps
starting from 2^21 and keeps bits 22 and up, clipped to 0..255. Two passes: horizontal, then vertical over only the
rows the vertical pass reads, or vertical first. Which pass runs first depends on the Pillow version: Pillow 13 (the
version the reference pins, uv.lock) runs the vertical pass first when the height shrinks more than twice as much as
the width (the reference's resize_pad and its test at tests/test_haruka.py:39-55); Pillow 12 (this image's) does so
when the source is more than 100 times as tall as it is wide (measured against Image.resize on both sides of the
boundary: 9 x 900 horizontal first, 9 x 910 vertical first, likewise at widths 2-50).
"""

from __future__ import annotations

import math

import numpy as np

PRECISION_BITS = 22  # 32 - 8 - 2 (Resample.c, 8 bits per channel)


def bicubic(x: np.ndarray) -> np.ndarray:
    """Keys' cubic with a = -0.5."""
    x = np.abs(x)
    a = -0.5
    return np.where(x < 1.0, ((a + 2.0) * x - (a + 3.0)) * x * x + 1.0,
                    np.where(x < 2.0, (((x - 5.0) * x + 8.0) * x - 4.0) * a, 0.0))


def coeffs(in_size: int, out_size: int) -> tuple[np.ndarray, np.ndarray]:
    """-> (kk int32 [out_size, ksize] fixed-point taps, bounds int32 [out_size, 2] = (first input, tap count))."""
    scale = in_size / out_size
    filterscale = max(scale, 1.0)
    support = 2.0 * filterscale
    ksize = int(math.ceil(support)) * 2 + 1
    kk = np.zeros((out_size, ksize), np.int32)
    bounds = np.zeros((out_size, 2), np.int32)
    for i in range(out_size):
        center = (i + 0.5) * scale
        xmin = max(int(center - support + 0.5), 0)  # int() truncates toward zero, as the C cast
        xmax = min(int(center + support + 0.5), in_size) - xmin
        w = [float(bicubic(np.float64((j + xmin - center + 0.5) * (1.0 / filterscale)))) for j in range(xmax)]
        total = 0.0
        for v in w:
            total += v
        if total != 0.0:
            w = [v / total for v in w]
        for j, v in enumerate(w):
            kk[i, j] = int(-0.5 + v * (1 << PRECISION_BITS)) if v < 0 else int(0.5 + v * (1 << PRECISION_BITS))
        bounds[i] = (xmin, xmax)
    return kk, bounds


def resample_pass(src: np.ndarray, axis: int, kk: np.ndarray, bounds: np.ndarray, out_hw: tuple[int, int],
                  region: tuple[int, int, int, int], row0: int = 0) -> np.ndarray:
    """One pass along axis (0: width, 1: height) of uint8 src [H, W, 3] into region (top, left, h, w) of a white
    uint8 canvas out_hw; inside the region, output (y, x) reads source row row0 + y (axis 0) or column x (axis 1)."""
    out = np.full((*out_hw, 3), 255, np.uint8)
    top, left, h, w = region
    s = src.astype(np.int64)
    for o in range(w if axis == 0 else h):
        first, taps = int(bounds[o, 0]), int(bounds[o, 1])
        k = kk[o, :taps].astype(np.int64)
        if axis == 0:
            acc = (s[row0 : row0 + h, first : first + taps, :] * k[None, :, None]).sum(1) + (1 << 21)
            out[top : top + h, left + o, :] = np.clip(acc >> PRECISION_BITS, 0, 255)
        else:
            acc = (s[row0 + first : row0 + first + taps, :w, :] * k[:, None, None]).sum(0) + (1 << 21)
            out[top + o, left : left + w, :] = np.clip(acc >> PRECISION_BITS, 0, 255)
    return out


def vertical_first(w: int, h: int, nw: int, nh: int, pillow_major: int) -> bool:
    """Whether Pillow resamples the height before the width for a w x h -> nw x nh resize."""
    if pillow_major >= 13:
        return h - nh > 0 and h - nh > (w - nw) * 2
    return h > 100 * w


def letterbox(rgb: np.ndarray, size: int, pillow_major: int = 12) -> np.ndarray:
    """uint8 [H, W, 3] -> uint8 [size, size, 3]: bicubic resize so the longer side is size (each side at least 1,
    truncated as int(side * ratio)), centered on white."""
    h, w = rgb.shape[:2]
    if (w, h) == (size, size):
        return rgb.copy()
    r = min(size / w, size / h)
    nw, nh = max(1, int(w * r)), max(1, int(h * r))
    top, left = (size - nh) // 2, (size - nw) // 2
    kh, bh = coeffs(w, nw)
    kv, bv = coeffs(h, nh)
    if vertical_first(w, h, nw, nh, pillow_major):
        tmp = resample_pass(rgb, 1, kv, bv, (nh, w), (0, 0, nh, w))
        return resample_pass(tmp, 0, kh, bh, (size, size), (top, left, nh, nw))
    row0 = int(bv[0, 0])
    rows = int(bv[-1, 0] + bv[-1, 1]) - row0
    tmp = resample_pass(rgb, 0, kh, bh, (rows, nw), (0, 0, rows, nw), row0)
    bv = bv - np.array([row0, 0], np.int32)
    return resample_pass(tmp, 1, kv, bv, (size, size), (top, left, nh, nw))


def bilinear_aa_matrix(in_size: int, out_size: int) -> np.ndarray:
    """Antialiased bilinear resampling along one axis as a float64 [out_size, in_size] matrix: what PixAI's
    preprocessing (torchvision's resize, i.e. torch's interpolate(mode="bilinear", antialias=True,
    align_corners=False); foidfinder/backends/cuda/preprocess.py:27-28) computes.

    scale = in / out. Output i is centered at input coordinate (i + 0.5) * scale; the filter is the triangle
    max(0, 1 - |t|) with t = (j + 0.5 - center) / max(scale, 1), i.e. stretched over the downscale factor so that
    every input pixel contributes (plain bilinear when enlarging). The taps are the input indices j in
    [trunc(center - support + 0.5), trunc(center + support + 0.5)) clipped to the input, support = max(scale, 1), and
    their weights are divided by their sum (so rows at the borders renormalize instead of reading past the edge)."""
    scale = in_size / out_size
    stretch = max(scale, 1.0)
    out = np.zeros((out_size, in_size), np.float64)
    for i in range(out_size):
        center = (i + 0.5) * scale
        lo = max(int(center - stretch + 0.5), 0)
        hi = min(int(center + stretch + 0.5), in_size)
        j = np.arange(lo, hi)
        w = np.maximum(0.0, 1.0 - np.abs((j + 0.5 - center) / stretch))
        if w.sum() > 0:
            out[i, lo:hi] = w / w.sum()
    return out


def resize_2d(x: np.ndarray, rows: np.ndarray, cols: np.ndarray) -> np.ndarray:
    """x [H, W, C] -> rows @ x @ cols^T per channel: [nh, nw, C] (separable resampling, float64)."""
    t = np.tensordot(rows, x, axes=(1, 0))  # [nh, W, C]
    return np.tensordot(t, cols, axes=(1, 1)).transpose(0, 2, 1)  # [nh, C, nw] -> [nh, nw, C]


def letterbox_pixai(rgb: np.ndarray, size: int) -> np.ndarray:
    """PixAI's letterbox (foidfinder/backends/cuda/preprocess.py:16-32) in float64: uint8 RGB [H, W, 3] scaled to
    [0, 1], resized with the antialiased bilinear filter so the longer side is `size` (the other side int(side * r),
    r = min(size / H, size / W); no resize when that leaves the size unchanged), normalized to [-1, 1] and centered on
    a canvas of -1 at offsets ((size - nh) // 2, (size - nw) // 2). Returns float64 [size, size, 3].
    Each side is at least 1: the reference's int(side * r) is 0 for an image more than `size` times as wide as tall
    (or tall as wide), where its interpolate call raises; the served letterbox keeps one row (or column) instead."""
    h, w = rgb.shape[:2]
    x = rgb.astype(np.float64) / 255.0
    r = min(size / h, size / w)
    nh, nw = max(1, int(h * r)), max(1, int(w * r))
    if (nh, nw) != (h, w):
        x = resize_2d(x, bilinear_aa_matrix(h, nh), bilinear_aa_matrix(w, nw))
    out = np.full((size, size, 3), -1.0)
    top, left = (size - nh) // 2, (size - nw) // 2
    out[top : top + nh, left : left + nw] = x * 2.0 - 1.0
    return out
