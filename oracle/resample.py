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
