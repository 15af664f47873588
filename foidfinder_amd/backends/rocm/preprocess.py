"""Letterbox preprocessing.

`preprocess` (PixAI, EVA02 int8): alpha composited onto white, antialiased bilinear resize on the GPU so the longer
side is `size`, pixels normalized to [-1, 1], padded with -1, NHWC fp16 (the engine's input layout); the steps of the
reference's PixAI preprocessing (foidfinder/backends/cuda/preprocess.py:16-32), at the model's own input size.

`preprocess_haruka` (Haruka): the model card's preprocessing (foidfinder/backends/mlx/haruka.py:63-72, the
reference's tests/test_haruka.py:19-34): composited onto white, Pillow bicubic resize so the longer side is `size`,
pasted centered on a white canvas, raw uint8 pixels NHWC (the normalization is folded into the patch weights). The
resize runs on the GPU (`ff_resample_u8`, two separable passes with Pillow's fixed-point taps computed here) and is
bit-exact with Pillow 13's `Image.resize(BICUBIC)` (the version the reference pins), as the reference's Metal resize
is (foidfinder/backends/mlx/kernels.py:75-186).
"""

from __future__ import annotations

import math

import numpy as np
import PIL
import torch
import torch.nn.functional as F
from PIL import Image

PILLOW_MAJOR = int(PIL.__version__.split(".")[0])


def vertical_first(w: int, h: int, nw: int, nh: int) -> bool:
    """Whether the resize resamples the height before the width (the passes do not commute: each rounds to 8 bits).
    Always the rule of Pillow 13, the version the reference pins (uv.lock) and hard-codes in its own resize: the
    vertical pass first when the height shrinks more than twice as much as the width (the reference's resize_pad,
    foidfinder/backends/mlx/kernels.py:180-182). So the served pixels do not depend on the Pillow installed here
    (Pillow 12 orders the passes by another rule and differs in the last bit on tall images such as 448 x 900)."""
    return h - nh > 0 and h - nh > (w - nw) * 2


def rgb_on_white(image: Image.Image) -> Image.Image:
    """RGB with any transparency composited onto a white background."""
    if image.mode == "RGB":
        return image
    rgba = image.convert("RGBA")
    canvas = Image.new("RGBA", rgba.size, (255, 255, 255, 255))
    canvas.alpha_composite(rgba)
    return canvas.convert("RGB")


@torch.no_grad()
def preprocess(images: list[Image.Image], size: int, device: str | torch.device = "cuda") -> torch.Tensor:
    """PIL images -> [B, size, size, 3] fp16 normalized pixels."""
    out = torch.full((len(images), size, size, 3), -1.0, device=device, dtype=torch.half)
    for b, image in enumerate(images):
        rgb = torch.from_numpy(np.array(rgb_on_white(image))).to(device, non_blocking=True)
        x = rgb.permute(2, 0, 1)[None].float().div_(255.0)
        h, w = x.shape[-2:]
        r = min(size / h, size / w)
        nh, nw = max(1, int(h * r)), max(1, int(w * r))
        if (nh, nw) != (h, w):
            x = F.interpolate(x, size=(nh, nw), mode="bilinear", align_corners=False, antialias=True)
        top, left = (size - nh) // 2, (size - nw) // 2
        out[b, top : top + nh, left : left + nw] = (x[0].permute(1, 2, 0) * 2.0 - 1.0).half()
    return out


def bicubic_taps(in_size: int, out_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Pillow's bicubic filter taps along one axis (libImaging/Resample.c precompute_coeffs + normalize_coeffs_8bpc,
    a = -0.5): kk int32 [out_size, ksize] in 22-bit fixed point, bounds int32 [out_size, 2] = (first input index, tap
    count). The same float64 operations in the same order as the C code, so the taps are Pillow's to the bit."""
    scale = in_size / out_size
    filterscale = max(scale, 1.0)
    support = 2.0 * filterscale
    ksize = math.ceil(support) * 2 + 1
    center = (np.arange(out_size, dtype=np.float64) + 0.5) * scale
    first = np.maximum(np.trunc(center - support + 0.5), 0.0).astype(np.int64)
    count = np.minimum(np.trunc(center + support + 0.5).astype(np.int64), in_size) - first
    j = np.arange(ksize)
    x = np.abs(((j[None, :] + first[:, None]) - center[:, None] + 0.5) * (1.0 / filterscale))
    w = np.where(x < 1.0, (1.5 * x - 2.5) * x * x + 1.0, np.where(x < 2.0, (((x - 5.0) * x + 8.0) * x - 4.0) * -0.5, 0.0))
    w[j[None, :] >= count[:, None]] = 0.0
    total = np.zeros(out_size)
    for t in range(ksize):  # sequential sum, as the C loop
        total = total + w[:, t]
    w = np.divide(w, total[:, None], out=w.copy(), where=total[:, None] != 0.0)
    kk = np.trunc(np.where(w < 0, -0.5 + w * (1 << 22), 0.5 + w * (1 << 22))).astype(np.int32)
    return kk, np.stack([first, count], axis=1).astype(np.int32)


def letterbox_gpu(rgb: np.ndarray, size: int, out: torch.Tensor) -> None:
    """uint8 [H, W, 3] -> out uint8 [size, size, 3] on the GPU: bicubic resize so the longer side is size (the other
    side int(side * ratio), at least 1), centered on white; two passes of ff_resample_u8."""
    from ...kernels import resample_u8

    h, w = rgb.shape[:2]
    dev = out.device
    src = torch.from_numpy(np.require(rgb, requirements=["C", "W"])).to(dev)  # PIL arrays are read-only
    if (w, h) == (size, size):
        out.copy_(src)
        return
    r = min(size / w, size / h)
    nw, nh = max(1, int(w * r)), max(1, int(h * r))
    top, left = (size - nh) // 2, (size - nw) // 2
    kh, bh = bicubic_taps(w, nw)
    kv, bv = bicubic_taps(h, nh)

    def dev_t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    if vertical_first(w, h, nw, nh):
        tmp = torch.empty(nh, w, 3, dtype=torch.uint8, device=dev)
        resample_u8(src, 1, dev_t(kv), dev_t(bv), 0, tmp, (0, 0, nh, w))
        resample_u8(tmp, 0, dev_t(kh), dev_t(bh), 0, out, (top, left, nh, nw))
        return
    row0 = int(bv[0, 0])  # only the source rows the vertical pass reads
    rows = int(bv[-1, 0] + bv[-1, 1]) - row0
    tmp = torch.empty(rows, nw, 3, dtype=torch.uint8, device=dev)
    resample_u8(src, 0, dev_t(kh), dev_t(bh), row0, tmp, (0, 0, rows, nw))
    resample_u8(tmp, 1, dev_t(kv), dev_t(bv - np.array([row0, 0], np.int32)), 0, out, (top, left, nh, nw))


@torch.no_grad()
def preprocess_haruka(images: list[Image.Image], size: int, device: str | torch.device = "cuda") -> torch.Tensor:
    """PIL images -> [B, size, size, 3] uint8 letterboxed pixels on the GPU."""
    out = torch.empty(len(images), size, size, 3, dtype=torch.uint8, device=device)
    for b, image in enumerate(images):
        letterbox_gpu(np.asarray(rgb_on_white(image)), size, out[b])
    return out
