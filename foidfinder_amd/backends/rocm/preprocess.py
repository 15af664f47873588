"""Letterbox preprocessing.

`preprocess` (PixAI, EVA02 int8): alpha composited onto white, antialiased bilinear resize on the GPU so the longer
side is `size`, pixels normalized to [-1, 1], padded with -1, NHWC fp16 (the engine's input layout); the steps of the
reference's PixAI preprocessing (foidfinder/backends/cuda/preprocess.py:16-32), at the model's own input size.

`preprocess_haruka` (Haruka): the model card's preprocessing (foidfinder/backends/mlx/haruka.py:63-72, the
reference's tests/test_haruka.py:19-34): composited onto white, Pillow bicubic resize so the longer side is `size`,
pasted centered on a white canvas, raw uint8 pixels NHWC (the normalization is folded into the patch weights).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F
from PIL import Image


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


@torch.no_grad()
def preprocess_haruka(images: list[Image.Image], size: int, device: str | torch.device = "cuda") -> torch.Tensor:
    """PIL images -> [B, size, size, 3] uint8 letterboxed pixels on the GPU."""
    out = np.empty((len(images), size, size, 3), np.uint8)
    for b, image in enumerate(images):
        rgb = rgb_on_white(image)
        w, h = rgb.size
        if (w, h) != (size, size):
            r = min(size / w, size / h)
            nw, nh = max(1, int(w * r)), max(1, int(h * r))
            canvas = Image.new("RGB", (size, size), (255, 255, 255))
            canvas.paste(rgb.resize((nw, nh), Image.Resampling.BICUBIC), ((size - nw) // 2, (size - nh) // 2))
            rgb = canvas
        out[b] = np.asarray(rgb)
    return torch.from_numpy(out).to(device)
