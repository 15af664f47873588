"""ROCm backend: the gfx950 int8 engines behind the reference's Backend protocol.

Mirrors CUDABackend (foidfinder/backends/cuda/__init__.py:15-43): constructor (model_dir) raising RuntimeError with
a readable message when unsupported, `name`, `device`, and `predict(image) -> float32 probabilities [num_tags]`
(sigmoid applied), called from one thread. Adds `predict_batch(images) -> [B, num_tags]` for batched serving.
Model directories: PixAI Tagger v1.0 (the reference's own, config.json + model.safetensors with official or
converted weights), Haruka Tagger (config architecture "haruka-eva02-tree", the folded or compressed checkpoint that
foidfinder/haruka.py and haruka_quant.py write; the reference serves it on MLX only), and this package's EVA02 int8
taggers (config architecture "eva02-int8").
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from .preprocess import preprocess, preprocess_haruka


class ROCmBackend:
    name = "rocm"

    def __init__(self, model_dir: Path):
        if not torch.cuda.is_available() or not torch.version.hip:
            raise RuntimeError("ROCm backend: no AMD GPU visible (needs a ROCm build of PyTorch)")
        arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
        if arch != "gfx950":
            raise RuntimeError(f"ROCm backend: kernels are built for gfx950 (MI355X), found {arch}")
        config = json.loads((Path(model_dir) / "config.json").read_text())
        arch_name = config.get("model", {}).get("architecture") if isinstance(config.get("model"), dict) else None
        self._preprocess = preprocess
        if arch_name == "eva02-int8":  # this package's EVA02 int8 tagger format
            from ...engine import load_model_dir

            self.engine, self.config = load_model_dir(model_dir)
        elif arch_name == "haruka-eva02-tree":  # as the MLX backend selects it (mlx/__init__.py:22-23)
            from ...haruka import load_haruka_dir

            self.engine, self.config = load_haruka_dir(model_dir)
            self._preprocess = preprocess_haruka
        elif "categories" in config:
            raise RuntimeError(f"ROCm backend: unsupported model architecture {arch_name!r}")
        else:  # PixAI Tagger v1.0: official weights or the converted int8 format (cuda/__init__.py:28-31)
            from ...pixai import load_pixai_dir

            self.engine, self.config = load_pixai_dir(model_dir)
        self.size = self.engine.cfg.img_size
        self.device = torch.cuda.get_device_name()

    @torch.no_grad()
    def predict(self, image) -> np.ndarray:
        return self.predict_batch([image])[0]

    @torch.no_grad()
    def predict_batch(self, images: list) -> np.ndarray:
        logits = self.engine(self._preprocess(images, self.size))
        return torch.sigmoid(logits).cpu().numpy()
