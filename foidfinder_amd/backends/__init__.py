"""Compute backends, imported lazily so only the selected one's dependencies are needed.

Mirrors foidfinder/backends/__init__.py:14-53 with a `rocm` entry: `detect()` returns "rocm" when PyTorch is a ROCm
build with a visible GPU (the reference returns "cuda" whenever torch.cuda.is_available(), which is also true on
ROCm), and `load("rocm", model_dir)` builds the MI355X int8 engine.
"""

from __future__ import annotations

import platform
import sys
from importlib.util import find_spec
from pathlib import Path
from typing import ClassVar, Protocol

import numpy as np

NAMES = ("mlx", "cuda", "rocm")


class Backend(Protocol):
    name: ClassVar[str]
    device: str

    def predict(self, image) -> np.ndarray:
        """Decoded image -> [num_tags] float32 probabilities. Call from one thread only."""
        ...


def detect() -> str:
    """The backend this machine can run: MLX on Apple Silicon, ROCm on an AMD GPU, else CUDA if a GPU is visible."""
    if sys.platform == "darwin" and platform.machine() == "arm64" and find_spec("mlx"):
        return "mlx"
    if find_spec("torch"):
        import torch

        if torch.cuda.is_available():
            return "rocm" if torch.version.hip else "cuda"
    raise RuntimeError(
        "no supported accelerator: install the mlx extra on Apple Silicon, or run on a machine with an AMD "
        "(ROCm) or NVIDIA GPU"
    )


def load(name: str, model_dir: Path) -> Backend:
    """name: "auto", "mlx", "cuda" or "rocm". Only "rocm" is provided by this package."""
    if name == "auto":
        name = detect()
    if name == "rocm":
        from .rocm import ROCmBackend

        return ROCmBackend(model_dir)
    if name in ("mlx", "cuda"):
        raise RuntimeError(f"the {name} backend belongs to the reference package (foidfinder.backends.{name})")
    raise ValueError(f"unknown backend {name!r}; choose auto, {', '.join(NAMES)}")
