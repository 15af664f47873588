"""The gfx950 kernel library behind a C ABI (include/foidfinder_rocm.h), loaded with ctypes and registered as
`torch.ops.foidfinder_rocm.*` with the reference's op schemas.

Mirrors foidfinder/backends/cuda/kernels.py:38-48 (`kernels()` -> the op namespace) and the op registration of
foidfinder/backends/cuda/csrc/kernels.cu:267-281. Every op is out-param / in-place, returns nothing, allocates
nothing and launches on the current stream, so a forward built from them can be captured in a HIP graph. Failed
preconditions raise RuntimeError, as TORCH_CHECK does in the reference.

There is no CPU fallback: without the built library every call raises.
"""

from __future__ import annotations

import ctypes
import os
from functools import cache
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libfoidfinder_rocm.so"
ENV = "FOIDFINDER_ROCM_KERNELS"  # path to a prebuilt library (the reference's $FOIDFINDER_KERNELS)

# Epilogue codes (include/foidfinder_rocm.h); 0-2 as foidfinder/backends/cuda/engine.py:24.
EPI_QKV_ROPE, EPI_RESIDUAL, EPI_GELU_F16, EPI_SWIGLU, EPI_BIAS_F16, EPI_I32 = 0, 1, 2, 3, 4, 5

_vp, _i64, _f32, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
SIGNATURES = {
    "ff_abi_version": ([], _int),
    "ff_last_error": ([], ctypes.c_char_p),
    "ff_rot_q8_1024": ([_vp, _vp, _vp, _f32, _i64, _vp, _vp, _vp], _int),
    "ff_rot_q8_h128": ([_vp, _i64, _i64, _i64, _vp, _vp, _f32, _vp, _vp, _vp], _int),
    "ff_gemm_s8": ([_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _int, _int, _vp, _vp, _i64, _f32, _vp], _int),
    "ff_gemm_s8_variants": ([], _int),
    "ff_attention": ([_vp, _vp, _i64, _i64, _i64, _vp], _int),
    "ff_resample_u8": ([_vp, _i64, _i64, _int, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp],
                       _int),
    "ff_layer_norm2": ([_vp, _i64, _i64, _vp, _vp, _vp, _vp, _f32, _vp, _vp], _int),
    "ff_slot_weights_blocks": ([_i64], _i64),
    "ff_slot_weights": ([_vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp], _int),
}
ABI_VERSION = 3


@cache
def lib() -> ctypes.CDLL:
    """The loaded C library. torch is imported first so the library binds to the HIP runtime torch already loaded."""
    path = Path(os.environ.get(ENV, LIB_PATH))
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it with `python -m foidfinder_amd.build`")
    handle = ctypes.CDLL(str(path))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes, fn.restype = args, res
    if handle.ff_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI {handle.ff_abi_version()}, expected {ABI_VERSION}")
    return handle


def _check(status: int) -> None:
    if status != 0:
        raise RuntimeError(lib().ff_last_error().decode())


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _on_gpu(*ts: torch.Tensor | None) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        _require(t.is_cuda, "foidfinder_rocm ops take GPU tensors")
        _require(t.is_contiguous(), "foidfinder_rocm ops take contiguous tensors")
        dev = dev or t.device
        _require(t.device == dev, "all tensors must be on one device")


# ---- op implementations (raw; also callable directly, bypassing the dispatcher) ----


def rot_q8_1024(
    x: torch.Tensor,
    gamma: torch.Tensor | None,
    beta: torch.Tensor | None,
    out: torch.Tensor,
    row_scale: torch.Tensor,
    eps: float = 1e-5,
) -> None:
    """x fp16 [T, 1024] -> out int8 [T, 1024], row_scale fp32 [T]; LayerNorm(gamma, beta, eps) first if given."""
    _on_gpu(x, gamma, beta, out, row_scale)
    _require(x.dim() == 2 and x.size(1) == 1024 and x.dtype == torch.float16, "x must be fp16 [T, 1024]")
    _require(out.dtype == torch.int8 and out.shape == x.shape, "out must be int8 [T, 1024]")
    _require(row_scale.dtype == torch.float32 and row_scale.numel() == x.size(0), "row_scale must be fp32 [T]")
    if gamma is not None:
        _require(beta is not None, "gamma and beta go together")
        _require(gamma.dtype == beta.dtype == torch.float32 and gamma.numel() == beta.numel() == 1024,
                 "gamma/beta must be fp32 [1024]")
    with torch.cuda.device(x.device):
        _check(lib().ff_rot_q8_1024(_ptr(x), _ptr(gamma), _ptr(beta), eps, x.size(0), _ptr(out), _ptr(row_scale),
                                    _stream(x)))


def rot_q8_h128(
    x: torch.Tensor,
    out: torch.Tensor,
    row_scale: torch.Tensor,
    gamma: torch.Tensor | None = None,
    beta: torch.Tensor | None = None,
    c_real: int = 0,
    eps: float = 1e-6,
) -> None:
    """x fp16 [T, C] (C % 128 == 0) -> out int8 [T, C], row_scale fp32 [T]; LayerNorm over the first c_real columns
    (default: all) first if gamma is given. gamma/beta are fp32 [C] with zeros in columns >= c_real
    (`pad_norm` builds them)."""
    _on_gpu(x, out, row_scale, gamma, beta)
    _require(x.dim() == 2 and x.dtype == torch.float16, "x must be fp16 [T, C]")
    _require(out.dtype == torch.int8 and out.shape == x.shape, "out must be int8 [T, C]")
    _require(row_scale.dtype == torch.float32 and row_scale.numel() == x.size(0), "row_scale must be fp32 [T]")
    C = x.size(1)
    cr = c_real or C
    if gamma is not None:
        _require(beta is not None, "gamma and beta go together")
        _require(gamma.dtype == beta.dtype == torch.float32 and gamma.numel() == beta.numel() == C,
                 "gamma/beta must be fp32 [C], zero past c_real")
    with torch.cuda.device(x.device):
        _check(lib().ff_rot_q8_h128(_ptr(x), x.size(0), C, cr, _ptr(gamma), _ptr(beta), eps, _ptr(out),
                                    _ptr(row_scale), _stream(x)))


def pad_norm(weight: torch.Tensor, bias: torch.Tensor, C: int) -> tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm gamma/beta over c_real columns -> fp32 [C] with zeros past c_real, as rot_q8_h128 takes them."""
    g = torch.zeros(C, dtype=torch.float32, device=weight.device)
    b = torch.zeros(C, dtype=torch.float32, device=weight.device)
    g[: weight.numel()] = weight.float().reshape(-1)
    b[: bias.numel()] = bias.float().reshape(-1)
    return g, b


def out_shape(M: int, N: int, epi: int) -> tuple[int, int]:
    return (M, N // 2) if epi == EPI_SWIGLU else (M, N)


def gemm_s8(
    A: torch.Tensor,
    W: torch.Tensor,
    row_scale: torch.Tensor,
    col_scale: torch.Tensor,
    bias: torch.Tensor,
    out: torch.Tensor,
    epi: int,
    stages: int,
    rope_cos: torch.Tensor | None,
    rope_sin: torch.Tensor | None,
    q_scale: float,
) -> None:
    """A int8 [M, K] x W int8 [N, K] -> epilogue into out. `stages` selects the tile variant (0 = default), the
    knob the engine autotunes (the reference's pipeline depth)."""
    _on_gpu(A, W, row_scale, col_scale, bias, out, rope_cos, rope_sin)
    _require(A.dtype == W.dtype == torch.int8 and A.dim() == W.dim() == 2, "A and W must be int8 matrices")
    M, K = A.shape
    N = W.size(0)
    _require(W.size(1) == K, "A and W must share K")
    want = torch.int32 if epi == EPI_I32 else torch.float16
    _require(out.dtype == want and tuple(out.shape) == out_shape(M, N, epi), f"out must be {want} {out_shape(M, N, epi)}")
    if epi != EPI_I32:
        _require(row_scale.dtype == col_scale.dtype == bias.dtype == torch.float32, "scales and bias must be fp32")
        _require(row_scale.numel() == M and col_scale.numel() == N and bias.numel() == N, "scale/bias sizes")
    rope_len = 0
    if epi == EPI_QKV_ROPE:
        _require(rope_cos is not None and rope_sin is not None, "QKV epilogue needs RoPE tables")
        _require(rope_cos.dtype == rope_sin.dtype == torch.float32 and rope_cos.shape == rope_sin.shape
                 and rope_cos.dim() == 2 and rope_cos.size(1) == 32, "RoPE tables must be fp32 [L, 32]")
        rope_len = rope_cos.size(0)
    with torch.cuda.device(A.device):
        _check(lib().ff_gemm_s8(_ptr(A), _ptr(W), M, N, K, _ptr(row_scale), _ptr(col_scale), _ptr(bias), _ptr(out),
                                epi, stages, _ptr(rope_cos), _ptr(rope_sin), rope_len, q_scale, _stream(A)))


def attention(qkv: torch.Tensor, out: torch.Tensor, seq_len: int) -> None:
    """qkv fp16 [T, 3C] (q rotated and pre-scaled, k rotated) -> out fp16 [T, C]; heads of 64, any seq_len."""
    _on_gpu(qkv, out)
    _require(qkv.dtype == out.dtype == torch.float16, "qkv and out must be fp16")
    _require(qkv.dim() == 2 and qkv.size(1) % 192 == 0, "qkv must be [T, 3 * heads * 64]")
    C = qkv.size(1) // 3
    _require(out.shape == (qkv.size(0), C), "out must be [T, C]")
    with torch.cuda.device(qkv.device):
        _check(lib().ff_attention(_ptr(qkv), _ptr(out), qkv.size(0), C // 64, seq_len, _stream(qkv)))


def resample_u8(src: torch.Tensor, axis: int, kk: torch.Tensor, bounds: torch.Tensor, row0: int, out: torch.Tensor,
                region: tuple[int, int, int, int]) -> None:
    """One Pillow resampling pass (include/foidfinder_rocm.h, ff_resample_u8): src uint8 [H, W, 3] -> out uint8
    [out_h, out_w, 3], `region` = (top, left, h, w) resampled along axis 0 (width) or 1 (height), the rest white."""
    _on_gpu(src, kk, bounds, out)
    _require(src.dtype == out.dtype == torch.uint8 and src.dim() == out.dim() == 3 and src.size(2) == out.size(2) == 3,
             "src and out must be uint8 [rows, cols, 3]")
    _require(src.is_contiguous() and out.is_contiguous(), "src and out must be contiguous")
    _require(kk.dtype == bounds.dtype == torch.int32 and kk.dim() == 2 and bounds.dim() == 2 and bounds.size(1) == 2
             and kk.is_contiguous() and bounds.is_contiguous(), "kk int32 [n, ksize], bounds int32 [n, 2]")
    top, left, h, w = region
    n = w if axis == 0 else h
    _require(kk.size(0) >= n and bounds.size(0) >= n, "kk/bounds need a row per output index of the region")
    with torch.cuda.device(src.device):
        _check(lib().ff_resample_u8(_ptr(src), src.size(0), src.size(1), axis, _ptr(kk), _ptr(bounds), kk.size(1),
                                    row0, _ptr(out), out.size(0), out.size(1), top, left, h, w, _stream(src)))


def layer_norm2(x: torch.Tensor, g1: torch.Tensor, b1: torch.Tensor, g2: torch.Tensor, b2: torch.Tensor, eps: float,
                out: torch.Tensor) -> None:
    """out = LN(fp16(LN(x; g1, b1)); g2, b2) over the last dimension of fp16 x [..., C] (fp16 params [C])."""
    _on_gpu(x, g1, b1, g2, b2, out)
    C = x.size(-1)
    _require(x.dtype == out.dtype == torch.float16 and x.is_contiguous() and out.is_contiguous()
             and out.shape == x.shape, "x and out must be contiguous fp16 of one shape")
    _require(all(t.dtype == torch.float16 and t.numel() == C for t in (g1, b1, g2, b2)), "params must be fp16 [C]")
    with torch.cuda.device(x.device):
        _check(lib().ff_layer_norm2(_ptr(x), x.numel() // C, C, _ptr(g1), _ptr(b1), _ptr(g2), _ptr(b2), eps, _ptr(out),
                                    _stream(x)))


def slot_weights_blocks(N: int) -> int:
    return lib().ff_slot_weights_blocks(N)


def slot_weights(logits: torch.Tensor, c: torch.Tensor, bias: torch.Tensor, heads: int, a_t: torch.Tensor,
                 partial: torch.Tensor) -> None:
    """Tree-pool weights (include/foidfinder_rocm.h, ff_slot_weights): logits fp16 [B, N, heads*M] + c fp32 ([heads*M]
    shared or [B, heads*M]) -> a_t fp16 [B, heads*M, N], partial fp32 [B, blocks, heads*M]."""
    _on_gpu(logits, c, bias, a_t, partial)
    B, N, GM = logits.shape
    M = bias.numel()
    _require(logits.dtype == torch.float16 and logits.is_contiguous() and GM == heads * M, "logits fp16 [B, N, heads*M]")
    _require(c.dtype == bias.dtype == torch.float32 and c.is_contiguous() and bias.is_contiguous(), "c, bias fp32")
    _require(c.numel() in (GM, B * GM), "c must be [heads*M] or [B, heads*M]")
    _require(a_t.dtype == torch.float16 and a_t.is_contiguous() and a_t.shape == (B, GM, N), "a_t fp16 [B, heads*M, N]")
    _require(partial.dtype == torch.float32 and partial.is_contiguous()
             and partial.shape == (B, slot_weights_blocks(N), GM), "partial fp32 [B, blocks, heads*M]")
    with torch.cuda.device(logits.device):
        _check(lib().ff_slot_weights(_ptr(logits), _ptr(c), 0 if c.numel() == GM else GM, _ptr(bias), B, N, heads, M,
                                     _ptr(a_t), _ptr(partial), _stream(logits)))


# ---- torch.ops.foidfinder_rocm registration (schemas as kernels.cu:268-273, plus eps / the fused norm) ----

_LIB = torch.library.Library("foidfinder_rocm", "DEF")
_LIB.define(
    "gemm_s8(Tensor A, Tensor W, Tensor row_scale, Tensor col_scale, Tensor bias, Tensor(a!) out, int epi, "
    "int stages, Tensor? rope_cos, Tensor? rope_sin, float q_scale) -> ()"
)
_LIB.define("rot_q8_1024(Tensor x, Tensor? gamma, Tensor? beta, Tensor(a!) out, Tensor(b!) row_scale, "
            "float eps=1e-05) -> ()")
_LIB.define("rot_q8_h128(Tensor x, Tensor(a!) out, Tensor(b!) row_scale, Tensor? gamma=None, Tensor? beta=None, "
            "int c_real=0, float eps=1e-06) -> ()")
_LIB.define("attention(Tensor qkv, Tensor(a!) out, int seq_len) -> ()")
_LIB.impl("gemm_s8", gemm_s8, "CUDA")
_LIB.impl("rot_q8_1024", rot_q8_1024, "CUDA")
_LIB.impl("rot_q8_h128", rot_q8_h128, "CUDA")
_LIB.impl("attention", attention, "CUDA")
# Haruka's tree pool (no reference CUDA op; out-param ops in the same style)
_LIB.define("layer_norm2(Tensor x, Tensor g1, Tensor b1, Tensor g2, Tensor b2, float eps, Tensor(a!) out) -> ()")
_LIB.define("slot_weights(Tensor logits, Tensor c, Tensor bias, int heads, Tensor(a!) a_t, Tensor(b!) partial) -> ()")
_LIB.impl("layer_norm2", layer_norm2, "CUDA")
_LIB.impl("slot_weights", slot_weights, "CUDA")


@cache
def kernels():
    """The op namespace, loading the library (raises if it is missing). Mirrors the reference's `kernels()`."""
    lib()
    return torch.ops.foidfinder_rocm
