"""The EVA02 tagger's float forward and the single W8A8 linear in PyTorch on the CPU: the CPU baseline.

Test and measurement infrastructure, like the rest of this package: `bench.py`'s `cpu_baseline` leg times these on
the host cores. tests/test_oracle.py pins them against the numpy restatements: `forward_float`'s logits against
`model.head_logits(model.forward_float_x(...))` (float64) on a 2-block model, `rot_q8` code for code and scale for
scale against `rotq8.rot_q8_1024`, and `w8a8_linear` within one fp16 ulp of `rotq8.rot_q8_1024` followed by
`gemm.gemm_s8(..., EPI_BIAS_F16)`. Nothing in the product imports them.

`forward_float` follows the op order of the reference's PyTorch model (foidfinder/backends/cuda/reference.py:109-131:
patch GEMM + positions, per block LayerNorm -> qkv linear -> RoPE on q and k -> scaled-dot-product attention -> proj
linear + residual -> LayerNorm -> MLP -> + residual, then the head), adapted to EVA02-L/14-448: a cls token, EVA02's
axial RoPE on the patch tokens only (foidfinder/backends/mlx/haruka.py:22-33), and the SwiGLU MLP with its LayerNorm
(foidfinder/backends/mlx/haruka.py:86-99), in fp32 throughout.

`w8a8_linear` is the plumbing config's single linear on the CPU: the 1024-point Walsh-Hadamard rotation of the
activations in the reference's butterfly order, per-token symmetric int8 quantization (`rot_q8`,
foidfinder/backends/cuda/csrc/kernels.cu:13-108), the int8 x int8 product accumulated exactly (fp32 products of
integers below 2^24 in magnitude are exact, K * 127^2 < 2^24 for K <= 1040), and the dequant + bias epilogue
(gemm.cuh:135-136; here `acc * rs * cs + bias` rounds after each operation, where the reference's compiler fuses the
last multiply and add).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair rotation of x [B, H, L, 64] by cos/sin [L, 32]."""
    x0, x1 = x[..., 0::2], x[..., 1::2]
    return torch.stack((x0 * cos - x1 * sin, x0 * sin + x1 * cos), dim=-1).flatten(-2)


@torch.no_grad()
def forward_float(images: torch.Tensor, raw: dict[str, torch.Tensor], depth: int, heads: int, patch: int,
                  hidden: int, rope: tuple[torch.Tensor, torch.Tensor], eps: float = 1e-6) -> torch.Tensor:
    """images [B, S, S, 3] float -> logits [B, tags] fp32. `raw` is the float EVA02 state dict (the engine's
    synthetic_checkpoint layout: fc1 gate rows then value rows), `rope` the fp32 cos/sin [L, 32] tables."""
    B, S = images.shape[0], images.shape[1]
    g = S // patch
    d = raw["cls_token"].numel()
    L = 1 + g * g
    x = images.float().view(B, g, patch, g, patch, 3).permute(0, 1, 3, 2, 4, 5).reshape(B, g * g, -1)
    x = F.linear(x, raw["patch_embed.weight"], raw["patch_embed.bias"])
    x = torch.cat((raw["cls_token"].view(1, 1, d).expand(B, 1, d), x), dim=1) + raw["pos_embed"].view(1, L, d)
    cos, sin = rope
    for i in range(depth):
        p = f"blocks.{i}."
        h = F.layer_norm(x, (d,), raw[p + "norm1.weight"], raw[p + "norm1.bias"], eps)
        q, k, v = F.linear(h, raw[p + "attn.qkv.weight"], raw[p + "attn.qkv.bias"]).view(B, L, 3, heads, 64).permute(
            2, 0, 3, 1, 4)
        o = F.scaled_dot_product_attention(_rope(q, cos, sin), _rope(k, cos, sin), v)
        x = x + F.linear(o.transpose(1, 2).reshape(B, L, d), raw[p + "attn.proj.weight"], raw[p + "attn.proj.bias"])
        h = F.layer_norm(x, (d,), raw[p + "norm2.weight"], raw[p + "norm2.bias"], eps)
        gv = F.linear(h, raw[p + "mlp.fc1.weight"], raw[p + "mlp.fc1.bias"])
        h = F.silu(gv[..., :hidden]) * gv[..., hidden:]
        h = F.layer_norm(h, (hidden,), raw[p + "mlp.norm.weight"], raw[p + "mlp.norm.bias"], eps)
        x = x + F.linear(h, raw[p + "mlp.fc2.weight"], raw[p + "mlp.fc2.bias"])
    cls = F.layer_norm(x[:, 0], (d,), raw["norm.weight"], raw["norm.bias"], eps)
    return F.linear(cls, raw["head.weight"], raw["head.bias"])


def fwht_1024(x: torch.Tensor) -> torch.Tensor:
    """Rows of x [M, 1024] times the normalized Sylvester Hadamard matrix, in fp32 butterflies over the column bits
    in the reference's stage order 0, 1, 2, 8, 9, 3, 4, 5, 6, 7 (kernels.cu:13-47), then x 1/32."""
    m = x.shape[0]
    for bit in (0, 1, 2, 8, 9, 3, 4, 5, 6, 7):
        half = 1 << bit
        v = x.reshape(m, 1024 // (2 * half), 2, half)
        x = torch.stack((v[:, :, 0] + v[:, :, 1], v[:, :, 0] - v[:, :, 1]), dim=2).reshape(m, 1024)
    return x * 0.03125


@torch.no_grad()
def rot_q8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x fp16 [M, 1024] -> (int8 codes as fp32 [M, 1024], fp32 row scale [M]): rotate, then per-token absmax int8
    (scale = max(amax, 1e-12) / 127, codes = clamp(round-half-even(v * (1 / scale)), -127, 127); kernels.cu:93-107)."""
    v = fwht_1024(x.float())
    scale = v.abs().amax(1).clamp_min(1e-12) / 127.0
    return torch.round(v * (1.0 / scale)[:, None]).clamp_(-127, 127), scale


@torch.no_grad()
def w8a8_linear(x: torch.Tensor, qweight: torch.Tensor, wscale: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """x fp16 [M, 1024] -> fp16 [M, N]: rotate, quantize per token, exact int8 product, dequantize, add bias."""
    codes, scale = rot_q8(x)
    acc = codes @ qweight.float().t()  # integer-valued fp32, exact for K * 127^2 < 2^24
    return (acc * scale[:, None] * wscale[None, :] + bias[None, :]).half()
