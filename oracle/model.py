"""Weight conversion, RoPE tables, synthetic EVA02-L/14-448 weights and the int8-semantics forward, in numpy.

Block dataflow (the reference's int8 block, foidfinder/backends/cuda/engine.py:150-160, with the EVA02 block of
foidfinder/backends/mlx/haruka.py:196-209):

  a8, rs = rot_q8_1024(x, norm1)            qkv = gemm(a8, Wqkv, QKV_ROPE)          o = attention(qkv)
  a8, rs = rot_q8_1024(o)                    x = gemm(a8, Wproj, RESIDUAL, x)
  a8, rs = rot_q8_1024(x, norm2)             h = gemm(a8, Wfc1, SWIGLU)  [M, 2816]
  h8, rs = rot_q8_h128(h, mlp_norm, 2730)    x = gemm(h8, Wfc2, RESIDUAL, x)

Weights carry the same rotations (W' = W H, engine.py:49-62) and are quantized per output channel (engine.py:37-41).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import attention as attn_mod
from . import gemm as G
from . import rotq8

F32 = np.float32
Q_SCALE = 0.125 * math.log2(math.e)  # engine.py:26: softmax scale x log2(e), folded into q by the QKV epilogue


def hadamard(n: int) -> np.ndarray:
    """Normalized Sylvester Hadamard matrix in float64 (engine.py:29-34): H[i, j] = (-1)^popcount(i & j) / sqrt(n)."""
    h = np.ones((1, 1), np.float64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h / math.sqrt(n)


def block_hadamard(k: int, n: int) -> np.ndarray:
    """blockdiag(H_n, ..., H_n) of size k (k a multiple of n), float64."""
    out = np.zeros((k, k), np.float64)
    h = hadamard(n)
    for b in range(k // n):
        out[b * n : (b + 1) * n, b * n : (b + 1) * n] = h
    return out


def quantize_rows_int8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-channel int8 (engine.py:37-41), in float32:
    scale = max(amax_row, 1e-12) / 127; q = clamp(round_half_even(w / scale), -127, 127)."""
    w = w.astype(F32)
    scale = np.maximum(np.abs(w).max(axis=1), F32(1e-12)) / F32(127.0)
    q = np.clip(np.rint(w / scale[:, None]), -127, 127).astype(np.int8)
    return np.ascontiguousarray(q), scale.astype(F32)


def rotate_rows64(w: np.ndarray, block: int) -> np.ndarray:
    """W [N, K] @ blockdiag(H_block) in float64 as a fast Walsh-Hadamard transform per block of K columns: butterflies
    (a, b) -> (a + b, a - b) over column bits 0, 1, 2, ... in that order, then x 1/sqrt(block); each step one IEEE
    float64 operation, so the bits do not depend on a BLAS summation order."""
    n, k = w.shape
    v = w.astype(np.float64).reshape(n, k // block, block)
    half = 1
    while half < block:
        v = v.reshape(n, k // block, block // (2 * half), 2, half)
        v = np.stack((v[..., 0, :] + v[..., 1, :], v[..., 0, :] - v[..., 1, :]), axis=-2)
        half *= 2
    return v.reshape(n, k) * (1.0 / math.sqrt(block))


def rotate_quantize(w: np.ndarray, block: int) -> tuple[np.ndarray, np.ndarray]:
    """W [N, K] -> quantize_rows_int8(W @ blockdiag(H_block)); the product in float64 (rotate_rows64), rounded to
    float32 once (the reference multiplies in float32, engine.py:59; float64 makes the codes platform-independent)."""
    return quantize_rows_int8(rotate_rows64(w, block).astype(F32))


def eva02_rope_tables(grid: int, ref: int, head_dim: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """EVA02 axial RoPE as consumed by the QKV epilogue: cos/sin fp32 [1 + grid^2, head_dim/2], one entry per
    interleaved (even, odd) pair; row 0 (cls) is the identity. Angles: pairs 0..15 use the row (y) position, pairs
    16..31 the column (x) position, positions rescaled to the pretraining grid. Every step in float32, as the
    reference's recipe (foidfinder/backends/mlx/haruka.py:22-33: float32 bands and positions, float32 products,
    numpy's float32 cos and sin; its tables repeat each pair's angle twice, kept here once per pair)."""
    q = head_dim // 4
    bands = F32(1.0) / (F32(10000.0) ** (np.arange(q, dtype=F32) / F32(q)))
    t = np.arange(grid, dtype=F32) / F32(grid) * F32(ref)
    ty, tx = np.meshgrid(t, t, indexing="ij")
    ang = np.concatenate([ty.reshape(-1, 1) * bands, tx.reshape(-1, 1) * bands], axis=1)
    cos = np.concatenate([np.ones((1, head_dim // 2), F32), np.cos(ang)])
    sin = np.concatenate([np.zeros((1, head_dim // 2), F32), np.sin(ang)])
    assert cos.dtype == F32 and sin.dtype == F32
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


@dataclass(frozen=True)
class Eva02Config:
    """EVA02-L/14 at 448 px by default: 1 cls + 32x32 patch tokens, d 1024, 16 heads of 64, 24 blocks, SwiGLU hidden
    2730 (padded to 2816 = 22 x 128 for the block-128 rotation), LayerNorm eps 1e-6, 30877 tags."""

    img_size: int = 448
    patch: int = 14
    dim: int = 1024
    heads: int = 16
    depth: int = 24
    hidden: int = 2730
    hidden_pad: int = 2816
    tags: int = 30877
    rope_ref: int = 16
    eps: float = 1e-6

    @property
    def grid(self) -> int:
        return self.img_size // self.patch

    @property
    def tokens(self) -> int:
        return 1 + self.grid * self.grid

    def gemm_ops_per_image(self) -> dict[str, int]:
        """2*M*N*K per image with the unpadded model dims (the algorithmic work)."""
        L, d, h = self.tokens, self.dim, self.hidden
        per = {"qkv": 2 * L * 3 * d * d, "proj": 2 * L * d * d, "fc1": 2 * L * 2 * h * d, "fc2": 2 * L * d * h}
        return {k: v * self.depth for k, v in per.items()}

    def attention_flops_per_image(self) -> int:
        return 4 * self.heads * self.tokens * self.tokens * 64 * self.depth


EVA02_L = Eva02Config()


@dataclass
class FloatWeights:
    cfg: Eva02Config
    patch_w: np.ndarray  # [dim, patch*patch*3] in (kh, kw, c) order
    patch_b: np.ndarray
    cls: np.ndarray
    pos: np.ndarray  # [tokens, dim]
    blocks: list[dict[str, np.ndarray]] = field(default_factory=list)
    norm_w: np.ndarray | None = None
    norm_b: np.ndarray | None = None
    head_w: np.ndarray | None = None
    head_b: np.ndarray | None = None


def synthetic_weights(cfg: Eva02Config, seed: int = 0, head_std: float = 0.05) -> FloatWeights:
    """Random-init float32 weights: linears N(0, 0.02), LayerNorm gamma 1 + N(0, 0.02) and beta N(0, 0.02), k bias 0
    (EVA02, foidfinder/haruka.py:55-57). fc1 rows are gate rows then value rows (foidfinder/haruka.py:59-60)."""
    rng = np.random.default_rng(seed)

    def n(*shape, std=0.02):
        return (rng.standard_normal(shape, dtype=F32) * F32(std)).astype(F32)

    d, hd = cfg.dim, cfg.hidden
    w = FloatWeights(
        cfg=cfg,
        patch_w=n(d, cfg.patch * cfg.patch * 3),
        patch_b=n(d),
        cls=n(d),
        pos=n(cfg.tokens, d),
    )
    for _ in range(cfg.depth):
        qkv_b = n(3 * d)
        qkv_b[d : 2 * d] = 0.0
        w.blocks.append(
            {
                "norm1_w": (1.0 + n(d)).astype(F32),
                "norm1_b": n(d),
                "qkv_w": n(3 * d, d),
                "qkv_b": qkv_b,
                "proj_w": n(d, d),
                "proj_b": n(d),
                "norm2_w": (1.0 + n(d)).astype(F32),
                "norm2_b": n(d),
                "fc1_w": n(2 * hd, d),
                "fc1_b": n(2 * hd),
                "mlp_norm_w": (1.0 + n(hd)).astype(F32),
                "mlp_norm_b": n(hd),
                "fc2_w": n(d, hd),
                "fc2_b": n(d),
            }
        )
    w.norm_w = (1.0 + n(d)).astype(F32)
    w.norm_b = n(d)
    w.head_w = n(cfg.tags, d, std=head_std)
    w.head_b = n(cfg.tags)
    return w


def interleave_swiglu(fc1_w: np.ndarray, fc1_b: np.ndarray, hidden: int, hidden_pad: int):
    """Gate-first fc1 [2h, K] -> rows (gate j, value j) interleaved and zero-padded to 2*hidden_pad, so one GEMM
    tile holds both operands of each SwiGLU output."""
    k = fc1_w.shape[1]
    w = np.zeros((2 * hidden_pad, k), F32)
    b = np.zeros(2 * hidden_pad, F32)
    w[0 : 2 * hidden : 2] = fc1_w[:hidden]
    w[1 : 2 * hidden : 2] = fc1_w[hidden:]
    b[0 : 2 * hidden : 2] = fc1_b[:hidden]
    b[1 : 2 * hidden : 2] = fc1_b[hidden:]
    return w, b


def convert_block(blk: dict[str, np.ndarray], cfg: Eva02Config) -> dict[str, np.ndarray]:
    """Float block -> int8 engine block: qweight int8 [N, K] (rotated), wscale fp32 [N], bias fp32 [N], norms fp32.

    qkv/proj/fc1 carry H1024 on K; fc2 is zero-padded to K = hidden_pad and carries blockdiag(H128)."""
    out = {}
    for name, src, block in (("qkv", "qkv", cfg.dim), ("proj", "proj", cfg.dim)):
        out[name + ".qweight"], out[name + ".wscale"] = rotate_quantize(blk[src + "_w"], block)
        out[name + ".bias"] = blk[src + "_b"].astype(F32)
    fw, fb = interleave_swiglu(blk["fc1_w"], blk["fc1_b"], cfg.hidden, cfg.hidden_pad)
    out["fc1.qweight"], out["fc1.wscale"] = rotate_quantize(fw, cfg.dim)
    out["fc1.bias"] = fb
    w2 = np.zeros((cfg.dim, cfg.hidden_pad), F32)
    w2[:, : cfg.hidden] = blk["fc2_w"]
    out["fc2.qweight"], out["fc2.wscale"] = rotate_quantize(w2, 128)
    out["fc2.bias"] = blk["fc2_b"].astype(F32)
    for k in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "mlp_norm_w", "mlp_norm_b"):
        out[k] = blk[k].astype(F32)
    return out


def patchify(images: np.ndarray, patch: int) -> np.ndarray:
    """[B, S, S, 3] -> [B, (S/p)^2, p*p*3] patches in (kh, kw, c) order, row-major over the grid."""
    B, S, _, _ = images.shape
    g = S // patch
    x = images.reshape(B, g, patch, g, patch, 3).transpose(0, 1, 3, 2, 4, 5)
    return x.reshape(B, g * g, patch * patch * 3)


def stem(images: np.ndarray, w: FloatWeights) -> np.ndarray:
    """Patch embedding (conv 14x14 stride 14 as a GEMM) + bias, cls token, + pos -> fp16 residual stream [B*L, d]."""
    cfg = w.cfg
    B = images.shape[0]
    p = patchify(images.astype(F32), cfg.patch)
    x = np.empty((B, cfg.tokens, cfg.dim), F32)
    x[:, 0] = w.cls + w.pos[0]
    x[:, 1:] = (p.astype(np.float64) @ w.patch_w.T.astype(np.float64)).astype(F32) + w.patch_b + w.pos[1:]
    return x.reshape(B * cfg.tokens, cfg.dim).astype(np.float16)


def layer_norm(x: np.ndarray, g: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def head_logits(x: np.ndarray, w: FloatWeights) -> np.ndarray:
    """Final LayerNorm on the cls token and the tag head GEMM, float64 -> logits [B, tags]."""
    cfg = w.cfg
    cls = x.reshape(-1, cfg.tokens, cfg.dim)[:, 0]
    h = layer_norm(cls, w.norm_w, w.norm_b, cfg.eps)
    return h @ w.head_w.T.astype(np.float64) + w.head_b


def head(x: np.ndarray, w: FloatWeights) -> np.ndarray:
    """head_logits then the sigmoid -> float32 probabilities [B, tags]."""
    return (1.0 / (1.0 + np.exp(-head_logits(x, w)))).astype(F32)


def block_int8(
    x: np.ndarray,
    qb: dict[str, np.ndarray],
    cfg: Eva02Config,
    rope: tuple[np.ndarray, np.ndarray],
    *,
    attention_out: np.ndarray | None = None,
    hidden_out: np.ndarray | None = None,
    record: dict | None = None,
):
    """One int8 block on the fp16 residual stream x [B*L, d] -> new x.

    attention_out and hidden_out, if given, replace the attention output and the SwiGLU output (teacher forcing at
    the two floating-point ops whose GPU results are not bit-reproducible: every other op is then a pure function of
    its inputs, so a kernel implementation must reproduce the block bit for bit); record collects qkv, o and h."""
    cos, sin = rope
    a8, rs = rotq8.rot_q8_1024(x, qb["norm1_w"], qb["norm1_b"], cfg.eps)
    qkv = G.gemm_s8(
        a8, qb["qkv.qweight"], rs, qb["qkv.wscale"], qb["qkv.bias"], G.EPI_QKV_ROPE,
        rope_cos=cos, rope_sin=sin, q_scale=Q_SCALE,
    )
    o = attn_mod.attention(qkv, cfg.tokens) if attention_out is None else attention_out
    if record is not None:
        record["qkv"], record["o"] = qkv, o
    a8, rs = rotq8.rot_q8_1024(o)
    x = G.gemm_s8(a8, qb["proj.qweight"], rs, qb["proj.wscale"], qb["proj.bias"], G.EPI_RESIDUAL, residual=x)
    a8, rs = rotq8.rot_q8_1024(x, qb["norm2_w"], qb["norm2_b"], cfg.eps)
    h = G.gemm_s8(a8, qb["fc1.qweight"], rs, qb["fc1.wscale"], qb["fc1.bias"], G.EPI_SWIGLU)
    if record is not None:
        record["h"] = h
    if hidden_out is not None:
        h = hidden_out
    h8, rs = rotq8.rot_q8_h128(h, cfg.hidden, qb["mlp_norm_w"], qb["mlp_norm_b"], cfg.eps)
    return G.gemm_s8(h8, qb["fc2.qweight"], rs, qb["fc2.wscale"], qb["fc2.bias"], G.EPI_RESIDUAL, residual=x)


def forward_int8_x(images: np.ndarray, w: FloatWeights, qblocks: list[dict[str, np.ndarray]]) -> np.ndarray:
    """images [B, S, S, 3] -> the fp16 residual stream [B*L, d] after the last block, with the int8 engine's
    semantics."""
    cfg = w.cfg
    rope = eva02_rope_tables(cfg.grid, cfg.rope_ref)
    x = stem(images, w)
    for qb in qblocks:
        x = block_int8(x, qb, cfg, rope)
    return x


def forward_int8(images: np.ndarray, w: FloatWeights, qblocks: list[dict[str, np.ndarray]]) -> np.ndarray:
    """images [B, S, S, 3] -> probabilities [B, tags] with the int8 engine's semantics."""
    return head(forward_int8_x(images, w, qblocks), w)


def forward_float(images: np.ndarray, w: FloatWeights) -> np.ndarray:
    """The same model without quantization, float64 throughout (the float reference the int8 path approximates)."""
    return head(forward_float_x(images, w), w)


def forward_float_x(images: np.ndarray, w: FloatWeights) -> np.ndarray:
    """forward_float's residual stream [B*L, d] after the last block, float64."""
    cfg = w.cfg
    cos, sin = eva02_rope_tables(cfg.grid, cfg.rope_ref)
    B, L, d, H = images.shape[0], cfg.tokens, cfg.dim, cfg.heads
    x = stem(images, w).astype(np.float64)
    for blk in w.blocks:
        h = layer_norm(x, blk["norm1_w"], blk["norm1_b"], cfg.eps)
        qkv = h @ blk["qkv_w"].T.astype(np.float64) + blk["qkv_b"]
        qk = qkv[:, : 2 * d].reshape(B * L, 2 * H, 32, 2)
        c = np.tile(cos, (B, 1))[:, None, :]
        s = np.tile(sin, (B, 1))[:, None, :]
        r0 = qk[..., 0] * c - qk[..., 1] * s
        r1 = qk[..., 0] * s + qk[..., 1] * c
        qk = np.stack([r0, r1], -1).reshape(B * L, 2 * d)
        qk[:, :d] *= 0.125
        q = qk[:, :d].reshape(B, L, H, 64).transpose(0, 2, 1, 3)
        k = qk[:, d:].reshape(B, L, H, 64).transpose(0, 2, 1, 3)
        v = qkv[:, 2 * d :].reshape(B, L, H, 64).transpose(0, 2, 1, 3)
        sc = q @ k.transpose(0, 1, 3, 2)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        o = (p / p.sum(-1, keepdims=True)) @ v
        o = o.transpose(0, 2, 1, 3).reshape(B * L, d)
        x = x + o @ blk["proj_w"].T.astype(np.float64) + blk["proj_b"]
        h = layer_norm(x, blk["norm2_w"], blk["norm2_b"], cfg.eps)
        gx = h @ blk["fc1_w"].T.astype(np.float64) + blk["fc1_b"]
        g, val = gx[:, : cfg.hidden], gx[:, cfg.hidden :]
        h = layer_norm(g / (1.0 + np.exp(-g)) * val, blk["mlp_norm_w"], blk["mlp_norm_b"], cfg.eps)
        x = x + h @ blk["fc2_w"].T.astype(np.float64) + blk["fc2_b"]
    return x


def synthetic_images(batch: int, size: int, seed: int = 1) -> np.ndarray:
    """[B, S, S, 3] fp16 uniform in [-1, 1] (NHWC, the engine's input layout)."""
    rng = np.random.default_rng(seed)
    return rng.uniform(-1.0, 1.0, (batch, size, size, 3)).astype(np.float16)


def w8a8_linear_inputs(m: int = 1025, k: int = 1024, n: int = 3072, seed: int = 0, outliers: float = 0.01):
    """The single W8A8 linear of the plumbing config: x fp16 [m, k] ~ N(0, 1) with 1% of channels x20,
    W [n, k] ~ N(0, 0.02) rotated by H_k and quantized per row (scales rounded to fp16, held as fp32),
    bias ~ N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=F32)
    cols = rng.choice(k, max(1, int(round(k * outliers))), replace=False)
    x[:, cols] *= F32(20.0)
    w = rng.standard_normal((n, k), dtype=F32) * F32(0.02)
    qw, ws = rotate_quantize(w, k)
    ws = ws.astype(np.float16).astype(F32)
    bias = rng.standard_normal(n, dtype=F32) * F32(0.02)
    return x.astype(np.float16), qw, ws, bias.astype(F32)


def blocks_from_state(state: dict[str, np.ndarray], depth: int) -> list[dict[str, np.ndarray]]:
    """Engine-format state dict (keys `blocks.{i}.attn.qkv.qweight`, ...) -> the per-block dicts block_int8 takes."""
    names = {"qkv": "attn.qkv", "proj": "attn.proj", "fc1": "mlp.fc1", "fc2": "mlp.fc2"}
    out = []
    for i in range(depth):
        p = f"blocks.{i}."
        qb = {}
        for short, long in names.items():
            for f in ("qweight", "wscale", "bias"):
                qb[f"{short}.{f}"] = state[p + long + "." + f]
        for short, long in (("norm1", "norm1"), ("norm2", "norm2"), ("mlp_norm", "mlp.norm")):
            qb[short + "_w"] = state[p + long + ".weight"].astype(F32)
            qb[short + "_b"] = state[p + long + ".bias"].astype(F32)
        out.append(qb)
    return out


def float_weights_from_state(state: dict[str, np.ndarray], cfg: Eva02Config) -> FloatWeights:
    """The non-block tensors of an engine-format state dict as FloatWeights (stem and head)."""
    w = FloatWeights(
        cfg=cfg,
        patch_w=state["patch_embed.weight"].astype(F32),
        patch_b=state["patch_embed.bias"].astype(F32),
        cls=state["cls_token"].astype(F32).reshape(cfg.dim),
        pos=state["pos_embed"].astype(F32).reshape(cfg.tokens, cfg.dim),
    )
    w.norm_w, w.norm_b = state["norm.weight"].astype(F32), state["norm.bias"].astype(F32)
    w.head_w, w.head_b = state["head.weight"].astype(F32), state["head.bias"].astype(F32)
    return w


def forward_int8_state(images: np.ndarray, state: dict[str, np.ndarray], cfg: Eva02Config) -> np.ndarray:
    """forward_int8 driven by an engine-format state dict."""
    return forward_int8(images, float_weights_from_state(state, cfg), blocks_from_state(state, cfg.depth))
