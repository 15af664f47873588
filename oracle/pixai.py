"""PixAI Tagger v1.0 in numpy: window layout, axial RoPE, the int8-semantics forward and the float forward.

Test infrastructure (like every module of this package): only the tests, the smoke check and the benchmark's CPU
baseline use it, as the checker of the GPU engine, never as a path of the product.

Model (foidfinder/backends/cuda/reference.py:11-140): the token grid is kept in window order; blocks in
`global_blocks` attend over the whole grid with the grid RoPE, the others over each window with the window RoPE;
GELU MLP; attention-pool head. Int8 block dataflow (foidfinder/backends/cuda/engine.py:150-160):

  a8, rs = rot_q8_1024(x, norm1)   qkv = gemm(a8, Wqkv, QKV_ROPE)      o = attention(qkv, window or grid)
  a8, rs = rot_q8_1024(o)          x = gemm(a8, Wproj, RESIDUAL, x)
  a8, rs = rot_q8_1024(x, norm2)   h = gemm(a8, Wfc1, GELU)             [M, hidden]
  h8, rs = rot_q8_h128(h)          x = gemm(h8, Wfc2, RESIDUAL, x)
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import attention as attn_mod
from . import gemm as G
from . import rotq8
from .model import Q_SCALE, layer_norm, rotate_quantize

F32 = np.float32
QUANTIZED = {"attn.qkv": 1024, "attn.proj": 1024, "mlp.fc1": 1024, "mlp.fc2": 128}  # engine.py:45


@dataclass(frozen=True)
class PixAIConfig:
    img_size: int = 1008
    patch: int = 14
    dim: int = 1024
    heads: int = 16
    depth: int = 32
    win: int = 24
    pretrain_grid: int = 24
    global_blocks: tuple[int, ...] = (7, 15, 23, 31)
    hidden: int = 4736
    tags: int = 30877
    eps: float = 1e-5

    @property
    def grid(self) -> int:
        return self.img_size // self.patch

    @property
    def windows(self) -> int:
        return self.grid // self.win

    @property
    def tokens(self) -> int:
        return self.grid * self.grid

    @property
    def win_tokens(self) -> int:
        return self.win * self.win


def window_perm(cfg: PixAIConfig) -> np.ndarray:
    """perm[p] = row-major grid index of window-order position p (reference.py:21-24), by explicit loops."""
    g, w, nw = cfg.grid, cfg.win, cfg.windows
    out = []
    for wr in range(nw):
        for wc in range(nw):
            for r in range(w):
                for c in range(w):
                    out.append((wr * w + r) * g + wc * w + c)
    return np.array(out, np.int64)


def axial_rope64(end: int, scale: float, head_dim: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """The axial RoPE angles of reference.py:27-34 evaluated in float64: for grid position t (row-major over end x
    end), pair i < head_dim/4 rotates by (t mod end) * scale * f_i, pair head_dim/4 + i by floor(t / end) * scale *
    f_i, with f_i = 10000^(-4i/head_dim). The engine's fp32 tables must lie within a few fp32 ulps of these."""
    q = head_dim // 4
    f = 10000.0 ** (-(4.0 * np.arange(q)) / head_dim)
    t = np.arange(end * end)
    ang = np.concatenate([np.outer((t % end) * scale, f), np.outer((t // end) * scale, f)], axis=1)
    return np.cos(ang), np.sin(ang)


def convert_checkpoint(raw: dict[str, np.ndarray], cfg: PixAIConfig) -> dict[str, np.ndarray]:
    """Float state dict -> int8 engine format (engine.py:49-62), rotation product in float64."""
    out = {k: v for k, v in raw.items() if not any(f".{n}." in k for n in QUANTIZED)}
    for i in range(cfg.depth):
        for name, n in QUANTIZED.items():
            p = f"blocks.{i}.{name}"
            out[p + ".qweight"], out[p + ".wscale"] = rotate_quantize(raw[p + ".weight"].astype(F32), n)
            out[p + ".bias"] = raw[p + ".bias"].astype(F32)
    return out


def patchify(images: np.ndarray, cfg: PixAIConfig) -> np.ndarray:
    """[B, S, S, 3] -> [B, tokens, p*p*3] in window order: token p of image b is the patch at grid index
    window_perm[p], flattened in (kh, kw, c) order."""
    B, p, g = images.shape[0], cfg.patch, cfg.grid
    grid = images.reshape(B, g, p, g, p, 3).transpose(0, 1, 3, 2, 4, 5).reshape(B, g * g, p * p * 3)
    return grid[:, window_perm(cfg)]


def stem(images: np.ndarray, state: dict[str, np.ndarray], cfg: PixAIConfig) -> np.ndarray:
    """Patch GEMM (no bias), + tiled pretraining positions, ln_pre -> fp16 residual stream [B*tokens, d]
    (reference.py:70-73, :114-116), in float64."""
    d, pre, g = cfg.dim, cfg.pretrain_grid, cfg.grid
    B = images.shape[0]
    w = state["patch_embed.proj.weight"].astype(np.float64).transpose(0, 2, 3, 1).reshape(d, -1)
    x = patchify(images.astype(F32), cfg).astype(np.float64) @ w.T
    pos = state["pos_embed"][0, 1:].astype(np.float64).reshape(pre, pre, d)
    pos = np.tile(pos, (g // pre, g // pre, 1)).reshape(g * g, d)[window_perm(cfg)]
    x = x + pos[None]
    x = layer_norm(x, state["ln_pre.weight"].astype(np.float64), state["ln_pre.bias"].astype(np.float64), cfg.eps)
    return x.reshape(B * cfg.tokens, d).astype(np.float16)


def pool_head(x: np.ndarray, state: dict[str, np.ndarray], cfg: PixAIConfig) -> np.ndarray:
    """Attention pool (one learned query per head over all tokens) + projection + classifier -> float64 logits
    [B, tags] (reference.py:133-140)."""
    d, H, L = cfg.dim, cfg.heads, cfg.tokens
    s = {k: v.astype(np.float64) for k, v in state.items() if k.startswith("head")}
    x = x.astype(np.float64).reshape(-1, L, d)
    B = x.shape[0]
    h = layer_norm(x, s["head_pool.norm.weight"], s["head_pool.norm.bias"], cfg.eps)
    h = h + s["head_pool.pos_embed"].reshape(L, d)[window_perm(cfg)][None]
    kv = h @ s["head_pool.kv.weight"].T + s["head_pool.kv.bias"]
    k, v = kv[..., :d].reshape(B, L, H, 64), kv[..., d:].reshape(B, L, H, 64)
    q = s["head_pool.q"].reshape(H, 64)
    sc = np.einsum("hd,blhd->bhl", q, k) / 8.0
    sc = np.exp(sc - sc.max(-1, keepdims=True))
    p = sc / sc.sum(-1, keepdims=True)
    o = np.einsum("bhl,blhd->bhd", p, v).reshape(B, d)
    o = o @ s["head_pool.proj.weight"].T + s["head_pool.proj.bias"]
    return o @ s["head.weight"].T + s["head.bias"]


def block_int8(
    x: np.ndarray,
    state: dict[str, np.ndarray],
    i: int,
    cfg: PixAIConfig,
    rope: tuple[np.ndarray, np.ndarray],
    seq: int,
    *,
    attention_out: np.ndarray | None = None,
    hidden_out: np.ndarray | None = None,
    record: dict | None = None,
) -> np.ndarray:
    """Block i of the int8 engine on the fp16 residual stream x [B*tokens, d]; `rope` is the table of this block's
    attention span (window or grid) and `seq` that span in tokens. attention_out / hidden_out replace the attention
    and GELU outputs (teacher forcing at the two ops that are not bit-reproducible on the CPU); record collects
    qkv, o and h."""
    p = f"blocks.{i}."

    def lin(n):
        return state[p + n + ".qweight"], state[p + n + ".wscale"].astype(F32), state[p + n + ".bias"].astype(F32)

    def norm(n):
        return state[p + n + ".weight"].astype(F32), state[p + n + ".bias"].astype(F32)

    cos, sin = rope
    a8, rs = rotq8.rot_q8_1024(x, *norm("norm1"), cfg.eps)
    w, ws, b = lin("attn.qkv")
    qkv = G.gemm_s8(a8, w, rs, ws, b, G.EPI_QKV_ROPE, rope_cos=cos, rope_sin=sin, q_scale=Q_SCALE)
    o = attn_mod.attention(qkv, seq) if attention_out is None else attention_out
    if record is not None:
        record["qkv"], record["o"] = qkv, o
    a8, rs = rotq8.rot_q8_1024(o)
    w, ws, b = lin("attn.proj")
    x = G.gemm_s8(a8, w, rs, ws, b, G.EPI_RESIDUAL, residual=x)
    a8, rs = rotq8.rot_q8_1024(x, *norm("norm2"), cfg.eps)
    w, ws, b = lin("mlp.fc1")
    h = G.gemm_s8(a8, w, rs, ws, b, G.EPI_GELU_F16)
    if record is not None:
        record["h"] = h
    if hidden_out is not None:
        h = hidden_out
    h8, rs = rotq8.rot_q8_h128(h)
    w, ws, b = lin("mlp.fc2")
    return G.gemm_s8(h8, w, rs, ws, b, G.EPI_RESIDUAL, residual=x)


def ropes(cfg: PixAIConfig) -> dict[str, tuple[np.ndarray, np.ndarray]]:
    """fp32 tables: window (scale 1) and grid (scale win/grid, in window order)."""
    cw, sw = axial_rope64(cfg.win, 1.0)
    cg, sg = axial_rope64(cfg.grid, cfg.win / cfg.grid)
    perm = window_perm(cfg)
    return {"win": (cw.astype(F32), sw.astype(F32)), "glob": (cg[perm].astype(F32), sg[perm].astype(F32))}


def forward_int8(images: np.ndarray, state: dict[str, np.ndarray], cfg: PixAIConfig,
                 rope: dict[str, tuple[np.ndarray, np.ndarray]] | None = None) -> np.ndarray:
    """images [B, S, S, 3] -> probabilities [B, tags] with the int8 engine's semantics (converted state)."""
    rope = ropes(cfg) if rope is None else rope
    x = stem(images, state, cfg)
    for i in range(cfg.depth):
        glob = i in cfg.global_blocks
        x = block_int8(x, state, i, cfg, rope["glob" if glob else "win"], cfg.tokens if glob else cfg.win_tokens)
    return 1.0 / (1.0 + np.exp(-pool_head(x, state, cfg)))


def forward_float(images: np.ndarray, raw: dict[str, np.ndarray], cfg: PixAIConfig) -> np.ndarray:
    """The unquantized model in float64 (reference.py:109-131, exact erf GELU) -> probabilities [B, tags]."""
    from math import sqrt

    from scipy.special import erf

    d, H = cfg.dim, cfg.heads
    B, L = images.shape[0], cfg.tokens
    rope = {k: (c.astype(np.float64), s.astype(np.float64)) for k, (c, s) in ropes(cfg).items()}
    x = stem(images, raw, cfg).astype(np.float64)
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        s = {k[len(p):]: v.astype(np.float64) for k, v in raw.items() if k.startswith(p)}
        glob = i in cfg.global_blocks
        n = L if glob else cfg.win_tokens
        cos, sin = rope["glob" if glob else "win"]
        h = layer_norm(x, s["norm1.weight"], s["norm1.bias"], cfg.eps)
        qkv = (h @ s["attn.qkv.weight"].T + s["attn.qkv.bias"]).reshape(-1, n, 3, H, 32, 2)
        c, sn = cos[None, :, None, :], sin[None, :, None, :]
        for j in (0, 1):  # rotate q and k
            t = qkv[:, :, j]
            r0 = t[..., 0] * c - t[..., 1] * sn
            r1 = t[..., 0] * sn + t[..., 1] * c
            qkv[:, :, j] = np.stack([r0, r1], -1)
        q, k, v = (qkv[:, :, j].reshape(-1, n, H, 64) for j in range(3))
        sc = np.einsum("snhd,smhd->shnm", q, k) / 8.0
        sc = np.exp(sc - sc.max(-1, keepdims=True))
        o = np.einsum("shnm,smhd->snhd", sc / sc.sum(-1, keepdims=True), v).reshape(B * L, d)
        x = x + o @ s["attn.proj.weight"].T + s["attn.proj.bias"]
        h = layer_norm(x, s["norm2.weight"], s["norm2.bias"], cfg.eps)
        h = h @ s["mlp.fc1.weight"].T + s["mlp.fc1.bias"]
        h = 0.5 * h * (1.0 + erf(h / sqrt(2.0)))
        x = x + h @ s["mlp.fc2.weight"].T + s["mlp.fc2.bias"]
    return 1.0 / (1.0 + np.exp(-pool_head(x, raw, cfg)))
