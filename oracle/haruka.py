"""Haruka Tagger (EVA02-B/14 at 448 px + slot-sigmoid tree pool) in numpy: weight conversion, stem, the
int8-semantics forward, the tree-pool head and the float forward.

Test infrastructure (like every module of this package): only the tests, the smoke check and the benchmark's CPU
baseline use it, as the checker of the GPU engine, never as a path of the product.

Model (foidfinder/backends/mlx/haruka.py:74-136 on the folded checkpoint of foidfinder/haruka.py:33-89). Int8 block
dataflow of the engine; every activation row (768 or 2048 wide) is rotated by block-diagonal 128-point Hadamards,
and q's softmax scale is already in the folded weights, so the QKV epilogue multiplies q by log2(e):

  a8, rs = rot_q8_h128(x, norm1)      qkv = gemm(a8, Wqkv, QKV_ROPE)     o = attention(qkv)
  a8, rs = rot_q8_h128(o)             x = gemm(a8, Wproj, RESIDUAL, x)
  a8, rs = rot_q8_h128(x, norm2)      h = gemm(a8, Wfc1, SWIGLU)          [M, hidden]
  h8, rs = rot_q8_h128(h, mlp_norm)   x = gemm(h8, Wfc2, RESIDUAL, x)
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import attention as attn_mod
from . import gemm as G
from . import rotq8
from .model import eva02_rope_tables, layer_norm, patchify, rotate_quantize

F32 = np.float32
Q_SCALE = math.log2(math.e)  # the folded q rows carry 1/sqrt(64); the epilogue adds log2(e) for the base-2 softmax


@dataclass(frozen=True)
class HarukaConfig:
    img_size: int = 448
    patch: int = 14
    dim: int = 768
    heads: int = 12
    depth: int = 12
    hidden: int = 2048
    pool_heads: int = 16
    coarse: int = 6
    leaves: int = 18
    leaf_dim: int = 64
    rope_ref: int = 16
    tags: int = 98782
    eps: float = 1e-6

    @property
    def grid(self) -> int:
        return self.img_size // self.patch

    @property
    def tokens(self) -> int:
        return 1 + self.grid * self.grid


def convert_checkpoint(folded: dict[str, np.ndarray], cfg: HarukaConfig) -> dict[str, np.ndarray]:
    """Folded state dict -> int8 engine format: each backbone linear W -> quantize_rows(W blockdiag(H128)) (product in
    float64); fc1's gate rows j and value rows j interleaved as rows 2j, 2j + 1 (the SwiGLU epilogue's pairs)."""
    h = cfg.hidden
    out = {k: v for k, v in folded.items() if not k.startswith("blocks.")}
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        for name in ("qkv", "proj", "fc2"):
            out[p + name + ".qweight"], out[p + name + ".wscale"] = rotate_quantize(
                folded[p + name + ".weight"].astype(F32), 128)
            out[p + name + ".bias"] = folded[p + name + ".bias"].astype(F32)
        w1, b1 = folded[p + "fc1.weight"].astype(F32), folded[p + "fc1.bias"].astype(F32)
        wi, bi = np.empty_like(w1), np.empty_like(b1)
        for j in range(h):
            wi[2 * j], wi[2 * j + 1] = w1[j], w1[h + j]
            bi[2 * j], bi[2 * j + 1] = b1[j], b1[h + j]
        out[p + "fc1.qweight"], out[p + "fc1.wscale"] = rotate_quantize(wi, 128)
        out[p + "fc1.bias"] = bi
        for n in ("norm1", "norm2", "mlp_norm"):
            out[p + n + ".weight"] = folded[p + n + ".weight"].astype(F32)
            out[p + n + ".bias"] = folded[p + n + ".bias"].astype(F32)
    return out


def stem(images: np.ndarray, state: dict[str, np.ndarray], cfg: HarukaConfig) -> np.ndarray:
    """Raw pixels [B, S, S, 3] -> fp16 residual stream [B*tokens, d]: token 0 is `cls`, token 1 + t is patch t
    (row-major over the grid, (kh, kw, c) order) times patch_w plus patch_b (mlx/haruka.py:77-80), in float64."""
    B, d = images.shape[0], cfg.dim
    w = state["patch_w"].astype(np.float64).reshape(d, -1)
    x = np.empty((B, cfg.tokens, d))
    x[:, 0] = state["cls"].astype(np.float64).reshape(d)
    x[:, 1:] = patchify(images.astype(np.float64), cfg.patch) @ w.T + state["patch_b"].astype(np.float64)
    return x.reshape(B * cfg.tokens, d).astype(np.float16)


def pool_head(xn: np.ndarray, state: dict[str, np.ndarray], cfg: HarukaConfig) -> np.ndarray:
    """Tree attention pool over normalized tokens xn [B, L, d] -> float64 logits [B, tags] (mlx/haruka.py:104-136).

    slot_attend(q, bias): logits = q . k per pool head (the key rows carry 1/sqrt(head_dim)); weights = softmax over
    the QUERIES of each token x sigmoid(logit + bias of the query); pooled = weights @ v. Coarse queries pool first;
    their LayerNormed results, each repeated for its leaves, plus the learned child queries (LayerNormed) query
    again; each leaf is LayerNorm(parent + child) scaled by m / (m + 4), m its weight mass summed over tokens and
    averaged over heads, then projected by its own [d, leaf_dim] matrix; the concatenated leaves feed the head."""
    d, Hp, C, Q, f = cfg.dim, cfg.pool_heads, cfg.coarse, cfg.leaves, cfg.leaf_dim
    hd = d // Hp
    s = {k: v.astype(np.float64) for k, v in state.items() if k.startswith(("pool.", "head."))}
    xn = xn.astype(np.float64)
    B, L, _ = xn.shape

    def ln(t, name):
        return layer_norm(t, s[f"pool.{name}.weight"], s[f"pool.{name}.bias"], cfg.eps)

    kv = ln(xn, "norm") @ s["pool.kv.weight"].T + s["pool.kv.bias"]
    k, v = kv[..., :d].reshape(B, L, Hp, hd), kv[..., d:].reshape(B, L, Hp, hd)

    def attend(q, bias):
        M = q.shape[1]
        logits = np.einsum("bmhe,blhe->bhml", q.reshape(B, M, Hp, hd), k)
        e = np.exp(logits - logits.max(axis=2, keepdims=True))
        attn = e / e.sum(axis=2, keepdims=True) / (1.0 + np.exp(-(logits + bias[None, None, :, None])))
        return attn, np.einsum("bhml,blhe->bmhe", attn, v).reshape(B, M, d)

    _, z = attend(np.broadcast_to(s["pool.q_coarse"].reshape(C, d), (B, C, d)), s["pool.q_coarse_bias"].reshape(C))
    z_parent = np.repeat(ln(z, "trunk_norm"), Q // C, axis=1)
    attn, z_child = attend(ln(z_parent + s["pool.q_child"].reshape(Q, d), "child_q_norm"),
                           s["pool.q_child_bias"].reshape(Q))
    z_tree = ln(z_parent + z_child, "leaf_norm")
    mass = attn.sum(-1).mean(1)[..., None]
    z_tree = z_tree * (mass / (mass + 4.0))
    leaf = np.einsum("bqd,qdf->bqf", z_tree, s["pool.leaf.weight"].reshape(Q, d, f)) + s["pool.leaf.bias"].reshape(Q, f)
    return leaf.reshape(B, Q * f) @ s["head.weight"].T + s["head.bias"]


def head(x: np.ndarray, state: dict[str, np.ndarray], cfg: HarukaConfig) -> np.ndarray:
    """Residual stream [B*L, d] -> final LayerNorm over every token -> tree pool -> float64 logits [B, tags]."""
    xn = layer_norm(x.astype(np.float64).reshape(-1, cfg.tokens, cfg.dim), state["norm.weight"].astype(np.float64),
                    state["norm.bias"].astype(np.float64), cfg.eps)
    return pool_head(xn, state, cfg)


def block_int8(
    x: np.ndarray,
    state: dict[str, np.ndarray],
    i: int,
    cfg: HarukaConfig,
    rope: tuple[np.ndarray, np.ndarray],
    *,
    attention_out: np.ndarray | None = None,
    hidden_out: np.ndarray | None = None,
    record: dict | None = None,
) -> np.ndarray:
    """Block i of the int8 engine on the fp16 residual stream x [B*tokens, d]. attention_out / hidden_out replace
    the attention and SwiGLU outputs (teacher forcing at the two ops that are not bit-reproducible on the CPU);
    record collects qkv, o and h."""
    p = f"blocks.{i}."
    d, eps = cfg.dim, cfg.eps

    def lin(n):
        return state[p + n + ".qweight"], state[p + n + ".wscale"].astype(F32), state[p + n + ".bias"].astype(F32)

    def norm(n):
        return state[p + n + ".weight"].astype(F32), state[p + n + ".bias"].astype(F32)

    cos, sin = rope
    a8, rs = rotq8.rot_q8_h128(x, d, *norm("norm1"), eps)
    w, ws, b = lin("qkv")
    qkv = G.gemm_s8(a8, w, rs, ws, b, G.EPI_QKV_ROPE, rope_cos=cos, rope_sin=sin, q_scale=Q_SCALE)
    o = attn_mod.attention(qkv, cfg.tokens) if attention_out is None else attention_out
    if record is not None:
        record["qkv"], record["o"] = qkv, o
    a8, rs = rotq8.rot_q8_h128(o)
    w, ws, b = lin("proj")
    x = G.gemm_s8(a8, w, rs, ws, b, G.EPI_RESIDUAL, residual=x)
    a8, rs = rotq8.rot_q8_h128(x, d, *norm("norm2"), eps)
    w, ws, b = lin("fc1")
    h = G.gemm_s8(a8, w, rs, ws, b, G.EPI_SWIGLU)
    if record is not None:
        record["h"] = h
    if hidden_out is not None:
        h = hidden_out
    h8, rs = rotq8.rot_q8_h128(h, cfg.hidden, *norm("mlp_norm"), eps)
    w, ws, b = lin("fc2")
    return G.gemm_s8(h8, w, rs, ws, b, G.EPI_RESIDUAL, residual=x)


def forward_int8(images: np.ndarray, state: dict[str, np.ndarray], cfg: HarukaConfig) -> np.ndarray:
    """Raw pixels [B, S, S, 3] -> probabilities [B, tags] with the int8 engine's semantics (converted state)."""
    rope = eva02_rope_tables(cfg.grid, cfg.rope_ref)
    x = stem(images, state, cfg)
    for i in range(cfg.depth):
        x = block_int8(x, state, i, cfg, rope)
    return 1.0 / (1.0 + np.exp(-head(x, state, cfg)))


def forward_float(images: np.ndarray, folded: dict[str, np.ndarray], cfg: HarukaConfig) -> np.ndarray:
    """The unquantized model in float64 on the folded weights (mlx/haruka.py:74-101) -> probabilities [B, tags]."""
    cos, sin = (t.astype(np.float64) for t in eva02_rope_tables(cfg.grid, cfg.rope_ref))
    B, L, d, H, hid = images.shape[0], cfg.tokens, cfg.dim, cfg.heads, cfg.hidden
    x = stem(images, folded, cfg).astype(np.float64)
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        s = {k[len(p):]: v.astype(np.float64) for k, v in folded.items() if k.startswith(p)}
        h = layer_norm(x, s["norm1.weight"], s["norm1.bias"], cfg.eps)
        qkv = h @ s["qkv.weight"].T + s["qkv.bias"]
        qk = qkv[:, : 2 * d].reshape(B, L, 2 * H, 32, 2)
        c, sn = cos[None, :, None], sin[None, :, None]
        qk = np.stack([qk[..., 0] * c - qk[..., 1] * sn, qk[..., 0] * sn + qk[..., 1] * c], -1).reshape(B, L, 2 * d)
        q = qk[..., :d].reshape(B, L, H, 64).transpose(0, 2, 1, 3)
        k = qk[..., d:].reshape(B, L, H, 64).transpose(0, 2, 1, 3)
        v = qkv[:, 2 * d :].reshape(B, L, H, 64).transpose(0, 2, 1, 3)
        sc = q @ k.transpose(0, 1, 3, 2)  # the softmax scale is in the folded q rows
        e = np.exp(sc - sc.max(-1, keepdims=True))
        o = ((e / e.sum(-1, keepdims=True)) @ v).transpose(0, 2, 1, 3).reshape(B * L, d)
        x = x + o @ s["proj.weight"].T + s["proj.bias"]
        h = layer_norm(x, s["norm2.weight"], s["norm2.bias"], cfg.eps)
        gx = h @ s["fc1.weight"].T + s["fc1.bias"]
        g, val = gx[:, :hid], gx[:, hid:]
        h = layer_norm(g / (1.0 + np.exp(-g)) * val, s["mlp_norm.weight"], s["mlp_norm.bias"], cfg.eps)
        x = x + h @ s["fc2.weight"].T + s["fc2.bias"]
    return 1.0 / (1.0 + np.exp(-head(x, folded, cfg)))
