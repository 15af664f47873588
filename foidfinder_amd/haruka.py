"""Haruka Tagger (EVA02-B/14 at 448 px + slot-sigmoid tree pool) on the gfx950 int8 engine.

The model the reference serves on Apple GPUs only (foidfinder/backends/mlx/haruka.py:36-136; its CUDA backend refuses
Haruka directories, foidfinder/backends/cuda/__init__.py:19-20). Here the backbone runs on the same kernels as the
EVA02-L engine, with every activation row (768 or 2048 wide) rotated by block-diagonal 128-point Hadamards:

  LN1 -> block-H128 rotation -> int8 (per-token scale) -> QKV GEMM + bias + RoPE, q x log2(e) -> fp16
  flash attention (12 heads of 64)                      -> fp16
  block-H128 rotation -> int8                           -> proj GEMM + bias + residual (fp16 stream)
  LN2 -> block-H128 rotation -> int8                    -> fc1 GEMM + bias + SwiGLU -> fp16 [T, 2048]
  mlp LayerNorm -> block-H128 rotation -> int8          -> fc2 GEMM + bias + residual

Input checkpoints are the reference's folded Haruka format (foidfinder/haruka.py:33-89: ImageNet normalization
in the patch embedding, 1/sqrt(head_dim) in the q rows and the pool's key rows, QKV and SwiGLU as single matrices)
or its compressed download format (foidfinder/haruka_quant.py: per-row step x integer codes in gzipped zigzag byte
planes). The folded q rows already carry the softmax scale, so the QKV epilogue multiplies q by log2(e) only.
Stem (patch GEMM on raw 0..255 pixels) and the tree-pool head run in fp16 through PyTorch, as the reference runs
them through MLX.
"""

from __future__ import annotations

import gzip
import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

from .engine import Int8Engine, eva02_rope_tables, rotate_quantize
from .kernels import EPI_QKV_ROPE, EPI_RESIDUAL, EPI_SWIGLU, kernels, pad_norm, slot_weights_blocks

ARCHITECTURE = "haruka-eva02-tree"  # foidfinder/haruka.py:14
QUANTIZED = ("qkv", "proj", "fc1", "fc2")  # the backbone linears that run as W8A8
COMPRESSED_FORMAT = "foidfinder-haruka-rowstep1"  # foidfinder/haruka_quant.py:29


@dataclass(frozen=True)
class HarukaConfig:
    """Haruka Tagger by default (foidfinder/haruka.py:13-27): 448 px, patch 14 (1 cls + 32x32 tokens), d 768, 12
    heads of 64, 12 blocks, SwiGLU hidden 2048 with its LayerNorm, tree pool of 16 heads with 6 coarse and 18 leaf
    queries, 64 features per leaf, RoPE positions on a 16-cell pretraining grid, LayerNorm eps 1e-6."""

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

    def validate(self) -> None:
        if self.dim % 128 or self.heads * 64 != self.dim:
            raise ValueError("the int8 engine needs heads of 64 and dim a multiple of 128 (block-128 rotation)")
        if self.hidden % 128:
            raise ValueError("hidden must be a multiple of 128")
        if self.leaves % self.coarse or self.dim % self.pool_heads:
            raise ValueError("leaves must be a multiple of coarse and dim a multiple of pool_heads")
        if self.img_size % self.patch:
            raise ValueError("img_size must be a multiple of patch")

    @classmethod
    def from_model(cls, model: dict, tags: int, **overrides) -> HarukaConfig:
        """From config.json's "model" entry (foidfinder/haruka.py:13-27 key names)."""
        keys = {"img_size": "img_size", "patch_size": "patch", "dim": "dim", "heads": "heads", "depth": "depth",
                "mlp_hidden": "hidden", "pool_heads": "pool_heads", "coarse_queries": "coarse",
                "leaf_queries": "leaves", "leaf_dim": "leaf_dim", "rope_ref_grid": "rope_ref"}
        fields = {dst: model[src] for src, dst in keys.items() if src in model}
        return cls(tags=tags, **{**fields, **overrides})

    def gemm_ops(self, batch: int) -> dict[str, int]:
        """Algorithmic int8 work per forward: 2*M*N*K summed over blocks."""
        M, d, h = batch * self.tokens, self.dim, self.hidden
        per = {"qkv": 2 * M * 3 * d * d, "proj": 2 * M * d * d, "fc1": 2 * M * 2 * h * d, "fc2": 2 * M * d * h}
        return {k: v * self.depth for k, v in per.items()}

    def attention_flops(self, batch: int) -> int:
        return 4 * batch * self.heads * self.tokens * self.tokens * 64 * self.depth


def decode_planes(planes: list[bytes], shape: tuple[int, int]) -> np.ndarray:
    """Gzipped byte planes of zigzag-coded integers (byte i of every code in plane i, row-major) -> int32 codes
    (the format of foidfinder/haruka_quant.py:1-15, :75-86)."""
    z = np.zeros(shape[0] * shape[1], np.uint32)
    for i, p in enumerate(planes):
        z |= np.frombuffer(gzip.decompress(p), np.uint8).astype(np.uint32) << np.uint32(8 * i)
    return ((z >> np.uint32(1)).astype(np.int64) * (1 - 2 * (z & 1).astype(np.int64)) - (z & 1)).astype(
        np.int32).reshape(shape)


def load_compressed(model_dir: Path, layers: dict) -> dict[str, torch.Tensor]:
    """All weights of a compressed Haruka checkpoint, each quantized matrix rebuilt as fp32 code x step[row]
    (foidfinder/haruka_quant.py:162-173)."""
    from safetensors.numpy import load_file

    raw = load_file(str(Path(model_dir) / "model.safetensors"))
    out = {k: torch.from_numpy(v.copy()) for k, v in raw.items()
           if not k.rsplit(".", 1)[-1].startswith(("step", "plane"))}
    for k, spec in layers.items():
        planes = [raw[f"{k}.plane{i}"].tobytes() for i in range(spec["planes"])]
        codes = decode_planes(planes, tuple(spec["shape"]))
        out[k] = torch.from_numpy(codes.astype(np.float32) * raw[k + ".step"].astype(np.float32)[:, None])
    return out


def convert_checkpoint(folded: dict[str, torch.Tensor], cfg: HarukaConfig) -> dict[str, torch.Tensor]:
    """Folded Haruka state dict -> engine format. Each backbone linear becomes `<name>.qweight` (int8, rotated by
    W blockdiag(H128)), `<name>.wscale` (fp32 per output channel) and `<name>.bias` (fp32); fc1 (gate rows, then
    value rows, foidfinder/haruka.py:59-60) is interleaved as (gate j, value j) row pairs for the SwiGLU epilogue;
    norms become fp32; every other tensor is copied."""
    h = cfg.hidden
    out = {k: v for k, v in folded.items() if not k.startswith("blocks.")}
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        for name in ("qkv", "proj", "fc2"):
            out[p + name + ".qweight"], out[p + name + ".wscale"] = rotate_quantize(folded[p + name + ".weight"], 128)
            out[p + name + ".bias"] = folded[p + name + ".bias"].float().contiguous()
        w1, b1 = folded[p + "fc1.weight"].float(), folded[p + "fc1.bias"].float()
        wi, bi = torch.empty_like(w1), torch.empty_like(b1)
        wi[0::2], wi[1::2] = w1[:h], w1[h:]
        bi[0::2], bi[1::2] = b1[:h], b1[h:]
        out[p + "fc1.qweight"], out[p + "fc1.wscale"] = rotate_quantize(wi, 128)
        out[p + "fc1.bias"] = bi.contiguous()
        for n in ("norm1", "norm2", "mlp_norm"):
            out[p + n + ".weight"] = folded[p + n + ".weight"].float().contiguous()
            out[p + n + ".bias"] = folded[p + n + ".bias"].float().contiguous()
    return out


def synthetic_checkpoint(cfg: HarukaConfig, seed: int = 0, head_std: float = 0.05) -> dict[str, torch.Tensor]:
    """Random-init Haruka state dict in the folded format (foidfinder/haruka.py:33-89 key names and shapes), from a
    seeded CPU generator: linears N(0, 0.02) with the q rows and the pool's key rows carrying their folded scales,
    patch weights N(0, 0.02) / (255 x 0.226) as if the pixel normalization were folded in, LayerNorm gamma
    1 + N(0, 0.02) and beta N(0, 0.02), pool queries N(0, 1), query biases -2 + N(0, 0.1) (the model card's init
    plus noise)."""
    g = torch.Generator().manual_seed(seed)
    d, h, C, Q, f = cfg.dim, cfg.hidden, cfg.coarse, cfg.leaves, cfg.leaf_dim

    def n(*shape, std=0.02):
        return torch.randn(*shape, generator=g) * std

    def ln(prefix, width):
        return {prefix + ".weight": 1.0 + n(width), prefix + ".bias": n(width)}

    sd = {
        "patch_w": n(d, cfg.patch * cfg.patch * 3) / (255.0 * 0.226),
        "patch_b": n(cfg.grid * cfg.grid, d),
        "cls": n(1, d),
        **ln("norm", d),
        "pool.kv.weight": n(2 * d, d),
        "pool.kv.bias": n(2 * d),
        "pool.q_coarse": n(C, d, std=1.0),
        "pool.q_coarse_bias": -2.0 + n(C, std=0.1),
        "pool.q_child": n(Q, d, std=1.0),
        "pool.q_child_bias": -2.0 + n(Q, std=0.1),
        "pool.leaf.weight": n(Q, d, f),
        "pool.leaf.bias": n(Q, f),
        "head.weight": n(cfg.tags, Q * f, std=head_std),
        "head.bias": n(cfg.tags),
    }
    pool_scale = (d // cfg.pool_heads) ** -0.5
    sd["pool.kv.weight"][:d] *= pool_scale
    sd["pool.kv.bias"][:d] *= pool_scale
    for name in ("norm", "trunk_norm", "child_q_norm", "leaf_norm"):
        sd.update(ln("pool." + name, d))
    scale = 64**-0.5
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        qkv_w, qkv_b = n(3 * d, d), n(3 * d)
        qkv_w[:d] *= scale
        qkv_b[:d] *= scale
        qkv_b[d : 2 * d] = 0
        sd.update({
            p + "qkv.weight": qkv_w, p + "qkv.bias": qkv_b,
            p + "proj.weight": n(d, d), p + "proj.bias": n(d),
            p + "fc1.weight": n(2 * h, d), p + "fc1.bias": n(2 * h),
            p + "fc2.weight": n(d, h), p + "fc2.bias": n(d),
            **ln(p + "norm1", d), **ln(p + "norm2", d), **ln(p + "mlp_norm", h),
        })
    return sd


class HarukaInt8(Int8Engine):
    """images [B, S, S, 3] raw pixels 0..255 (NHWC; any dtype, uint8 from preprocessing) -> logits [B, tags] fp32,
    one HIP graph per batch size (the Int8Engine plan: buffers, GEMM variant autotune, warm-up, capture, replay)."""

    q_scale = math.log2(math.e)  # the folded q rows already carry 1/sqrt(64)

    def __init__(self, state: dict[str, torch.Tensor], cfg: HarukaConfig, *, device: str | torch.device = "cuda"):
        cfg.validate()
        self.cfg = cfg
        self.device = torch.device(device)
        self.k = kernels()
        dev = self.device
        if "blocks.0.qkv.qweight" not in state:
            state = convert_checkpoint({k: v.to(dev) for k, v in state.items()}, cfg)
        t = {k: v.to(dev) for k, v in state.items()}
        d, h = cfg.dim, cfg.hidden

        def lin(p):
            return t[p + ".qweight"].contiguous(), t[p + ".wscale"].float().contiguous(), t[p + ".bias"].float().contiguous()

        def norm(p, width):
            return pad_norm(t[p + ".weight"], t[p + ".bias"], width)

        def half(x):
            return x.half().contiguous()

        # stem (mlx/haruka.py:77-80): patch weights over (kh, kw, c) with the pixel normalization folded in
        self.patch_w_t = half(t["patch_w"].reshape(d, -1).t())
        self.patch_b = half(t["patch_b"].reshape(cfg.grid * cfg.grid, d))
        self.cls = half(t["cls"].reshape(d))
        self.norm = (half(t["norm.weight"]), half(t["norm.bias"]))  # fp16, as the reference's weights
        self.layers = [
            {
                "n1": norm(f"blocks.{i}.norm1", d),
                "n2": norm(f"blocks.{i}.norm2", d),
                "nm": norm(f"blocks.{i}.mlp_norm", h),
                **{name: lin(f"blocks.{i}.{name}") for name in QUANTIZED},
            }
            for i in range(cfg.depth)
        ]
        # tree pool (mlx/haruka.py:104-136)
        self.pool = {name: (half(t[f"pool.{name}.weight"]), half(t[f"pool.{name}.bias"]))
                     for name in ("norm", "trunk_norm", "child_q_norm", "leaf_norm")}
        # Keys and values are never formed: per pool head h, a query's logit against token x is
        # x . (Wk_h^T q) + q . bk_h, and its pooled value is Wv_h (sum_n a_n x_n) + bv_h sum_n a_n. The coarse queries
        # are weights, so their Wk_h^T q columns are precomputed (float64, rounded once).
        Hp, hd, C = cfg.pool_heads, d // cfg.pool_heads, cfg.coarse
        kv_w, kv_b = t["pool.kv.weight"].double(), t["pool.kv.bias"].double()
        wk, bk = kv_w[:d].reshape(Hp, hd, d), kv_b[:d].reshape(Hp, hd)
        qc = t["pool.q_coarse"].double().reshape(C, Hp, hd)
        self.coarse_uT = half(torch.einsum("hed,mhe->dhm", wk, qc).reshape(d, Hp * C))  # column h*C + m
        self.coarse_c = torch.einsum("he,mhe->hm", bk, qc).reshape(Hp * C).float().contiguous()
        self.pool_kT = half(wk.transpose(1, 2))  # [Hp, d, hd]: Wk_h^T
        self.pool_bk = bk.float().contiguous()
        self.pool_vT = half(kv_w[d:].reshape(Hp, hd, d).transpose(1, 2))  # [Hp, d, hd]: Wv_h^T
        self.pool_bv = kv_b[d:].reshape(Hp, hd).float().contiguous()
        self.q_coarse_bias = t["pool.q_coarse_bias"].float().reshape(cfg.coarse).contiguous()
        self.q_child = half(t["pool.q_child"].reshape(cfg.leaves, d))
        self.q_child_bias = t["pool.q_child_bias"].float().reshape(cfg.leaves).contiguous()
        self.leaf_w = half(t["pool.leaf.weight"].reshape(cfg.leaves, d, cfg.leaf_dim))
        self.leaf_b = half(t["pool.leaf.bias"].reshape(cfg.leaves, cfg.leaf_dim))
        self.head = (half(t["head.weight"]), half(t["head.bias"]))
        cos, sin = eva02_rope_tables(cfg.grid, cfg.rope_ref)  # mlx/haruka.py:22-33
        self.rope = (cos.to(dev), sin.to(dev))
        self.variants: dict[tuple[str, int], int] = {}
        self._graphs: dict[int, tuple] = {}

    def _buffers(self, B: int) -> dict[str, torch.Tensor]:
        cfg, dev = self.cfg, self.device
        T, d, h = B * cfg.tokens, cfg.dim, cfg.hidden
        return {
            "x": torch.empty(T, d, device=dev, dtype=torch.half),
            "patch": torch.empty(B * cfg.grid * cfg.grid, d, device=dev, dtype=torch.half),
            "a8": torch.empty(T, d, device=dev, dtype=torch.int8),
            "rs": torch.empty(T, device=dev),
            "qkv": torch.empty(T, 3 * d, device=dev, dtype=torch.half),
            "o16": torch.empty(T, d, device=dev, dtype=torch.half),
            "h16": torch.empty(T, h, device=dev, dtype=torch.half),
            "h8": torch.empty(T, h, device=dev, dtype=torch.int8),
        }

    def _gemm_jobs(self, buf):
        lw = self.layers[0]
        return {
            "qkv": lambda v: self._gemm(buf["a8"], lw["qkv"], buf["rs"], EPI_QKV_ROPE, v, buf["qkv"], self.rope),
            "proj": lambda v: self._gemm(buf["a8"], lw["proj"], buf["rs"], EPI_RESIDUAL, v, buf["o16"]),
            "fc1": lambda v: self._gemm(buf["a8"], lw["fc1"], buf["rs"], EPI_SWIGLU, v, buf["h16"]),
            "fc2": lambda v: self._gemm(buf["h8"], lw["fc2"], buf["rs"], EPI_RESIDUAL, v, buf["o16"]),
        }

    def patchify(self, img: torch.Tensor) -> torch.Tensor:
        """[B, S, S, 3] -> [B * g * g, p*p*3] fp16 patches in (kh, kw, c) order, row-major over the grid (pixel
        values 0..255 are exact in fp16)."""
        cfg = self.cfg
        B, g, p = img.shape[0], cfg.grid, cfg.patch
        x = img.to(torch.half).view(B, g, p, g, p, 3).permute(0, 1, 3, 2, 4, 5)
        return x.reshape(B * g * g, p * p * 3)

    def pool_head(self, x: torch.Tensor) -> torch.Tensor:
        """Final LayerNorm + tree attention pool over the residual stream x [B, N, d] fp16 -> logits [B, tags] fp32
        (mlx/haruka.py:100-136): queries compete per token (softmax over the queries) and each token is also gated
        by sigmoid(logit + bias); 6 coarse queries feed 3 leaf queries each; leaves are weighted by their patch mass.

        Same algebra as the reference with the key/value projection moved onto the queries' side (see __init__):
        logits = xn @ [Wk_h^T q] + q . bk_h, pooled = (w^T xn) Wv_h^T + bv_h sum(w), so the [B, N, 2d] key/value
        tensor is never formed. The two LayerNorms (backbone, then pool) are one kernel (ff_layer_norm2), and the
        weights w (softmax over queries x sigmoid gate), their transpose for the pooling product and their sums over
        the tokens are another (ff_slot_weights)."""
        cfg, k = self.cfg, self.k
        B, N, d = x.shape
        Hp, C, Q = cfg.pool_heads, cfg.coarse, cfg.leaves
        hd = d // Hp

        def ln(t, name):
            w, b = self.pool[name]
            return F.layer_norm(t, (d,), w, b, cfg.eps)

        xn = torch.empty_like(x)
        k.layer_norm2(x, *self.norm, *self.pool["norm"], cfg.eps, xn)
        nblk = slot_weights_blocks(N)

        def attend(logits, c, bias, M):
            """logits fp16 [B, N, Hp*M] (column h*M + m) + c -> (mass [B, Hp, M] fp32, pooled [B, M, d] fp16)."""
            a_t = torch.empty(B, Hp * M, N, device=x.device, dtype=torch.half)
            partial = torch.empty(B, nblk, Hp * M, device=x.device, dtype=torch.float32)
            k.slot_weights(logits, c, bias, Hp, a_t, partial)
            mass = partial.sum(1).view(B, Hp, M)
            pooled = torch.bmm(a_t, xn).view(B, Hp, M, d).transpose(0, 1).reshape(Hp, B * M, d)
            z = torch.bmm(pooled, self.pool_vT).view(Hp, B, M, hd).permute(1, 2, 0, 3).float()
            z = z + mass.permute(0, 2, 1)[..., None] * self.pool_bv
            return mass, z.reshape(B, M, d).half()

        logits = torch.matmul(xn.view(B * N, d), self.coarse_uT).view(B, N, Hp * C)
        _, z = attend(logits, self.coarse_c, self.q_coarse_bias, C)
        z_parent = ln(z, "trunk_norm").repeat_interleave(Q // C, dim=1)  # coarse c feeds leaves c*Q/C ..
        q_leaf = ln(z_parent + self.q_child, "child_q_norm").view(B, Q, Hp, hd)
        qh = q_leaf.permute(2, 3, 0, 1).reshape(Hp, hd, B * Q)
        u_t = torch.bmm(self.pool_kT, qh).view(Hp, d, B, Q).permute(2, 1, 0, 3).reshape(B, d, Hp * Q)
        c_leaf = torch.einsum("he,bqhe->bhq", self.pool_bk, q_leaf.float()).reshape(B, Hp * Q).contiguous()
        mass, z_child = attend(torch.bmm(xn, u_t), c_leaf, self.q_child_bias, Q)
        z_tree = ln(z_parent + z_child, "leaf_norm")
        mass = mass.mean(1)[..., None]  # [B, Q, 1]: patch mass per leaf, averaged over heads
        z_tree = z_tree * (mass / (mass + 4.0)).half()
        leaf = torch.bmm(z_tree.transpose(0, 1).contiguous(), self.leaf_w).transpose(0, 1) + self.leaf_b
        return F.linear(leaf.reshape(B, Q * cfg.leaf_dim), *self.head).float()

    def _forward(self, img: torch.Tensor, buf: dict[str, torch.Tensor], trace: dict | None = None) -> torch.Tensor:
        """One forward into the preallocated buffers; `trace` (eager debugging only) collects the stem output and,
        per block, the qkv, attention output, SwiGLU output and block output."""
        k, cfg = self.k, self.cfg
        B, L, d = img.shape[0], cfg.tokens, cfg.dim
        x, a8, rs = buf["x"], buf["a8"], buf["rs"]
        torch.matmul(self.patchify(img), self.patch_w_t, out=buf["patch"])
        xv = x.view(B, L, d)
        torch.add(buf["patch"].view(B, L - 1, d), self.patch_b, out=xv[:, 1:])
        xv[:, 0] = self.cls
        v = {name: self.variants.get((name, B), 0) for name in QUANTIZED}
        eps = cfg.eps
        if trace is not None:
            trace["stem"] = x.clone()
        for i, lw in enumerate(self.layers):
            k.rot_q8_h128(x, a8, rs, *lw["n1"], d, eps)
            self._gemm(a8, lw["qkv"], rs, EPI_QKV_ROPE, v["qkv"], buf["qkv"], self.rope)
            k.attention(buf["qkv"], buf["o16"], L)
            if trace is not None:
                trace[f"qkv{i}"], trace[f"attn{i}"] = buf["qkv"].clone(), buf["o16"].clone()
            k.rot_q8_h128(buf["o16"], a8, rs)
            self._gemm(a8, lw["proj"], rs, EPI_RESIDUAL, v["proj"], x)
            k.rot_q8_h128(x, a8, rs, *lw["n2"], d, eps)
            self._gemm(a8, lw["fc1"], rs, EPI_SWIGLU, v["fc1"], buf["h16"])
            if trace is not None:
                trace[f"h{i}"] = buf["h16"].clone()
            k.rot_q8_h128(buf["h16"], buf["h8"], rs, *lw["nm"], cfg.hidden, eps)
            self._gemm(buf["h8"], lw["fc2"], rs, EPI_RESIDUAL, v["fc2"], x)
            if trace is not None:
                trace[f"x{i}"] = x.clone()
        return self.pool_head(xv)


def load_haruka_dir(model_dir: str | Path, device: str | torch.device = "cuda", **overrides) -> tuple[HarukaInt8, dict]:
    """A Haruka model directory (config.json with "model", "tags", "categories", "thresholds" and model.safetensors,
    folded or compressed, foidfinder/haruka.py:101-110 and haruka_quant.py:150-160) -> (engine, config)."""
    from safetensors.torch import load_file

    model_dir = Path(model_dir)
    config = json.loads((model_dir / "config.json").read_text())
    model = config.get("model", {})
    if model.get("architecture") != ARCHITECTURE:
        raise RuntimeError(f"{model_dir}: not a Haruka model (architecture {model.get('architecture')!r})")
    quant = config.get("quantization")
    if quant is not None:
        if quant.get("format") != COMPRESSED_FORMAT:
            raise RuntimeError(f"{model_dir}: unknown Haruka weight format {quant.get('format')!r}")
        state = load_compressed(model_dir, quant["layers"])
    else:
        state = load_file(str(model_dir / "model.safetensors"))
    cfg = HarukaConfig.from_model(model, tags=state["head.weight"].shape[0], **overrides)
    return HarukaInt8(state, cfg, device=device), config
