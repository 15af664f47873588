"""PixAI Tagger v1.0 (the reference's served model) on the gfx950 int8 engine.

The model (foidfinder/backends/cuda/reference.py:11-140): 1008 px images, 14 px patches, a 72 x 72 token grid kept
in window order (3 x 3 windows of 24 x 24), 32 ViT-L blocks with a GELU MLP (hidden 4736 = 37 x 128), windowed
attention over 576 tokens in every block except 7, 15, 23 and 31, which attend over all 5184 tokens; axial RoPE per
window (scale 1) or over the whole grid (scale 24/72); an attention-pool head (one learned query per head) and a
linear classifier. The int8 block dataflow is the reference engine's (foidfinder/backends/cuda/engine.py:1-10,
:142-161): the same four kernels as the EVA02 engine, with the GELU epilogue and no MLP LayerNorm. Stem and head run
in fp16 through PyTorch, as the reference's do through cuBLAS.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F

from .engine import Int8Engine, rotate_quantize
from .kernels import EPI_GELU_F16, EPI_QKV_ROPE, EPI_RESIDUAL, kernels

FORMAT = "foidfinder-pixai-int8-v1"  # the reference's converted-checkpoint format name (engine.py:46)
# Quantized block linears -> Hadamard block size of their input rotation (engine.py:45).
QUANTIZED = {"attn.qkv": 1024, "attn.proj": 1024, "mlp.fc1": 1024, "mlp.fc2": 128}


@dataclass(frozen=True)
class PixAIConfig:
    """PixAI Tagger v1.0 by default; smaller grids, windows and depths describe test models of the same structure."""

    img_size: int = 1008
    patch: int = 14
    dim: int = 1024
    heads: int = 16
    depth: int = 32
    win: int = 24  # window side in tokens
    pretrain_grid: int = 24  # the position table's grid (336 / 14), tiled over the full grid
    global_blocks: tuple[int, ...] = (7, 15, 23, 31)
    hidden: int = 4736
    tags: int = 30877
    eps: float = 1e-5

    @property
    def grid(self) -> int:
        return self.img_size // self.patch

    @property
    def windows(self) -> int:  # windows per side
        return self.grid // self.win

    @property
    def tokens(self) -> int:
        return self.grid * self.grid

    @property
    def win_tokens(self) -> int:
        return self.win * self.win

    def validate(self) -> None:
        if self.dim != 1024 or self.heads * 64 != self.dim:
            raise ValueError("the int8 engine needs dim 1024 (16 heads of 64) for the 1024-point rotation")
        if self.img_size % self.patch or self.grid % self.win or self.grid % self.pretrain_grid:
            raise ValueError("the grid must be a multiple of the window and of the pretraining grid")
        if self.hidden % 128:
            raise ValueError("hidden must be a multiple of 128 for the block-128 rotation")

    def gemm_ops(self, batch: int) -> dict[str, int]:
        M, d, h = batch * self.tokens, self.dim, self.hidden
        per = {"qkv": 2 * M * 3 * d * d, "proj": 2 * M * d * d, "fc1": 2 * M * h * d, "fc2": 2 * M * d * h}
        return {k: v * self.depth for k, v in per.items()}

    def attention_flops(self, batch: int) -> int:
        n_glob = sum(1 for i in self.global_blocks if i < self.depth)
        per_win = 4 * batch * self.windows**2 * self.heads * self.win_tokens**2 * 64
        per_glob = 4 * batch * self.heads * self.tokens**2 * 64
        return per_win * (self.depth - n_glob) + per_glob * n_glob


def window_perm(cfg: PixAIConfig) -> torch.Tensor:
    """Window-order position -> row-major grid index (reference.py:21-24): windows row-major, tokens row-major
    inside each window."""
    nw, w, g = cfg.windows, cfg.win, cfg.grid
    wr, wc, r, c = torch.meshgrid(*(torch.arange(n) for n in (nw, nw, w, w)), indexing="ij")
    return ((wr * w + r) * g + wc * w + c).reshape(-1)


def axial_rope(end: int, scale: float, head_dim: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin fp32 [end^2, head_dim/2] per interleaved pair over a row-major end x end grid: pairs 0..15 take the
    column position, 16..31 the row position, times `scale`; frequencies 10000^(-4i/head_dim). Computed in fp32 like
    the reference's tables (reference.py:27-34)."""
    q = head_dim // 4
    freqs = 1.0 / (10000.0 ** (torch.arange(0, head_dim, 4, dtype=torch.float32)[:q] / head_dim))
    t = torch.arange(end * end, dtype=torch.float32)
    col = (t % end) * scale
    row = torch.floor(t / end) * scale
    ang = torch.cat([torch.outer(col, freqs), torch.outer(row, freqs)], dim=-1)
    return torch.cos(ang).contiguous(), torch.sin(ang).contiguous()


def convert_checkpoint(raw: dict[str, torch.Tensor], cfg: PixAIConfig) -> dict[str, torch.Tensor]:
    """Official fp32 state dict -> engine format (engine.py:49-62): each block linear becomes `<name>.qweight`
    (int8, W rotated by blockdiag(H_n)), `<name>.wscale` (fp32 per output channel) and `<name>.bias` (fp32);
    everything else is copied. The rotation product is formed in float64 and rounded once (the reference forms it
    in fp32 on its GPU, so codes can differ by one at rounding ties)."""
    out = {k: v for k, v in raw.items() if not any(f".{n}." in k for n in QUANTIZED)}
    for i in range(cfg.depth):
        for name, n in QUANTIZED.items():
            p = f"blocks.{i}.{name}"
            out[p + ".qweight"], out[p + ".wscale"] = rotate_quantize(raw[p + ".weight"], n)
            out[p + ".bias"] = raw[p + ".bias"].float().contiguous()
    return out


def synthetic_checkpoint(cfg: PixAIConfig, seed: int = 0, head_std: float = 0.05) -> dict[str, torch.Tensor]:
    """Random-init official-format PixAI state dict (the reference's key names and shapes) from a seeded CPU
    generator: linears N(0, 0.02), LayerNorm gamma 1 + N(0, 0.02), beta N(0, 0.02)."""
    g = torch.Generator().manual_seed(seed)
    d, h, p = cfg.dim, cfg.hidden, cfg.patch

    def n(*shape, std=0.02):
        return torch.randn(*shape, generator=g) * std

    sd = {
        "patch_embed.proj.weight": n(d, 3, p, p),
        "pos_embed": n(1, 1 + cfg.pretrain_grid**2, d),
        "ln_pre.weight": 1.0 + n(d),
        "ln_pre.bias": n(d),
        "head_pool.norm.weight": 1.0 + n(d),
        "head_pool.norm.bias": n(d),
        "head_pool.pos_embed": n(cfg.tokens, d),
        "head_pool.q": n(1, 1, d, std=0.5),
        "head_pool.kv.weight": n(2 * d, d),
        "head_pool.kv.bias": n(2 * d),
        "head_pool.proj.weight": n(d, d),
        "head_pool.proj.bias": n(d),
        "head.weight": n(cfg.tags, d, std=head_std),
        "head.bias": n(cfg.tags),
    }
    for i in range(cfg.depth):
        b = f"blocks.{i}."
        sd.update(
            {
                b + "norm1.weight": 1.0 + n(d),
                b + "norm1.bias": n(d),
                b + "attn.qkv.weight": n(3 * d, d),
                b + "attn.qkv.bias": n(3 * d),
                b + "attn.proj.weight": n(d, d),
                b + "attn.proj.bias": n(d),
                b + "norm2.weight": 1.0 + n(d),
                b + "norm2.bias": n(d),
                b + "mlp.fc1.weight": n(h, d),
                b + "mlp.fc1.bias": n(h),
                b + "mlp.fc2.weight": n(d, h),
                b + "mlp.fc2.bias": n(d),
            }
        )
    return sd


def config_from_state(state: dict[str, torch.Tensor], **overrides) -> PixAIConfig:
    """Model dimensions read off a (float or converted) state dict: depth, MLP hidden, tags, pretraining grid."""
    depth = 1 + max(int(k.split(".")[1]) for k in state if k.startswith("blocks."))
    fc1 = state.get("blocks.0.mlp.fc1.weight", state.get("blocks.0.mlp.fc1.qweight"))
    pre = int(round((state["pos_embed"].shape[1] - 1) ** 0.5))
    fields = {"depth": depth, "hidden": fc1.shape[0], "tags": state["head.weight"].shape[0], "pretrain_grid": pre}
    fields.update(overrides)
    return PixAIConfig(**fields)


class PixAIInt8(Int8Engine):
    """images [B, S, S, 3] (normalized pixels, NHWC) -> logits [B, tags] fp32, one HIP graph per batch size;
    mirrors PixAICuda (foidfinder/backends/cuda/engine.py:65-184) on the gfx950 kernels."""

    def __init__(self, state: dict[str, torch.Tensor], cfg: PixAIConfig, *, device: str | torch.device = "cuda"):
        cfg.validate()
        self.cfg = cfg
        self.device = torch.device(device)
        self.k = kernels()
        dev = self.device
        if "blocks.0.attn.qkv.qweight" not in state:
            state = convert_checkpoint({k: v.to(dev) for k, v in state.items()}, cfg)
        t = {k: v.to(dev) for k, v in state.items()}
        d, g, pre = cfg.dim, cfg.grid, cfg.pretrain_grid
        perm = window_perm(cfg).to(dev)

        def lin(p):
            return t[p + ".qweight"].contiguous(), t[p + ".wscale"].float().contiguous(), t[p + ".bias"].float().contiguous()

        def norm(p):
            return t[p + ".weight"].float().contiguous(), t[p + ".bias"].float().contiguous()

        def half(x):
            return x.half().contiguous()

        # stem (reference.py:70-73): conv weight as [d, (kh, kw, c)], the pretraining position grid tiled over the
        # full grid and put in window order
        self.patch_w_t = half(t["patch_embed.proj.weight"].permute(0, 2, 3, 1).reshape(d, -1).t())
        pos = t["pos_embed"][0, 1:].reshape(pre, pre, d).repeat(g // pre, g // pre, 1).reshape(cfg.tokens, d)
        self.pos = half(pos[perm])
        self.ln_pre = (half(t["ln_pre.weight"]), half(t["ln_pre.bias"]))
        # attention-pool head (reference.py:93-98, :133-140)
        self.pool_norm = (half(t["head_pool.norm.weight"]), half(t["head_pool.norm.bias"]))
        self.pool_pos = half(t["head_pool.pos_embed"].reshape(cfg.tokens, d)[perm])
        self.pool_q = half(t["head_pool.q"].reshape(d))
        # the query per head in fp32, times the attention scale 1/sqrt(64) = 0.125 (exact), for pool_head's scores
        self.pool_q_scaled = self.pool_q.float().view(cfg.heads, 64) * 0.125
        self.pool_kv = (half(t["head_pool.kv.weight"]), half(t["head_pool.kv.bias"]))
        self.pool_proj = (half(t["head_pool.proj.weight"]), half(t["head_pool.proj.bias"]))
        self.head = (half(t["head.weight"]), half(t["head.bias"]))
        self.layers = [
            {
                "n1": norm(f"blocks.{i}.norm1"),
                "n2": norm(f"blocks.{i}.norm2"),
                "qkv": lin(f"blocks.{i}.attn.qkv"),
                "proj": lin(f"blocks.{i}.attn.proj"),
                "fc1": lin(f"blocks.{i}.mlp.fc1"),
                "fc2": lin(f"blocks.{i}.mlp.fc2"),
            }
            for i in range(cfg.depth)
        ]
        cw, sw = axial_rope(cfg.win, 1.0)
        cg, sg = axial_rope(g, cfg.win / g)
        pc = perm.cpu()
        self.rope_win = (cw.to(dev), sw.to(dev))
        self.rope_glob = (cg[pc].contiguous().to(dev), sg[pc].contiguous().to(dev))
        self.variants: dict[tuple[str, int], int] = {}
        self._graphs: dict[int, tuple] = {}

    def _buffers(self, B: int) -> dict[str, torch.Tensor]:
        cfg, dev = self.cfg, self.device
        T, d, h = B * cfg.tokens, cfg.dim, cfg.hidden
        return {
            "x": torch.empty(T, d, device=dev, dtype=torch.half),
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
            "qkv": lambda v: self._gemm(buf["a8"], lw["qkv"], buf["rs"], EPI_QKV_ROPE, v, buf["qkv"], self.rope_win),
            "proj": lambda v: self._gemm(buf["a8"], lw["proj"], buf["rs"], EPI_RESIDUAL, v, buf["o16"]),
            "fc1": lambda v: self._gemm(buf["a8"], lw["fc1"], buf["rs"], EPI_GELU_F16, v, buf["h16"]),
            "fc2": lambda v: self._gemm(buf["h8"], lw["fc2"], buf["rs"], EPI_RESIDUAL, v, buf["o16"]),
        }

    def patchify(self, img: torch.Tensor) -> torch.Tensor:
        """[B, S, S, 3] -> window-ordered patches [B * tokens, p*p*3] in (kh, kw, c) order (reference.py:103-107)."""
        cfg = self.cfg
        B, nw, w, p = img.shape[0], cfg.windows, cfg.win, cfg.patch
        x = img.to(torch.half).view(B, nw, w, p, nw, w, p, 3).permute(0, 1, 4, 2, 5, 3, 6, 7)
        return x.reshape(B * cfg.tokens, p * p * 3)

    def pool_head(self, x: torch.Tensor) -> torch.Tensor:
        """x fp16 [B, tokens, d] -> logits fp32 [B, tags] (reference.py:133-140).

        The attention of one learned query per head over the tokens is a matrix-vector product, a softmax and a
        weighted sum, done here in fp32 on the fp16 keys and values, instead of the reference's
        scaled_dot_product_attention of a single query (at 1008 px the stem, pool head and classifier took 316 us
        per image with it and 249 us this way, by kernel traces of one forward)."""
        cfg = self.cfg
        B, L, d, H = x.shape[0], cfg.tokens, cfg.dim, cfg.heads
        h = F.layer_norm(x, (d,), *self.pool_norm, cfg.eps) + self.pool_pos
        kv = F.linear(h, *self.pool_kv).view(B, L, 2, H, 64).permute(2, 0, 3, 1, 4)  # [2, B, H, L, 64] (a view)
        scores = (kv[0] * self.pool_q_scaled.view(H, 1, 64)).sum(-1)  # [B, H, L] fp32, the tokens last
        p = torch.softmax(scores, dim=-1)  # over the last dim (torch's softmax over an inner dim is far slower)
        o = (p.unsqueeze(-1) * kv[1]).sum(2).reshape(B, d).half()  # [B, H, 64] -> [B, d]
        o = F.linear(o, *self.pool_proj)
        return F.linear(o, *self.head).float()

    def _forward(self, img: torch.Tensor, buf: dict[str, torch.Tensor], trace: dict | None = None) -> torch.Tensor:
        """One forward into the preallocated buffers (engine.py:142-161). `trace` (eager debugging) collects the stem
        output and, per block, the qkv, attention output, GELU output and block output."""
        k, cfg = self.k, self.cfg
        B, L, d = img.shape[0], cfg.tokens, cfg.dim
        x, a8, rs = buf["x"], buf["a8"], buf["rs"]
        torch.matmul(self.patchify(img), self.patch_w_t, out=x)
        x.view(B, L, d).add_(self.pos)
        x.copy_(F.layer_norm(x, (d,), *self.ln_pre, cfg.eps))
        v = {name: self.variants.get((name, B), 0) for name in ("qkv", "proj", "fc1", "fc2")}
        eps = cfg.eps
        if trace is not None:
            trace["stem"] = x.clone()
        for i, lw in enumerate(self.layers):
            seq, rope = (L, self.rope_glob) if i in cfg.global_blocks else (cfg.win_tokens, self.rope_win)
            k.rot_q8_1024(x, *lw["n1"], a8, rs, eps)
            self._gemm(a8, lw["qkv"], rs, EPI_QKV_ROPE, v["qkv"], buf["qkv"], rope)
            k.attention(buf["qkv"], buf["o16"], seq)
            if trace is not None:
                trace[f"qkv{i}"], trace[f"attn{i}"] = buf["qkv"].clone(), buf["o16"].clone()
            k.rot_q8_1024(buf["o16"], None, None, a8, rs, eps)
            self._gemm(a8, lw["proj"], rs, EPI_RESIDUAL, v["proj"], x)
            k.rot_q8_1024(x, *lw["n2"], a8, rs, eps)
            self._gemm(a8, lw["fc1"], rs, EPI_GELU_F16, v["fc1"], buf["h16"])
            if trace is not None:
                trace[f"h{i}"] = buf["h16"].clone()
            k.rot_q8_h128(buf["h16"], buf["h8"], rs)
            self._gemm(buf["h8"], lw["fc2"], rs, EPI_RESIDUAL, v["fc2"], x)
            if trace is not None:
                trace[f"x{i}"] = x.clone()
        return self.pool_head(x.view(B, L, d))


def write_int8_dir(model_dir: str | Path, output: str | Path, device: str | torch.device | None = None) -> Path:
    """Writes the reference's converted PixAI checkpoint (the output of `foidfinder convert`, cli.py:143-161) from an
    official model directory: `model.safetensors` with each block linear as `<name>.qweight` int8 [N, K],
    `<name>.wscale` fp32 [N] and `<name>.bias` fp32 [N] (every other tensor copied unchanged) and the metadata
    `{"format": "foidfinder-pixai-int8-v1"}` (engine.py:44-62), plus the source's `config.json`. The conversion runs
    on `device` (the GPU when present, as the reference's does) and is the same bits on any device. Returns the
    output directory; `load_pixai_dir` and the reference's loader (engine.py:68-70) read it without converting."""
    import shutil

    from safetensors.torch import load_file, save_file

    model_dir, output = Path(model_dir), Path(output)
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    state = load_file(str(model_dir / "model.safetensors"), device=str(device))
    if "blocks.0.attn.qkv.qweight" in state:
        raise RuntimeError(f"{model_dir}: already in the int8 format")
    config = json.loads((model_dir / "config.json").read_text())
    over = dict(config.get("foidfinder_rocm", {}))
    if "global_blocks" in over:
        over["global_blocks"] = tuple(over["global_blocks"])
    out = convert_checkpoint(state, config_from_state(state, **over))
    output.mkdir(parents=True, exist_ok=True)
    save_file({k: v.contiguous().cpu() for k, v in out.items()}, str(output / "model.safetensors"), {"format": FORMAT})
    shutil.copy(model_dir / "config.json", output / "config.json")
    return output


def load_pixai_dir(model_dir: str | Path, device: str | torch.device = "cuda") -> tuple[PixAIInt8, dict]:
    """A PixAI model directory as the reference reads it (config.json + model.safetensors, official fp32 weights or
    the converted int8 format; engine.py:65-72). Dimensions come from the weights; an optional
    config["foidfinder_rocm"] object overrides PixAIConfig fields (image size, window, global blocks) for models of
    the same structure at other sizes."""
    from safetensors.torch import load_file

    model_dir = Path(model_dir)
    config = json.loads((model_dir / "config.json").read_text())
    state = load_file(str(model_dir / "model.safetensors"), device=str(device))
    over = dict(config.get("foidfinder_rocm", {}))
    if "global_blocks" in over:
        over["global_blocks"] = tuple(over["global_blocks"])
    cfg = config_from_state(state, **over)
    return PixAIInt8(state, cfg, device=device), config
