"""EVA02 int8 tagger on MI355X: gfx950 kernels for every block op, one HIP graph per batch size.

Per transformer block (the reference's int8 block, foidfinder/backends/cuda/engine.py:1-10 and :150-160, with the
EVA02 SwiGLU MLP of foidfinder/backends/mlx/haruka.py:196-209):

  LN1 -> H1024 rotation -> int8 (per-token scale)  -> QKV GEMM (int32 acc) + bias + RoPE, q x scale*log2(e) -> fp16
  flash attention (fp16 MFMA, fp32 accumulate)     -> fp16
  H1024 rotation -> int8                           -> proj GEMM + bias + residual (fp16 stream)
  LN2 -> H1024 rotation -> int8                    -> fc1 GEMM + bias + SwiGLU -> fp16 [T, 2816]
  mlp LayerNorm -> block-H128 rotation -> int8     -> fc2 GEMM + bias + residual

Weights carry the same rotations (W' = W H) and are quantized per output channel. Stem (patch GEMM) and head
(final LayerNorm, tag GEMM) run in fp16 through PyTorch (hipBLASLt), as the reference's stem and head run through
cuBLAS.
"""

from __future__ import annotations

import json
import math
from dataclasses import asdict, dataclass
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

from .kernels import EPI_QKV_ROPE, EPI_RESIDUAL, EPI_SWIGLU, kernels, lib, pad_norm

Q_SCALE = 0.125 * math.log2(math.e)  # softmax scale x log2(e), folded into q by the QKV epilogue (engine.py:26)
FORMAT = "foidfinder-eva02-int8-v1"


@dataclass(frozen=True)
class Eva02Config:
    """EVA02-L/14 at 448 px by default: 1 cls + 32x32 patch tokens, d 1024, 16 heads of 64, 24 blocks, SwiGLU hidden
    2730 padded to 2816 = 22 x 128 for the block-128 rotation, LayerNorm eps 1e-6, 30877 tags."""

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

    def validate(self) -> None:
        if self.dim != 1024 or self.heads * 64 != self.dim:
            raise ValueError("the int8 engine needs dim 1024 (16 heads of 64) for the 1024-point rotation")
        if self.hidden_pad % 128 or self.hidden_pad < self.hidden:
            raise ValueError("hidden_pad must be a multiple of 128 covering hidden")
        if self.img_size % self.patch:
            raise ValueError("img_size must be a multiple of patch")

    def gemm_ops(self, batch: int) -> dict[str, int]:
        """Algorithmic int8 work per forward: 2*M*N*K with the unpadded model dims, summed over blocks."""
        M, d, h = batch * self.tokens, self.dim, self.hidden
        per = {"qkv": 2 * M * 3 * d * d, "proj": 2 * M * d * d, "fc1": 2 * M * 2 * h * d, "fc2": 2 * M * d * h}
        return {k: v * self.depth for k, v in per.items()}

    def attention_flops(self, batch: int) -> int:
        return 4 * batch * self.heads * self.tokens * self.tokens * 64 * self.depth


def hadamard(n: int, device: torch.device | str = "cpu") -> torch.Tensor:
    """Normalized Sylvester Hadamard matrix (symmetric, orthogonal), built in float64 (engine.py:29-34)."""
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / math.sqrt(n)).to(device=device)


def quantize_rows_int8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-output-channel int8 in float32: w ~= q * scale[:, None] (engine.py:37-41):
    scale = max(amax, 1e-12) / 127 and q = clamp(round(w / scale), -127, 127), both divisions IEEE float32.

    Each float32 quotient is formed as a float64 division of tensors rounded to float32, which is the correctly
    rounded float32 quotient (double rounding is harmless for division when 53 >= 2 * 24 + 2) on every device:
    torch's float32 division on the GPU is not always correctly rounded (a division by a scalar becomes a multiply
    by its reciprocal), and a last-bit difference in a quotient near a rounding tie changes a code."""
    w = w.float()
    amax = w.abs().amax(1).clamp_min(1e-12).double()
    scale = (amax / torch.full_like(amax, 127.0)).float()
    q = torch.round((w.double() / scale.double()[:, None]).float()).clamp(-127, 127).to(torch.int8)
    return q.contiguous(), scale.contiguous()


def rotate_rows64(w: torch.Tensor, block: int) -> torch.Tensor:
    """W [N, K] @ blockdiag(H_block) in float64 by a fast Walsh-Hadamard transform over each block of K columns:
    butterflies (a, b) -> (a + b, a - b) over column bits 0, 1, 2, ... in that order, then x 1/sqrt(block). Every
    step is one IEEE float64 operation in a fixed order, so the result is the same bits on the CPU and on the GPU
    (a BLAS product sums in a device-dependent order and can differ in the last bit, which the rounding to float32
    and the quantization below can turn into a different code)."""
    n, k = w.shape
    v = w.double().reshape(n, k // block, block)
    half = 1
    while half < block:
        v = v.reshape(n, k // block, block // (2 * half), 2, half)
        a, b = v[..., 0, :], v[..., 1, :]
        v = torch.stack((a + b, a - b), dim=-2)
        half *= 2
    return v.reshape(n, k) * (1.0 / math.sqrt(block))


def rotate_quantize(w: torch.Tensor, block: int) -> tuple[torch.Tensor, torch.Tensor]:
    """quantize_rows_int8(W @ blockdiag(H_block)); the product in float64 (rotate_rows64), rounded to float32 once
    (the reference forms it in fp32 with cuBLAS, engine.py:59)."""
    return quantize_rows_int8(rotate_rows64(w, block).float())


def eva02_rope_tables(grid: int, ref: int, head_dim: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """EVA02 axial RoPE per interleaved pair: cos/sin fp32 [1 + grid^2, head_dim/2]; row 0 (cls) is the identity;
    pairs 0..15 take the row position, 16..31 the column position, rescaled to the pretraining grid. Computed as the
    reference computes its tables, in float32 numpy arithmetic throughout (bands, positions, angles, cos and sin;
    foidfinder/backends/mlx/haruka.py:22-33), so the served tables carry the reference's roundings."""
    q = head_dim // 4
    bands = np.float32(1.0) / (np.float32(10000.0) ** (np.arange(q, dtype=np.float32) / np.float32(q)))
    t = np.arange(grid, dtype=np.float32) / np.float32(grid) * np.float32(ref)
    ty, tx = np.meshgrid(t, t, indexing="ij")
    ang = np.concatenate([ty.reshape(-1, 1) * bands, tx.reshape(-1, 1) * bands], axis=1)
    cos = np.concatenate([np.ones((1, head_dim // 2), np.float32), np.cos(ang)])
    sin = np.concatenate([np.zeros((1, head_dim // 2), np.float32), np.sin(ang)])
    assert cos.dtype == np.float32 and sin.dtype == np.float32
    return torch.from_numpy(np.ascontiguousarray(cos)), torch.from_numpy(np.ascontiguousarray(sin))


def convert_checkpoint(raw: dict[str, torch.Tensor], cfg: Eva02Config) -> dict[str, torch.Tensor]:
    """Float EVA02 state dict -> engine format. Each block linear becomes `<name>.qweight` (int8, rotated by W H),
    `<name>.wscale` (fp32 per output channel) and `<name>.bias` (fp32); norms become fp32; everything else is copied.

    fc1 (gate rows then value rows, foidfinder/haruka.py:59-60) is interleaved as (gate j, value j) row pairs and
    zero-padded to 2 x hidden_pad rows so the SwiGLU epilogue finds both operands in one tile; fc2 is zero-padded to
    K = hidden_pad and rotated by blockdiag(H128). Mirrors convert_checkpoint, foidfinder/backends/cuda/engine.py:49-62."""
    d, h, hp = cfg.dim, cfg.hidden, cfg.hidden_pad
    out = {k: v for k, v in raw.items() if not k.startswith("blocks.")}
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        for name in ("attn.qkv", "attn.proj"):
            out[p + name + ".qweight"], out[p + name + ".wscale"] = rotate_quantize(raw[p + name + ".weight"], d)
            out[p + name + ".bias"] = raw[p + name + ".bias"].float().contiguous()
        w1, b1 = raw[p + "mlp.fc1.weight"].float(), raw[p + "mlp.fc1.bias"].float()
        wi = torch.zeros(2 * hp, d, device=w1.device)
        bi = torch.zeros(2 * hp, device=w1.device)
        wi[0 : 2 * h : 2], wi[1 : 2 * h : 2] = w1[:h], w1[h:]
        bi[0 : 2 * h : 2], bi[1 : 2 * h : 2] = b1[:h], b1[h:]
        out[p + "mlp.fc1.qweight"], out[p + "mlp.fc1.wscale"] = rotate_quantize(wi, d)
        out[p + "mlp.fc1.bias"] = bi
        w2 = torch.zeros(d, hp, device=w1.device)
        w2[:, :h] = raw[p + "mlp.fc2.weight"].float()
        out[p + "mlp.fc2.qweight"], out[p + "mlp.fc2.wscale"] = rotate_quantize(w2, 128)
        out[p + "mlp.fc2.bias"] = raw[p + "mlp.fc2.bias"].float().contiguous()
        for n in ("norm1", "norm2", "mlp.norm"):
            out[p + n + ".weight"] = raw[p + n + ".weight"].float().contiguous()
            out[p + n + ".bias"] = raw[p + n + ".bias"].float().contiguous()
    return out


def synthetic_checkpoint(cfg: Eva02Config, seed: int = 0, head_std: float = 0.05) -> dict[str, torch.Tensor]:
    """Random-init float EVA02 state dict from a seeded CPU generator: linears N(0, 0.02), LayerNorm gamma 1 + N(0, 0.02),
    beta N(0, 0.02), k bias zero (foidfinder/haruka.py:55-57)."""
    g = torch.Generator().manual_seed(seed)
    d, h = cfg.dim, cfg.hidden

    def n(*shape, std=0.02):
        return torch.randn(*shape, generator=g) * std

    sd = {
        "patch_embed.weight": n(d, cfg.patch * cfg.patch * 3),
        "patch_embed.bias": n(d),
        "cls_token": n(d),
        "pos_embed": n(cfg.tokens, d),
        "norm.weight": 1.0 + n(d),
        "norm.bias": n(d),
        "head.weight": n(cfg.tags, d, std=head_std),
        "head.bias": n(cfg.tags),
    }
    for i in range(cfg.depth):
        p = f"blocks.{i}."
        qkv_b = n(3 * d)
        qkv_b[d : 2 * d] = 0
        sd.update(
            {
                p + "norm1.weight": 1.0 + n(d),
                p + "norm1.bias": n(d),
                p + "attn.qkv.weight": n(3 * d, d),
                p + "attn.qkv.bias": qkv_b,
                p + "attn.proj.weight": n(d, d),
                p + "attn.proj.bias": n(d),
                p + "norm2.weight": 1.0 + n(d),
                p + "norm2.bias": n(d),
                p + "mlp.fc1.weight": n(2 * h, d),
                p + "mlp.fc1.bias": n(2 * h),
                p + "mlp.norm.weight": 1.0 + n(h),
                p + "mlp.norm.bias": n(h),
                p + "mlp.fc2.weight": n(d, h),
                p + "mlp.fc2.bias": n(d),
            }
        )
    return sd


GEMMS = ("qkv", "proj", "fc1", "fc2")


class Int8Engine:
    """What the int8 engines share (foidfinder/backends/cuda/engine.py:65-184): a per-batch buffer plan, GEMM tile
    variant autotune, two warm-up forwards on a side stream, graph capture, then replay. Subclasses provide
    `_buffers(B)`, `_gemm_jobs(buf)` (the four GEMMs of block 0 on those buffers) and `_forward(img, buf, trace)`."""

    device: torch.device
    variants: dict[tuple[str, int], int]
    _graphs: dict[int, tuple]
    q_scale: float = Q_SCALE  # factor on q after RoPE in the QKV epilogue: softmax scale (unless folded) x log2(e)

    def _buffers(self, B: int) -> dict[str, torch.Tensor]:
        raise NotImplementedError

    def _gemm_jobs(self, buf: dict[str, torch.Tensor]) -> dict:
        raise NotImplementedError

    def _forward(self, img: torch.Tensor, buf: dict[str, torch.Tensor], trace: dict | None = None) -> torch.Tensor:
        raise NotImplementedError

    def _gemm(self, a, lw, rs, epi, variant, out, rope=None):
        w, ws, b = lw
        cos, sin = rope if rope is not None else (None, None)
        self.k.gemm_s8(a, w, rs, ws, b, out, epi, variant, cos, sin, self.q_scale)

    def _autotune(self, B: int, buf: dict[str, torch.Tensor]) -> None:
        """Pick the fastest GEMM tile variant per GEMM for this batch size (engine.py:108-135). The activation
        operands are codes distributed like the rotations' output (a rotated row is close to Gaussian, and its
        absmax sits near 3.3 standard deviations, so codes ~ N(0, 38^2)), not zeros or uniform codes: MFMA power and
        so the clock depend on the data. Each variant's launches are captured in a HIP graph and replayed, so the
        host's launch cost (which exceeds a short GEMM's run time at small batches, and more so under a profiler)
        does not mask the differences; each is timed in three interleaved rounds and keeps its best round, so a
        momentary clock dip does not decide the pick."""
        g = torch.Generator(device=buf["a8"].device).manual_seed(0)
        for name in ("a8", "h8"):
            t = buf[name]
            codes = torch.randn(t.shape, device=t.device, generator=g).mul_(38.0).round_().clamp_(-127, 127)
            t.copy_(codes.to(torch.int8))
            del codes
        buf["rs"].fill_(1e-2)
        buf["o16"].zero_()
        n = lib().ff_gemm_s8_variants()
        for name, fn in self._gemm_jobs(buf).items():
            graphs = {}
            for v in range(1, n + 1):
                fn(v)  # eager first: a variant that rejects the shape raises here, outside any capture
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    for _ in range(5):
                        fn(v)
                graphs[v] = graph
            times = {v: float("inf") for v in graphs}
            for _ in range(3):
                for v, graph in graphs.items():
                    graph.replay()
                    start, end = torch.cuda.Event(True), torch.cuda.Event(True)
                    start.record()
                    graph.replay()
                    end.record()
                    torch.cuda.synchronize()
                    times[v] = min(times[v], start.elapsed_time(end))
            del graphs
            self.variants[(name, B)] = min(times, key=times.get)

    def eager(self, images: torch.Tensor, trace: dict | None = None) -> torch.Tensor:
        """One forward without graph capture (fresh buffers)."""
        buf = self._buffers(images.shape[0])
        return self._forward(images, buf, trace).clone()

    @torch.no_grad()
    def __call__(self, images: torch.Tensor) -> torch.Tensor:
        """images [B, S, S, 3] normalized pixels (any float dtype) -> logits [B, tags] fp32."""
        B = images.shape[0]
        if B not in self._graphs:
            buf = self._buffers(B)
            self._autotune(B, buf)
            static_in = torch.zeros(B, *images.shape[1:], device=self.device, dtype=torch.half)
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(2):  # warm up (library workspaces allocate outside capture)
                    self._forward(static_in, buf)
            torch.cuda.current_stream().wait_stream(stream)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                static_out = self._forward(static_in, buf)
            self._graphs[B] = (graph, static_in, static_out, buf)
        graph, static_in, static_out, _ = self._graphs[B]
        static_in.copy_(images)
        graph.replay()
        return static_out.clone()

    def replay(self, B: int) -> None:
        """Replays the captured graph for batch B on its current input (benchmarking)."""
        self._graphs[B][0].replay()


class Eva02Int8(Int8Engine):
    """images [B, S, S, 3] (normalized pixels, NHWC) -> logits [B, tags] fp32, one HIP graph per batch size.

    Mirrors PixAICuda (foidfinder/backends/cuda/engine.py:65-184): preallocated buffers, per-batch GEMM variant
    autotune, two warm-up forwards on a side stream, graph capture, then replay."""

    def __init__(self, state: dict[str, torch.Tensor], cfg: Eva02Config, *, device: str | torch.device = "cuda"):
        cfg.validate()
        self.cfg = cfg
        self.device = torch.device(device)
        self.k = kernels()
        dev = self.device
        if "blocks.0.attn.qkv.qweight" not in state:
            state = convert_checkpoint({k: v.to(dev) for k, v in state.items()}, cfg)
        t = {k: v.to(dev) for k, v in state.items()}

        def lin(p):
            return t[p + ".qweight"].contiguous(), t[p + ".wscale"].float().contiguous(), t[p + ".bias"].float().contiguous()

        def norm(p):
            return t[p + ".weight"].float().contiguous(), t[p + ".bias"].float().contiguous()

        d = cfg.dim
        self.patch_w_t = t["patch_embed.weight"].half().t().contiguous()  # [p*p*3, d]
        pos = t["pos_embed"].float().reshape(cfg.tokens, d)
        self.patch_bias_pos = (t["patch_embed.bias"].float() + pos[1:]).half().contiguous()  # [g*g, d]
        self.cls_pos = (t["cls_token"].float().reshape(d) + pos[0]).half().contiguous()
        self.norm = norm("norm")
        self.head_w = t["head.weight"].half().contiguous()
        self.head_b = t["head.bias"].half().contiguous()
        self.layers = [
            {
                "n1": norm(f"blocks.{i}.norm1"),
                "n2": norm(f"blocks.{i}.norm2"),
                "nm": pad_norm(*norm(f"blocks.{i}.mlp.norm"), cfg.hidden_pad),
                "qkv": lin(f"blocks.{i}.attn.qkv"),
                "proj": lin(f"blocks.{i}.attn.proj"),
                "fc1": lin(f"blocks.{i}.mlp.fc1"),
                "fc2": lin(f"blocks.{i}.mlp.fc2"),
            }
            for i in range(cfg.depth)
        ]
        cos, sin = eva02_rope_tables(cfg.grid, cfg.rope_ref)
        self.rope = (cos.to(dev), sin.to(dev))
        self.variants: dict[tuple[str, int], int] = {}
        self._graphs: dict[int, tuple] = {}

    # ---- buffer plan (engine.py:96-106) ----
    def _buffers(self, B: int) -> dict[str, torch.Tensor]:
        cfg, dev = self.cfg, self.device
        T, d, hp = B * cfg.tokens, cfg.dim, cfg.hidden_pad
        return {
            "x": torch.empty(T, d, device=dev, dtype=torch.half),
            "patch": torch.empty(B * cfg.grid * cfg.grid, d, device=dev, dtype=torch.half),
            "a8": torch.empty(T, d, device=dev, dtype=torch.int8),
            "rs": torch.empty(T, device=dev),
            "qkv": torch.empty(T, 3 * d, device=dev, dtype=torch.half),
            "o16": torch.empty(T, d, device=dev, dtype=torch.half),
            "h16": torch.empty(T, hp, device=dev, dtype=torch.half),
            "h8": torch.empty(T, hp, device=dev, dtype=torch.int8),
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
        """[B, S, S, 3] -> [B * g * g, p*p*3] patches in (kh, kw, c) order, row-major over the grid."""
        cfg = self.cfg
        B, g, p = img.shape[0], cfg.grid, cfg.patch
        x = img.to(torch.half).view(B, g, p, g, p, 3).permute(0, 1, 3, 2, 4, 5)
        return x.reshape(B * g * g, p * p * 3)

    def _forward(self, img: torch.Tensor, buf: dict[str, torch.Tensor], trace: dict | None = None) -> torch.Tensor:
        """One forward into the preallocated buffers. `trace` (eager debugging only) collects copies of the stem
        output and, per block, the qkv, attention output, SwiGLU output and block output."""
        k, cfg = self.k, self.cfg
        B, L, d = img.shape[0], cfg.tokens, cfg.dim
        x, a8, rs = buf["x"], buf["a8"], buf["rs"]
        torch.matmul(self.patchify(img), self.patch_w_t, out=buf["patch"])
        xv = x.view(B, L, d)
        torch.add(buf["patch"].view(B, L - 1, d), self.patch_bias_pos, out=xv[:, 1:])
        xv[:, 0] = self.cls_pos
        v = {name: self.variants.get((name, B), 0) for name in GEMMS}
        eps = cfg.eps
        if trace is not None:
            trace["stem"] = x.clone()
        for i, lw in enumerate(self.layers):
            k.rot_q8_1024(x, *lw["n1"], a8, rs, eps)
            self._gemm(a8, lw["qkv"], rs, EPI_QKV_ROPE, v["qkv"], buf["qkv"], self.rope)
            k.attention(buf["qkv"], buf["o16"], L)
            if trace is not None:
                trace[f"qkv{i}"], trace[f"attn{i}"] = buf["qkv"].clone(), buf["o16"].clone()
            k.rot_q8_1024(buf["o16"], None, None, a8, rs, eps)
            self._gemm(a8, lw["proj"], rs, EPI_RESIDUAL, v["proj"], x)
            k.rot_q8_1024(x, *lw["n2"], a8, rs, eps)
            self._gemm(a8, lw["fc1"], rs, EPI_SWIGLU, v["fc1"], buf["h16"])
            if trace is not None:
                trace[f"h{i}"] = buf["h16"].clone()
            k.rot_q8_h128(buf["h16"], buf["h8"], rs, *lw["nm"], cfg.hidden, eps)
            self._gemm(buf["h8"], lw["fc2"], rs, EPI_RESIDUAL, v["fc2"], x)
            if trace is not None:
                trace[f"x{i}"] = x.clone()
        cls = F.layer_norm(xv[:, 0].float(), (d,), *self.norm, eps).half()
        return F.linear(cls, self.head_w, self.head_b).float()


def save_model_dir(out_dir: str | Path, state: dict[str, torch.Tensor], cfg: Eva02Config, tags: list[str],
                   categories: list[str], thresholds: dict[str, float], name: str = "EVA02-L int8 tagger") -> None:
    """Writes model.safetensors (engine format) + config.json (the Haruka-style tag config TagIndex reads)."""
    from safetensors.torch import save_file

    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    save_file({k: v.contiguous().cpu() for k, v in state.items()}, str(out_dir / "model.safetensors"),
              {"format": FORMAT})
    config = {"model": {"name": name, "architecture": "eva02-int8", **asdict(cfg)}, "tags": tags,
              "categories": categories, "thresholds": thresholds}
    (out_dir / "config.json").write_text(json.dumps(config))


def load_model_dir(model_dir: str | Path, device: str | torch.device = "cuda") -> tuple[Eva02Int8, dict]:
    from safetensors.torch import load_file

    model_dir = Path(model_dir)
    config = json.loads((model_dir / "config.json").read_text())
    m = config.get("model", {})
    if m.get("architecture") != "eva02-int8":
        raise RuntimeError(f"{model_dir}: not an eva02-int8 model (architecture {m.get('architecture')!r})")
    fields = {f: m[f] for f in Eva02Config.__dataclass_fields__ if f in m}
    cfg = Eva02Config(**fields)
    state = load_file(str(model_dir / "model.safetensors"), device=str(device))
    return Eva02Int8(state, cfg, device=device), config
