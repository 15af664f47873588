"""Parity of the gfx950 kernels with the CPU oracle on identical seeded inputs, through the C ABI.

Bars: int8 codes, fp32 row scales and int32 accumulators bit-exact; fp16 epilogues bias, residual and QKV+RoPE
bit-exact; SwiGLU within one fp16 ulp (the GPU's silu uses its ~1-ulp exp and reciprocal units); GELU within one
fp16 ulp or 1e-6 absolute (the same units, in the sigmoid form); attention within 4e-3 absolute and 2e-3 relative
per output row of the float64 oracle (P is rounded to fp16 before the PV MFMA).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import gemm as OG
from oracle import model as OM
from oracle import rotq8 as OR

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def to_gpu(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def activations(rng, T: int, C: int, outlier_frac: float = 0.01) -> np.ndarray:
    x = rng.standard_normal((T, C), dtype=np.float32)
    cols = rng.choice(C, max(1, int(C * outlier_frac)), replace=False)
    x[:, cols] *= 20.0
    return x.astype(np.float16)


def special_rows(C: int) -> np.ndarray:
    """Zero row, one-hot rows, a constant row, a row of fp16 extremes, an alternating-sign row."""
    rows = np.zeros((6, C), np.float16)
    rows[1, 0] = 1.0
    rows[2, C - 1] = -3.5
    rows[3, :] = 0.25
    rows[4, ::3] = 60000.0
    rows[4, 1::3] = -60000.0
    rows[5, :] = np.where(np.arange(C) % 2 == 0, 1.0, -1.0)
    return rows


def run_rot1024(x, dev, gamma=None, beta=None, eps=1e-5):
    from foidfinder_amd import kernels as K

    xt = to_gpu(x, dev)
    out = torch.empty(x.shape, dtype=torch.int8, device=dev)
    rs = torch.empty(x.shape[0], dtype=torch.float32, device=dev)
    g = None if gamma is None else to_gpu(gamma, dev)
    b = None if beta is None else to_gpu(beta, dev)
    K.rot_q8_1024(xt, g, b, out, rs, eps)
    torch.cuda.synchronize()
    return out.cpu().numpy(), rs.cpu().numpy()


def assert_codes_equal(got, want, what):
    (q, s), (q0, s0) = got, want
    bad = np.flatnonzero((q != q0).any(axis=1) | (s.view(np.uint32) != s0.view(np.uint32)))
    assert bad.size == 0, f"{what}: {bad.size} rows differ, first {bad[:5]}; scales {s[bad[:3]]} vs {s0[bad[:3]]}"


@pytest.mark.parametrize("T", [1, 8, 13, 1025])
def test_rot_q8_1024_bit_exact(dev, rng, T):
    x = activations(rng, T, 1024)
    assert_codes_equal(run_rot1024(x, dev), OR.rot_q8_1024(x), f"rot_q8_1024 T={T}")


def test_rot_q8_1024_special_rows(dev):
    x = special_rows(1024)
    got = run_rot1024(x, dev)
    assert_codes_equal(got, OR.rot_q8_1024(x), "special rows")
    assert (got[0][0] == 0).all() and got[1][0] == np.float32(np.float32(1e-12) / np.float32(127))
    assert (np.abs(got[0][1].astype(int)) == 127).all()  # one-hot spreads evenly


@pytest.mark.parametrize("eps", [1e-5, 1e-6])
@pytest.mark.parametrize("T", [3, 1025])
def test_rot_q8_1024_layernorm_bit_exact(dev, rng, T, eps):
    x = activations(rng, T, 1024)
    g = (1.0 + 0.02 * rng.standard_normal(1024)).astype(np.float32)
    b = (0.02 * rng.standard_normal(1024)).astype(np.float32)
    assert_codes_equal(run_rot1024(x, dev, g, b, eps), OR.rot_q8_1024(x, g, b, eps), f"LN rot T={T}")


def run_h128(x, dev, c_real=0, gamma=None, beta=None, eps=1e-6):
    from foidfinder_amd import kernels as K

    xt = to_gpu(x, dev)
    out = torch.empty(x.shape, dtype=torch.int8, device=dev)
    rs = torch.empty(x.shape[0], dtype=torch.float32, device=dev)
    g = b = None
    if gamma is not None:
        g, b = K.pad_norm(to_gpu(gamma, dev), to_gpu(beta, dev), x.shape[1])
    K.rot_q8_h128(xt, out, rs, g, b, c_real, eps)
    torch.cuda.synchronize()
    return out.cpu().numpy(), rs.cpu().numpy()


@pytest.mark.parametrize("C", [128, 512, 640, 768, 2048, 2816, 4736])
@pytest.mark.parametrize("T", [1, 5, 300])
def test_rot_q8_h128_bit_exact(dev, rng, T, C):
    x = activations(rng, T, C)
    assert_codes_equal(run_h128(x, dev), OR.rot_q8_h128(x), f"h128 T={T} C={C}")


@pytest.mark.parametrize(("C", "c_real"), [(2816, 2730), (768, 768), (2048, 2048), (1024, 1000), (4736, 4736), (256, 130),
                                         (2816, 1000), (2048, 700), (4736, 4500)])
def test_rot_q8_h128_layernorm_bit_exact(dev, rng, C, c_real):
    x = activations(rng, 257, C)
    x[:, c_real:] = 0
    g = (1.0 + 0.02 * rng.standard_normal(c_real)).astype(np.float32)
    b = (0.02 * rng.standard_normal(c_real)).astype(np.float32)
    got = run_h128(x, dev, c_real, g, b, 1e-6)
    assert_codes_equal(got, OR.rot_q8_h128(x, c_real, g, b, 1e-6), f"LN h128 C={C}")


def assert_within_one_fp16_ulp(got: np.ndarray, want: np.ndarray, what: str) -> None:
    g, w = got.astype(np.float32), want.astype(np.float32)
    ulp = np.maximum(np.spacing(np.abs(want)), np.spacing(np.abs(got))).astype(np.float32)
    bad = np.argwhere(~(np.abs(g - w) <= ulp))
    assert bad.size == 0, f"{what}: {len(bad)} values off by more than one fp16 ulp, first {bad[:4].tolist()}"


def gemm_inputs(rng, M, N, K):
    a = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    rs = (rng.random(M, dtype=np.float32) * 0.05 + 1e-3).astype(np.float32)
    cs = (rng.random(N, dtype=np.float32) * 1e-3 + 1e-5).astype(np.float32)
    bias = (0.02 * rng.standard_normal(N)).astype(np.float32)
    return a, w, rs, cs, bias


def run_gemm(dev, a, w, rs, cs, bias, epi, variant, out=None, rope=None, q_scale=1.0):
    from foidfinder_amd import kernels as K

    M, N = a.shape[0], w.shape[0]
    dtype = torch.int32 if epi == K.EPI_I32 else torch.float16
    o = torch.empty(K.out_shape(M, N, epi), dtype=dtype, device=dev) if out is None else to_gpu(out, dev)
    cos, sin = (None, None) if rope is None else (to_gpu(rope[0], dev), to_gpu(rope[1], dev))
    K.gemm_s8(to_gpu(a, dev), to_gpu(w, dev), to_gpu(rs, dev), to_gpu(cs, dev), to_gpu(bias, dev), o, epi, variant,
              cos, sin, q_scale)
    torch.cuda.synchronize()
    return o.cpu().numpy()


GEMM_VARIANTS = [1, 2, 3, 4, 5, 6]  # ff_gemm_s8_variants()
PERSISTENT = 4  # the persistent 256 x 256 variant (with split-K blocks for the rows past the last whole tile)
GEMM_SHAPES = [(1, 16, 64), (17, 48, 128), (300, 3072, 1024), (1025, 5632, 1024), (129, 1024, 2816), (257, 272, 192),
               (300, 1024, 2816)]


def test_gemm_variant_list_is_complete(dev):
    from foidfinder_amd import kernels as K

    assert K.lib().ff_gemm_s8_variants() == max(GEMM_VARIANTS)


@pytest.mark.parametrize("variant", GEMM_VARIANTS)
@pytest.mark.parametrize(("M", "N", "K"), GEMM_SHAPES)
def test_gemm_s8_int32_bit_exact(dev, rng, M, N, K, variant):
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_I32, variant)
    want = OG.gemm_s8_i32(a, w)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"


def _random_gemm_shapes(n: int, seed: int = 7) -> list[tuple[int, int, int]]:
    """Seeded shapes off every tile grid: M anywhere in 1..600 (with the 64-, 128- and 256-row tile edges), N any
    multiple of 16 up to 512, K any multiple of 64 up to 1280 (odd multiples take the K-64 rings)."""
    r = np.random.default_rng(seed)
    edges = [63, 64, 65, 127, 129, 255, 256, 257, 511, 513]
    return [(int(edges[i] if i < len(edges) and i % 2 == 0 else r.integers(1, 601)), 16 * int(r.integers(1, 33)),
             64 * int(r.integers(1, 21))) for i in range(n)]


RANDOM_GEMM_SHAPES = _random_gemm_shapes(8)
_random_gemm_cache: dict = {}


@pytest.mark.parametrize("variant", GEMM_VARIANTS)
@pytest.mark.parametrize("shape", range(len(RANDOM_GEMM_SHAPES)))
def test_gemm_s8_random_shapes_int32_bit_exact(dev, shape, variant):
    """Every tile variant on the same seeded shapes (inputs drawn once per shape, the oracle product computed once)."""
    M, N, K = RANDOM_GEMM_SHAPES[shape]
    if shape not in _random_gemm_cache:
        a, w, *_ = gemm_inputs(np.random.default_rng(1000 + shape), M, N, K)
        _random_gemm_cache[shape] = (a, w, OG.gemm_s8_i32(a, w))
    a, w, want = _random_gemm_cache[shape]
    ones = np.ones(M, np.float32)
    got = run_gemm(dev, a, w, ones, np.ones(N, np.float32), np.zeros(N, np.float32), OG.EPI_I32, variant)
    bad = np.argwhere(got != want)
    assert bad.size == 0, (f"M={M} N={N} K={K} variant {variant}: {len(bad)} mismatches, first at "
                           f"{bad[:4].tolist()}")


@pytest.mark.parametrize("variant", GEMM_VARIANTS)
@pytest.mark.parametrize("epi", [OG.EPI_BIAS_F16, OG.EPI_RESIDUAL, OG.EPI_QKV_ROPE, OG.EPI_SWIGLU])
def test_gemm_s8_epilogue_bit_exact(dev, rng, epi, variant):
    M, K = 1025, 1024
    N = {OG.EPI_QKV_ROPE: 3072, OG.EPI_SWIGLU: 5632}.get(epi, 1024)
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    kw = {}
    out = None
    if epi == OG.EPI_RESIDUAL:
        out = rng.standard_normal((M, N)).astype(np.float16)
        kw["residual"] = out
    rope = None
    if epi == OG.EPI_QKV_ROPE:
        rope = OM.eva02_rope_tables(32, 16)
        kw.update(rope_cos=rope[0], rope_sin=rope[1], q_scale=OM.Q_SCALE)
    got = run_gemm(dev, a, w, rs, cs, bias, epi, variant, out=out, rope=rope, q_scale=kw.get("q_scale", 1.0))
    want = OG.gemm_s8(a, w, rs, cs, bias, epi, **kw)
    if epi == OG.EPI_SWIGLU:
        assert_within_one_fp16_ulp(got, want, f"SwiGLU epilogue, variant {variant}")
        return
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"


@pytest.mark.parametrize("variant", GEMM_VARIANTS)
def test_w8a8_linear_chain_bit_exact(dev, variant):
    """The plumbing config's single W8A8 linear at full size, with its own generator (fp16 [1025, 1024] ~ N(0, 1) with
    1 % of channels x20, weights N(0, 0.02) rotated and quantized per row with fp16-rounded scales, bias N(0, 0.02)):
    rot_q8_1024 then gemm_s8 with the bias epilogue at N = 3072, as the reference chains the two ops
    (kernels.cu:187-235). Codes, fp32 row scales and fp16 outputs bit-exact with the oracle's chain."""
    from foidfinder_amd import kernels as K

    x, qw, ws, b = OM.w8a8_linear_inputs()
    a8 = torch.empty(x.shape, dtype=torch.int8, device=dev)
    rs = torch.empty(x.shape[0], dtype=torch.float32, device=dev)
    K.rot_q8_1024(to_gpu(x, dev), None, None, a8, rs)
    y = torch.empty(x.shape[0], qw.shape[0], dtype=torch.float16, device=dev)
    K.gemm_s8(a8, to_gpu(qw, dev), rs, to_gpu(ws, dev), to_gpu(b, dev), y, K.EPI_BIAS_F16, variant, None, None, 1.0)
    torch.cuda.synchronize()
    q0, s0 = OR.rot_q8_1024(x)
    assert_codes_equal((a8.cpu().numpy(), rs.cpu().numpy()), (q0, s0), "config-1 rotation")
    want = OG.gemm_s8(q0, qw, s0, ws, b, OG.EPI_BIAS_F16)
    got = y.cpu().numpy()
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    assert bad.size == 0, f"{len(bad)} outputs differ, first at {bad[:4].tolist()}"


@pytest.mark.parametrize("variant", GEMM_VARIANTS)
@pytest.mark.parametrize("rope_len", [1, 5, 8, 65, 200])
def test_gemm_s8_qkv_short_rope_tables(dev, rng, rope_len, variant):
    # RoPE table row m % rope_len for tables shorter than a wave's rows (several wraps inside one output block), of a
    # length below the rows per store pass (1, 5), equal to it (8) and odd; 600 rows leave a partial row tile and the
    # persistent variant's split-K rows.
    M, N, K = 600, 3072, 128
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    cos = rng.uniform(-1, 1, (rope_len, 32)).astype(np.float32)
    sin = rng.uniform(-1, 1, (rope_len, 32)).astype(np.float32)
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_QKV_ROPE, variant, rope=(cos, sin), q_scale=OM.Q_SCALE)
    want = OG.gemm_s8(a, w, rs, cs, bias, OG.EPI_QKV_ROPE, rope_cos=cos, rope_sin=sin, q_scale=OM.Q_SCALE)
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    assert bad.size == 0, f"rope_len {rope_len}: {len(bad)} mismatches, first at {bad[:4].tolist()}"


# More 256 x 256 tiles than an MI355X holds workgroups (256): the persistent variant streams several tiles per
# workgroup, its K ring running across tile boundaries, and takes the partial row tile last.
MULTI_TILE_SHAPES = [(4100, 4096, 256), (32800, 1024, 128), (6000, 3072, 384)]


@pytest.mark.parametrize(("M", "N", "K"), MULTI_TILE_SHAPES)
def test_gemm_s8_persistent_multi_tile_int32_bit_exact(dev, rng, M, N, K):
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_I32, PERSISTENT)
    want = OG.gemm_s8_i32(a, w)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"


@pytest.mark.parametrize("epi", [OG.EPI_BIAS_F16, OG.EPI_RESIDUAL, OG.EPI_QKV_ROPE, OG.EPI_SWIGLU])
def test_gemm_s8_persistent_multi_tile_epilogues(dev, rng, epi):
    M, N, K = {OG.EPI_QKV_ROPE: (6000, 3072, 256), OG.EPI_SWIGLU: (4100, 5632, 256)}.get(epi, (32800, 1024, 128))
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    kw, out, rope = {}, None, None
    if epi == OG.EPI_RESIDUAL:
        out = rng.standard_normal((M, N)).astype(np.float16)
        kw["residual"] = out
    if epi == OG.EPI_QKV_ROPE:
        rope = OM.eva02_rope_tables(32, 16)
        kw.update(rope_cos=rope[0], rope_sin=rope[1], q_scale=OM.Q_SCALE)
    got = run_gemm(dev, a, w, rs, cs, bias, epi, PERSISTENT, out=out, rope=rope, q_scale=kw.get("q_scale", 1.0))
    want = OG.gemm_s8(a, w, rs, cs, bias, epi, **kw)
    if epi == OG.EPI_SWIGLU:
        assert_within_one_fp16_ulp(got, want, "SwiGLU epilogue, persistent variant")
        return
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"


def test_gemm_s8_swiglu_saturating_gates(dev, rng):
    """Gates from -100 to 100: silu's limits (0 below, identity above) and the transition, within one fp16 ulp."""
    M, N, K = 257, 512, 64
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    rs[:] = np.float32(1.0)
    cs[:] = np.float32(1.0 / (64 * 127 * 127) * 100)  # |y| up to ~100
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_SWIGLU, 0)
    want = OG.gemm_s8(a, w, rs, cs, bias, OG.EPI_SWIGLU)
    assert_within_one_fp16_ulp(got, want, "saturating SwiGLU")


def assert_gelu_close(got: np.ndarray, want: np.ndarray, what: str) -> None:
    """Within one fp16 ulp of the oracle's float32 tanh form, or 1e-6 absolute: for negative y that form cancels
    (1 + tanh(u) for tanh near -1) and is itself off by up to ~5e-7 from the exact value, which the kernel's
    y / (1 + e^(-2u)) form tracks."""
    g, w = got.astype(np.float32), want.astype(np.float32)
    ulp = np.maximum(np.spacing(np.abs(want)), np.spacing(np.abs(got))).astype(np.float32)
    bad = np.argwhere(~(np.abs(g - w) <= np.maximum(ulp, np.float32(1e-6))))
    assert bad.size == 0, f"{what}: {len(bad)} values off, first {bad[:4].tolist()}: {g[tuple(bad[0])]} vs {w[tuple(bad[0])]}"


def test_gemm_s8_gelu_epilogue(dev, rng):
    M, N, K = 513, 4736, 1024
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_GELU_F16, 0)
    want = OG.gemm_s8(a, w, rs, cs, bias, OG.EPI_GELU_F16)
    assert_gelu_close(got, want, "GELU epilogue")


@pytest.mark.parametrize("variant", GEMM_VARIANTS)
def test_gemm_s8_gelu_wide_range(dev, rng, variant):
    """y from about -30 to 30: GELU's limits (-0 below, identity above) and the transition, on every variant."""
    M, N, K = 600, 512, 64
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    rs[:] = np.float32(1.0)
    cs[:] = np.float32(1.0 / (64 * 127 * 127) * 30)  # |y| up to ~30
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_GELU_F16, variant)
    want = OG.gemm_s8(a, w, rs, cs, bias, OG.EPI_GELU_F16)
    assert_gelu_close(got, want, f"GELU over [-30, 30], variant {variant}")


def run_attention(dev, qkv, seq_len):
    from foidfinder_amd import kernels as K

    t = to_gpu(qkv, dev)
    out = torch.empty(qkv.shape[0], qkv.shape[1] // 3, dtype=torch.float16, device=dev)
    K.attention(t, out, seq_len)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# Attention bars: 4e-3 absolute per element, and 2e-3 relative per output row (the L2 norm of one query's 64-value
# output in one head), both against float64 attention on the same fp16 inputs. Expected error: the fp16 output
# rounding (2^-11 = 4.9e-4 relative per element), the fp16 P fed to the PV product (2^-11 relative per weight) and l
# summed from those fp16 p by a packed fp16 tree per 16 keys (a few 2^-11 per half sum, unbiased); measured up to
# 6.5e-4 row-relative (and 2.1e-3 absolute on the peaked-score cases).
ATT_ABS, ATT_ROW_REL = 4e-3, 2e-3


def check_attention(got, want, H):
    """Asserts the attention bars; returns (max abs error, max row-relative error) for the report."""
    assert np.isfinite(got).all()
    err = np.abs(got - want)
    d = (got - want).reshape(got.shape[0], H, 64)
    ref = want.reshape(want.shape[0], H, 64)
    rel = np.linalg.norm(d, axis=2) / np.maximum(np.linalg.norm(ref, axis=2), 1e-30)
    print(f"attention: max abs err {err.max():.3e}, max row-relative err {rel.max():.3e}")
    assert err.max() < ATT_ABS, f"max abs err {err.max()}"
    assert rel.max() < ATT_ROW_REL, f"max row-relative err {rel.max()}"
    return err.max(), rel.max()


def qkv_inputs(rng, S, L, H):
    x = rng.standard_normal((S * L, 3 * H * 64), dtype=np.float32)
    x[:, : H * 64] *= np.float32(OM.Q_SCALE)
    return x.astype(np.float16)


@pytest.mark.parametrize(("S", "L", "H"), [(1, 1, 16), (2, 65, 16), (1, 1025, 16), (2, 1025, 12), (1, 577, 16), (3, 128, 2)])
def test_attention_matches_float64(dev, rng, S, L, H):
    qkv = qkv_inputs(rng, S, L, H)
    got = run_attention(dev, qkv, L).astype(np.float64)
    want = OA.attention(qkv, L, out_dtype=np.float64)
    check_attention(got, want, H)


# Short last query blocks (at most two 32-query units past the last full 128-query block): two units are split over
# two waves each by key half, one unit over all four waves by key half and tile parity, and the partial results are
# merged. Covered: one or two units, the last tile's second key half empty (L mod 64 in 1..32) or not, a single key
# tile, waves that compute no tile at all (L 32, 2, 65: the odd tiles or the last second half hold no key), and
# PixAI's window (576) and grid (5184) lengths.
@pytest.mark.parametrize(("S", "L", "H"), [(2, 161, 4), (3, 33, 2), (2, 32, 2), (1, 168, 3), (4, 576, 2),
                                           (1, 5184, 1), (2, 2, 2), (1, 190, 2), (2, 129, 2), (2, 65, 3), (1, 97, 2),
                                           (1, 257, 2)])
def test_attention_split_tail_blocks(dev, rng, S, L, H):
    qkv = qkv_inputs(rng, S, L, H)
    got = run_attention(dev, qkv, L).astype(np.float64)
    want = OA.attention(qkv, L, out_dtype=np.float64)
    check_attention(got, want, H)


# The cases above launch at most as many 64-query blocks as an MI355X holds workgroups resident (1024), so they run as
# 64-query blocks, each 32-query unit over two waves by key half. These grids (PixAI's 9 windows of 576 tokens x 16
# heads: 1296 blocks of 64 queries; 2048 and 1728 blocks of 128) run as 128-query blocks, one unit per wave, with the
# split tail blocks at their ends.
@pytest.mark.parametrize(("S", "L", "H"), [(9, 576, 16), (64, 161, 16), (12, 1025, 16)])
def test_attention_wider_blocks_on_larger_grids(dev, rng, S, L, H):
    qkv = qkv_inputs(rng, S, L, H)
    got = run_attention(dev, qkv, L).astype(np.float64)
    want = OA.attention(qkv, L, out_dtype=np.float64)
    check_attention(got, want, H)


@pytest.mark.parametrize(("gain", "ramp"), [(8.0, 3.0), (30.0, 0.0), (4.0, 12.0)])
def test_attention_peaked_and_rising_scores(dev, rng, gain, ramp):
    """Scores of tens to hundreds (base 2) whose maxima grow along the keys: the running maximum must be raised on
    later key tiles, not only set on the first one."""
    S, L, H = 2, 1025, 4
    qkv = qkv_inputs(rng, S, L, H).astype(np.float32)
    qkv[:, : H * 64] *= np.float32(gain)
    pos = np.tile(np.arange(L, dtype=np.float32), S)
    qkv[:, H * 64 : 2 * H * 64] *= (1.0 + ramp * pos / L)[:, None]
    qkv = qkv.astype(np.float16)
    got = run_attention(dev, qkv, L).astype(np.float64)
    want = OA.attention(qkv, L, out_dtype=np.float64)
    check_attention(got, want, H)


def test_attention_identical_keys_give_mean_of_values(dev, rng):
    S, L, H = 1, 200, 4
    qkv = qkv_inputs(rng, S, L, H)
    qkv[:, H * 64 : 2 * H * 64] = qkv[0, H * 64 : 2 * H * 64]  # every key equal
    got = run_attention(dev, qkv, L).astype(np.float64)
    v = qkv[:, 2 * H * 64 :].astype(np.float64)
    np.testing.assert_allclose(got, np.broadcast_to(v.mean(0), got.shape), atol=2e-3)


def test_layer_norm2_matches_two_float_layer_norms(dev, rng):
    """ff_layer_norm2 against two float64 LayerNorms with the fp16 rounding between them: the 8-byte-vector kernel
    (C % 256 == 0 up to 1024, also with more rows than its grid has waves) and the per-column kernel (2048, 64, and
    768 on a tensor that starts 2 bytes past an 8-byte boundary)."""
    from foidfinder_amd import kernels as K

    for T, C, shift in ((300, 768, 0), (8300, 768, 0), (7, 1024, 0), (3, 256, 0), (5, 2048, 0), (1, 64, 0),
                        (9, 768, 1)):
        x = (rng.standard_normal((T, C)) * 3 + 0.5).astype(np.float16)
        g1, b1, g2, b2 = ((1 + 0.1 * rng.standard_normal(C)).astype(np.float16), (0.1 * rng.standard_normal(C)).astype(np.float16),
                          (1 + 0.1 * rng.standard_normal(C)).astype(np.float16), (0.1 * rng.standard_normal(C)).astype(np.float16))
        xd = torch.empty(T * C + shift, dtype=torch.float16, device=dev)[shift:].view(T, C)
        xd.copy_(to_gpu(x, dev))
        out = torch.empty(T, C, dtype=torch.float16, device=dev)
        K.layer_norm2(xd, *(to_gpu(a, dev) for a in (g1, b1, g2, b2)), 1e-6, out)
        torch.cuda.synchronize()

        def ln(v, g, b):
            v = v.astype(np.float64)
            m = v.mean(-1, keepdims=True)
            return (v - m) / np.sqrt(((v - m) ** 2).mean(-1, keepdims=True) + 1e-6) * g.astype(np.float64) + b.astype(np.float64)

        want = ln(ln(x, g1, b1).astype(np.float16), g2, b2)
        assert np.abs(out.cpu().numpy().astype(np.float64) - want).max() < 8e-3 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize(("B", "N", "G", "M", "shared_c", "offset"),
                         [(2, 1025, 16, 6, True, 0), (3, 65, 16, 18, False, 0), (1, 31, 4, 18, False, 0),
                          (2, 96, 16, 18, True, 0),
                          # the pair loops' bounds (G = 64 at M = 6 and G = 27 at M = 18 fill the kernel's pairs per
                          # thread), G*M not a multiple of 8 (2-byte logit copies), and a logits view one fp16 element
                          # past a 16-byte boundary (2-byte copies although G*M % 8 == 0)
                          (1, 40, 64, 6, True, 0), (2, 33, 27, 18, False, 0), (1, 50, 3, 6, True, 0),
                          (2, 70, 16, 6, False, 1)])
def test_slot_weights_matches_float(dev, rng, B, N, G, M, shared_c, offset):
    """ff_slot_weights: softmax over the M queries times sigmoid(logit + bias), transposed, and the per-block sums
    over the tokens (summed over blocks: each query's mass), against float64."""
    from foidfinder_amd import kernels as K

    logits = (rng.standard_normal((B, N, G * M)) * 3).astype(np.float16)
    lg = torch.empty(B * N * G * M + offset, dtype=torch.float16, device=dev)[offset:].view(B, N, G * M)
    lg.copy_(to_gpu(logits, dev))
    c = (rng.standard_normal(G * M if shared_c else (B, G * M)) * 0.5).astype(np.float32)
    bias = (-2 + 0.3 * rng.standard_normal(M)).astype(np.float32)
    nblk = K.slot_weights_blocks(N)
    a_t = torch.full((B, G * M, N), 7.0, dtype=torch.float16, device=dev)
    partial = torch.empty(B, nblk, G * M, dtype=torch.float32, device=dev)
    K.slot_weights(lg, to_gpu(c, dev), to_gpu(bias, dev), G, a_t, partial)
    torch.cuda.synchronize()
    l = logits.astype(np.float64).reshape(B, N, G, M) + c.astype(np.float64).reshape(-1, 1, G, M)
    e = np.exp(l - l.max(-1, keepdims=True))
    w = e / e.sum(-1, keepdims=True) / (1 + np.exp(-(l + bias.astype(np.float64))))
    want = w.reshape(B, N, G * M).transpose(0, 2, 1)
    assert np.abs(a_t.cpu().numpy().astype(np.float64) - want).max() < 1e-3
    mass = partial.sum(1).cpu().numpy().astype(np.float64)
    assert np.abs(mass - want.sum(-1)).max() < 1e-4 * N


def test_empty_inputs_are_no_ops(dev):
    """Zero tokens (or zero images) through every op: nothing is launched and the output buffers keep their bytes."""
    from foidfinder_amd import kernels as K

    f16, i8, f32 = torch.float16, torch.int8, torch.float32
    x = torch.empty(0, 1024, dtype=f16, device=dev)
    a8 = torch.empty(0, 1024, dtype=i8, device=dev)
    rs = torch.empty(0, dtype=f32, device=dev)
    K.rot_q8_1024(x, None, None, a8, rs)
    K.rot_q8_h128(torch.empty(0, 2816, dtype=f16, device=dev), torch.empty(0, 2816, dtype=i8, device=dev), rs)
    w = torch.ones(256, 1024, dtype=i8, device=dev)
    ones = torch.ones(256, dtype=f32, device=dev)
    K.gemm_s8(a8, w, rs, ones, ones, torch.empty(0, 256, dtype=f16, device=dev), K.EPI_BIAS_F16, 0, None, None, 1.0)
    K.attention(torch.empty(0, 3 * 1024, dtype=f16, device=dev), torch.empty(0, 1024, dtype=f16, device=dev), 1025)
    g = torch.ones(768, dtype=f16, device=dev)
    K.layer_norm2(torch.empty(0, 768, dtype=f16, device=dev), g, g, g, g, 1e-6, torch.empty(0, 768, dtype=f16, device=dev))
    sentinel = torch.full((0, 96, 10), 7.0, dtype=f16, device=dev)
    K.slot_weights(torch.empty(0, 10, 96, dtype=f16, device=dev), torch.zeros(96, dtype=f32, device=dev),
                   torch.zeros(6, dtype=f32, device=dev), 16, sentinel,
                   torch.empty(0, K.slot_weights_blocks(10), 96, dtype=f32, device=dev))
    # a real launch after the no-ops still works (nothing was left half-launched)
    y = torch.randn(4, 1024, device=dev).half()
    out = torch.empty(4, 1024, dtype=i8, device=dev)
    r4 = torch.empty(4, dtype=f32, device=dev)
    K.rot_q8_1024(y, None, None, out, r4)
    torch.cuda.synchronize()
    assert (r4 > 0).all()


# The persistent variant computes the rows past its last whole 256-row tile as split-K blocks inside its launch,
# before its tiles (32 x 32 output blocks, K in 128-byte chunks over 8 waves): tails of 1 .. 255 rows, a last column
# block of 16 columns, fewer K chunks than waves and more, and more tail blocks than workgroups (767 x 5632).
@pytest.mark.parametrize(("M", "N", "K"), [(511, 272, 384), (257, 96, 128), (288, 3072, 2816), (767, 5632, 1024)])
def test_gemm_s8_tail_rows_int32_bit_exact(dev, rng, M, N, K):
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    got = run_gemm(dev, a, w, rs, cs, bias, OG.EPI_I32, PERSISTENT)
    want = OG.gemm_s8_i32(a, w)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"


@pytest.mark.parametrize("epi", [OG.EPI_BIAS_F16, OG.EPI_RESIDUAL, OG.EPI_QKV_ROPE, OG.EPI_SWIGLU])
def test_gemm_s8_tail_rows_epilogues(dev, rng, epi):
    M, N, K = {OG.EPI_QKV_ROPE: (383, 3072, 256), OG.EPI_SWIGLU: (300, 5632, 384)}.get(epi, (511, 272, 384))
    a, w, rs, cs, bias = gemm_inputs(rng, M, N, K)
    kw, out, rope = {}, None, None
    if epi == OG.EPI_RESIDUAL:
        out = rng.standard_normal((M, N)).astype(np.float16)
        kw["residual"] = out
    if epi == OG.EPI_QKV_ROPE:
        rope = OM.eva02_rope_tables(32, 16)
        kw.update(rope_cos=rope[0], rope_sin=rope[1], q_scale=OM.Q_SCALE)
    got = run_gemm(dev, a, w, rs, cs, bias, epi, PERSISTENT, out=out, rope=rope, q_scale=kw.get("q_scale", 1.0))
    want = OG.gemm_s8(a, w, rs, cs, bias, epi, **kw)
    if epi == OG.EPI_SWIGLU:
        assert_within_one_fp16_ulp(got, want, "SwiGLU epilogue, tail rows")
        return
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"
