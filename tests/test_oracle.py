"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

The reference's tests hold no golden vectors or known-answer tests for this path (its only pin is an end-to-end
tolerance against the official checkpoint, which is not available offline). Each function is therefore checked
against what the mathematics fixes: closed forms, invariants, special cases and brute force on tiny inputs, chosen
so that a plausible mistake (a dropped term, a wrong sign or index, a transposed operand, a wrong divisor) fails.
The last tests plant such mistakes in copies of the oracle and show the checks catch them.
"""

from __future__ import annotations

import itertools
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import attention as OA
from oracle import gemm as OG
from oracle import model as OM
from oracle import rotq8 as OR

F32 = np.float32


# ---------------- Hadamard and weight quantization ----------------


@pytest.mark.parametrize("n", [2, 8, 128, 1024])
def test_hadamard_closed_form(n):
    h = OM.hadamard(n)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    pop = np.vectorize(lambda v: bin(v).count("1"))(i & j)
    np.testing.assert_array_equal(h, np.where(pop % 2 == 0, 1.0, -1.0) / math.sqrt(n))
    np.testing.assert_allclose(h @ h, np.eye(n), atol=1e-12)
    np.testing.assert_allclose(h[:, 0], np.full(n, 1 / math.sqrt(n)))


def brute_quant_row(w: np.ndarray) -> tuple[np.ndarray, np.float32]:
    scale = F32(max(F32(np.abs(w).max()), F32(1e-12)) / F32(127))
    codes = []
    for v in w:
        t = F32(v) / scale  # the reference divides (engine.py:40)
        cands = np.arange(-127, 128)
        d = np.abs(cands - np.float64(t))
        best = cands[d == d.min()]
        codes.append(best[best % 2 == 0][0] if len(best) > 1 else best[0])  # ties to even
    return np.array(codes, np.int8), scale


@pytest.mark.parametrize("block,k", [(1024, 1024), (128, 640), (128, 2816)])
def test_rotate_rows64_is_the_block_hadamard_product(rng, block, k):
    """The weight rotation's FWHT equals W @ blockdiag(H_block) formed by a float64 product, to float64 rounding; a
    planted sign error in one butterfly stage is far outside that bound."""
    w = (rng.standard_normal((48, k)) * 0.02).astype(F32)
    got = OM.rotate_rows64(w, block)
    want = w.astype(np.float64) @ OM.block_hadamard(k, block)
    assert np.abs(got - want).max() <= 1e-13 * np.abs(want).max()
    v = w.astype(np.float64).reshape(48, k // block, block // 2, 2)
    bad = np.stack((v[..., 0] + v[..., 1], v[..., 1] - v[..., 0]), -1).reshape(48, k // block, block)  # wrong sign
    bad = OM.rotate_rows64(bad.reshape(48, k), block)  # (stage 0 done twice: not the transform either)
    assert np.abs(bad - want).max() > 1e-3 * np.abs(want).max()


def test_quantize_rows_int8_brute_force(rng):
    w = rng.standard_normal((7, 33)).astype(F32) * 0.02
    w[1] = 0.0
    w[2, :5] = [127.0, 2.5, -3.5, 0.5, -0.5]  # exact ties at scale 1
    w[2, 5:] = 0.0
    q, s = OM.quantize_rows_int8(w)
    for r in range(w.shape[0]):
        bq, bs = brute_quant_row(w[r])
        np.testing.assert_array_equal(q[r], bq)
        assert s[r] == bs
    np.testing.assert_array_equal(q[2, :5], [127, 2, -4, 0, 0])


# ---------------- rotation + quantization ----------------


def test_fwht_matches_hadamard_product(rng):
    x = rng.standard_normal((16, 1024)).astype(F32)
    got = OR.fwht_rows(x, OR.STAGES_1024) * F32(1 / 32)
    want = x.astype(np.float64) @ OM.hadamard(1024)
    assert np.abs(got - want).max() < 1e-5 * np.abs(want).max()


def test_fwht_stage_order_changes_only_rounding(rng):
    x = rng.standard_normal((64, 1024)).astype(F32)
    a = OR.fwht_rows(x, OR.STAGES_1024)
    b = OR.fwht_rows(x, tuple(range(10)))
    assert not np.array_equal(a, b)  # the order is observable in the last bits (why kernels must follow it)
    assert np.abs(a - b).max() < 1e-5 * np.abs(a).max()


def test_quant_rows_ties_and_clamp():
    v = np.array([[127.0, 0.5, 1.5, -2.5, -127.0, 126.5, 3.0]], F32)
    q, s = OR.quant_rows(v)
    assert s[0] == F32(1.0)
    np.testing.assert_array_equal(q[0], [127, 0, 2, -2, -127, 126, 3])


def test_rot_q8_1024_reconstructs_rotation(rng):
    x = rng.standard_normal((32, 1024)).astype(np.float16)
    x[:, rng.choice(1024, 10, replace=False)] *= np.float16(20)
    q, s = OR.rot_q8_1024(x)
    exact = x.astype(np.float64) @ OM.hadamard(1024)
    err = np.abs(q.astype(np.float64) * s[:, None] - exact) / s[:, None]
    assert err.max() <= 0.5 + 1e-3
    assert (np.abs(q) == 127).any(axis=1).all()  # the row maximum maps to +-127


def test_rot_q8_1024_special_rows():
    x = np.zeros((2, 1024), np.float16)
    x[1, 0] = 3.0
    q, s = OR.rot_q8_1024(x)
    assert (q[0] == 0).all() and s[0] == F32(1e-12) / F32(127)
    assert (np.abs(q[1].astype(int)) == 127).all()  # a one-hot row spreads evenly: H e0 = 1/32
    assert (q[1] > 0).all()


def test_layer_norm_1024_matches_float64(rng):
    x = (rng.standard_normal((8, 1024)) * 3 + 1).astype(F32)
    g = (1 + 0.1 * rng.standard_normal(1024)).astype(F32)
    b = (0.1 * rng.standard_normal(1024)).astype(F32)
    got = OR.layer_norm_1024(x, g, b, 1e-5)
    want = OM.layer_norm(x, g, b, 1e-5)
    assert np.abs(got - want).max() < 2e-5  # a 1/1023 divisor or a dropped eps would be ~5e-4 off


def test_rot_q8_1024_layernorm_reconstructs(rng):
    x = rng.standard_normal((16, 1024)).astype(np.float16)
    g = (1 + 0.02 * rng.standard_normal(1024)).astype(F32)
    b = (0.02 * rng.standard_normal(1024)).astype(F32)
    q, s = OR.rot_q8_1024(x, g, b, 1e-6)
    want = OM.layer_norm(x.astype(F32), g, b, 1e-6) @ OM.hadamard(1024)
    assert (np.abs(q * s[:, None] - want) / s[:, None]).max() <= 0.5 + 1e-2


def test_rot_q8_h128_reconstructs_block_rotation(rng):
    x = rng.standard_normal((8, 640)).astype(np.float16)
    q, s = OR.rot_q8_h128(x)
    want = x.astype(np.float64) @ OM.block_hadamard(640, 128)
    assert (np.abs(q * s[:, None] - want) / s[:, None]).max() <= 0.5 + 1e-3


def test_rot_q8_h128_layernorm_over_real_columns(rng):
    C, cr = 2816, 2730
    x = rng.standard_normal((4, C)).astype(np.float16)
    x[:, cr:] = np.float16(7.0)  # padding content must be ignored
    g = (1 + 0.02 * rng.standard_normal(cr)).astype(F32)
    b = (0.02 * rng.standard_normal(cr)).astype(F32)
    y = OR.layer_norm_h128(x.astype(F32), cr, g, b, 1e-6)
    assert (y[:, cr:] == 0).all()
    np.testing.assert_allclose(y[:, :cr], OM.layer_norm(x[:, :cr].astype(F32), g, b, 1e-6), atol=2e-5)
    q, s = OR.rot_q8_h128(x, cr, g, b, 1e-6)
    full = np.zeros((4, C))
    full[:, :cr] = OM.layer_norm(x[:, :cr].astype(F32), g, b, 1e-6)
    want = full @ OM.block_hadamard(C, 128)
    assert (np.abs(q * s[:, None] - want) / s[:, None]).max() <= 0.5 + 1e-2


def test_outlier_channel_is_spread(rng):
    x = rng.standard_normal((64, 1024)).astype(np.float16)
    x[:, 3] = np.float16(200.0)
    q, s = OR.rot_q8_1024(x)
    # without rotation the scale would be set by the outlier (200/127) and N(0,1) entries would mostly quantize to
    # 0 or +-1; after the rotation every channel carries ~200/32 and the scale is ~10x smaller
    assert s.max() < 200 / 127 / 4


# ---------------- GEMM and epilogues ----------------


@pytest.mark.parametrize(("M", "N", "K"), [(1, 1, 1), (3, 5, 7), (17, 16, 64), (9, 48, 130)])
def test_gemm_s8_i32_brute_force(rng, M, N, K):
    a = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    want = np.zeros((M, N), np.int64)
    for m, n in itertools.product(range(M), range(N)):
        want[m, n] = int(np.dot(a[m].astype(np.int64), w[n].astype(np.int64)))
    np.testing.assert_array_equal(OG.gemm_s8_i32(a, w), want)


def test_gemm_s8_i32_extremes():
    K = 2816
    a = np.full((2, K), -127, np.int8)
    w = np.full((3, K), -127, np.int8)
    assert (OG.gemm_s8_i32(a, w) == 127 * 127 * K).all()


def test_dequant_matches_float64(rng):
    acc = rng.integers(-2**24, 2**24, (8, 16)).astype(np.int32)
    rs = rng.random(8).astype(F32)
    cs = rng.random(16).astype(F32)
    b = rng.standard_normal(16).astype(F32)
    got = OG.dequant(acc, rs, cs, b)
    want = acc.astype(np.float64) * rs[:, None] * cs[None, :] + b[None, :]
    assert np.abs(got - want).max() <= 4 * np.finfo(F32).eps * np.abs(want).max()


def _round_f32(x: Fraction) -> np.float32:
    """Correct round-to-nearest-even of a rational to float32 (normal and subnormal range), by integer arithmetic."""
    if x == 0:
        return F32(0.0)
    sign, x = (-1 if x < 0 else 1), abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    e = max(e, -126)
    q = x / Fraction(2) ** (e - 23)
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return F32(sign * n * 2.0 ** (e - 23))


def test_fma32_is_single_rounding(rng):
    n = 3000
    a = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 1e3], n)).astype(F32)
    b = rng.standard_normal(n).astype(F32)
    c = (rng.standard_normal(n) * rng.choice([1e-6, 1.0, 1e4], n)).astype(F32)
    got = OG.fma32(a, b, c)
    want = np.array([_round_f32(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z))) for x, y, z in zip(a, b, c)])
    assert np.array_equal(got.view(np.uint32), want.astype(F32).view(np.uint32))


def test_fma32_breaks_ties_by_the_addend():
    """(1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 is halfway between two float32 values: a tiny addend must decide the rounding
    (a float64 sum rounded to float32 rounds twice and ties to even, the planted mistake this guards against)."""
    x = np.array([1 + 2.0**-12], F32)
    up, down = F32(1 + 2.0**-11 + 2.0**-23), F32(1 + 2.0**-11)
    assert OG.fma32(x, x, np.array([2.0**-60], F32))[0] == up
    assert OG.fma32(x, x, np.array([-(2.0**-60)], F32))[0] == down
    assert OG.fma32(x, x, np.array([0.0], F32))[0] == down  # exact tie: to even
    assert F32(np.float64(x[0]) * np.float64(x[0]) + 2.0**-60) == down  # the double-rounded value is wrong


def test_dequant_is_fused(rng):
    acc = rng.integers(-2**20, 2**20, (4, 8)).astype(np.int32)
    rs, cs, b = rng.random(4).astype(F32), rng.random(8).astype(F32), rng.standard_normal(8).astype(F32)
    got = OG.dequant(acc, rs, cs, b)
    t = acc.astype(F32) * rs[:, None]
    for m in range(4):
        for n in range(8):
            assert got[m, n] == _round_f32(Fraction(float(t[m, n])) * Fraction(float(cs[n])) + Fraction(float(b[n])))


def test_qkv_rope_epilogue_closed_forms(rng):
    M, C = 5, 128
    acc = rng.integers(-1000, 1000, (M, 3 * C)).astype(np.int32)
    rs, cs = np.full(M, F32(0.01)), np.full(3 * C, F32(0.01))
    b = np.zeros(3 * C, F32)
    cos, sin = OM.eva02_rope_tables(2, 16)  # 5 tokens: cls + 2x2
    y = OG.epilogue(acc, rs, cs, b, OG.EPI_QKV_ROPE, rope_cos=cos, rope_sin=sin, q_scale=0.5).astype(np.float64)
    plain = OG.dequant(acc, rs, cs, b).astype(np.float64)
    np.testing.assert_allclose(y[0, :C], plain[0, :C] * 0.5, rtol=1e-3)  # cls row: identity rotation, q scaled
    np.testing.assert_allclose(y[0, C:], plain[0, C:], rtol=1e-3)
    np.testing.assert_allclose(y[:, 2 * C :], plain[:, 2 * C :], rtol=1e-3)  # v untouched
    n_y = np.hypot(y[:, C : 2 * C : 2], y[:, C + 1 : 2 * C : 2])  # k pairs keep their norm
    n_p = np.hypot(plain[:, C : 2 * C : 2], plain[:, C + 1 : 2 * C : 2])
    np.testing.assert_allclose(n_y, n_p, rtol=2e-3, atol=1e-3)
    # token 4 = grid (1, 1): pair 0 angle = 1 * 16/2 * band0 = 8 rad
    t, p = 4, 0
    ang = 8.0
    y0, y1 = plain[t, C + 2 * p], plain[t, C + 2 * p + 1]
    np.testing.assert_allclose(y[t, C + 2 * p], y0 * math.cos(ang) - y1 * math.sin(ang), rtol=2e-3, atol=1e-3)


def test_residual_epilogue_is_fp16_add(rng):
    acc = rng.integers(-5000, 5000, (4, 16)).astype(np.int32)
    rs, cs, b = np.full(4, F32(1e-3)), np.full(16, F32(0.5)), np.zeros(16, F32)
    x = rng.standard_normal((4, 16)).astype(np.float16)
    got = OG.epilogue(acc, rs, cs, b, OG.EPI_RESIDUAL, residual=x)
    np.testing.assert_array_equal(got, OG.dequant(acc, rs, cs, b).astype(np.float16) + x)


def test_exp_cw_accuracy():
    x = np.linspace(-80, 80, 200001).astype(F32)
    rel = np.abs(OG.exp_cw(x).astype(np.float64) / np.exp(x.astype(np.float64)) - 1)
    assert rel.max() < 3e-7
    assert OG.exp_cw(np.array([0.0], F32))[0] == 1.0


def test_swiglu_epilogue(rng):
    acc = rng.integers(-3000, 3000, (3, 8)).astype(np.int32)
    acc[:, 6:] = 0  # a zero-padded (gate, value) pair
    rs, cs, b = np.full(3, F32(1e-3)), np.full(8, F32(1.0)), np.zeros(8, F32)
    got = OG.epilogue(acc, rs, cs, b, OG.EPI_SWIGLU).astype(np.float64)
    y = OG.dequant(acc, rs, cs, b).astype(np.float64)
    g, v = y[:, 0::2], y[:, 1::2]
    np.testing.assert_allclose(got, g / (1 + np.exp(-g)) * v, rtol=2e-3, atol=1e-6)
    assert (got[:, 3] == 0).all() and got.shape == (3, 4)


def test_gelu_epilogue():
    y = np.array([-3.0, -1.0, 0.0, 1.0, 3.0], F32)
    want = 0.5 * y * (1 + np.tanh(math.sqrt(2 / math.pi) * (y + 0.044715 * y**3)))
    np.testing.assert_allclose(OG.gelu_tanh(y), want, rtol=1e-5, atol=1e-7)


# ---------------- attention ----------------


def brute_attention(qkv, L):
    T, W = qkv.shape
    C = W // 3
    out = np.zeros((T, C))
    for s in range(T // L):
        for h in range(C // 64):
            q = qkv[s * L : (s + 1) * L, h * 64 : (h + 1) * 64].astype(np.float64)
            k = qkv[s * L : (s + 1) * L, C + h * 64 : C + (h + 1) * 64].astype(np.float64)
            v = qkv[s * L : (s + 1) * L, 2 * C + h * 64 : 2 * C + (h + 1) * 64].astype(np.float64)
            for i in range(L):
                logits = [2.0 ** float(q[i] @ k[j]) for j in range(L)]
                out[s * L + i, h * 64 : (h + 1) * 64] = sum(p * v[j] for j, p in enumerate(logits)) / sum(logits)
    return out


def test_attention_brute_force(rng):
    qkv = (rng.standard_normal((2 * 5, 3 * 128)) * 0.3).astype(np.float16)
    np.testing.assert_allclose(OA.attention(qkv, 5, out_dtype=np.float64), brute_attention(qkv, 5), atol=1e-12)


def test_attention_closed_forms(rng):
    L, C = 9, 64
    qkv = rng.standard_normal((L, 3 * C)).astype(np.float16)
    same_k = qkv.copy()
    same_k[:, C : 2 * C] = same_k[0, C : 2 * C]
    np.testing.assert_allclose(OA.attention(same_k, L, out_dtype=np.float64),
                               np.broadcast_to(same_k[:, 2 * C :].astype(np.float64).mean(0), (L, C)), atol=1e-12)
    dom = qkv.copy()
    dom[:, :C] = np.float16(0)
    dom[:, 0] = np.float16(1.0)
    dom[:, C : 2 * C] = np.float16(0)
    dom[4, C] = np.float16(200.0)  # key 4 dominates every query's logits
    np.testing.assert_allclose(OA.attention(dom, L, out_dtype=np.float64),
                               np.broadcast_to(dom[4, 2 * C :].astype(np.float64), (L, C)), atol=1e-12)
    shifted = qkv.astype(np.float64)
    shifted[:, C : 2 * C] += shifted[0, C : 2 * C]  # adds q_i . k_0 to every logit of query i: softmax unchanged
    np.testing.assert_allclose(OA.attention(shifted, L, out_dtype=np.float64),
                               OA.attention(qkv.astype(np.float64), L, out_dtype=np.float64), atol=1e-9)


# ---------------- model pieces ----------------


def test_rope_tables_closed_form():
    cos, sin = OM.eva02_rope_tables(32, 16)
    assert cos.shape == (1025, 32) and (cos[0] == 1).all() and (sin[0] == 0).all()
    band = 1.0 / 10000 ** (np.arange(16) / 16)
    r, c = 5, 7  # token 1 + 5 * 32 + 7
    np.testing.assert_allclose(cos[1 + r * 32 + c, :16], np.cos(r / 32 * 16 * band), atol=2e-6)
    np.testing.assert_allclose(sin[1 + r * 32 + c, 16:], np.sin(c / 32 * 16 * band), atol=2e-6)
    # every entry against float64 angles: the float32 recipe stays within a few float32 roundings of the angle
    # (|angle| <= 16), never a wrong band or position (a planted swap of rows and columns is off by O(1))
    t = np.arange(32) / 32 * 16
    ang = np.concatenate([np.repeat(t, 32)[:, None] * band, np.tile(t, 32)[:, None] * band], axis=1)
    assert np.abs(cos[1:] - np.cos(ang)).max() < 4e-6 and np.abs(sin[1:] - np.sin(ang)).max() < 4e-6
    swapped = np.concatenate([ang[:, 16:], ang[:, :16]], axis=1)
    assert np.abs(cos[1:] - np.cos(swapped)).max() > 0.5


def test_rope_tables_follow_the_float32_recipe():
    """The tables are the reference's float32 computation (mlx/haruka.py:26-32) step for step, not a float64 one
    rounded once: the two differ in the last bits of thousands of entries at grid 32 / ref 16."""
    cos, sin = OM.eva02_rope_tables(32, 16)
    band = 1.0 / 10000 ** (np.arange(16) / 16)
    t = np.arange(32) / 32 * 16
    ang = np.concatenate([np.repeat(t, 32)[:, None] * band, np.tile(t, 32)[:, None] * band], axis=1)
    assert (cos[1:] != np.cos(ang).astype(F32)).sum() > 1000
    b32 = F32(1.0) / (F32(10000.0) ** (np.arange(16, dtype=F32) / F32(16)))
    t32 = np.arange(32, dtype=F32) / F32(32) * F32(16)
    a32 = (t32[5] * b32).astype(F32)
    np.testing.assert_array_equal(cos[1 + 5 * 32 + 7, :16], np.cos(a32))


def test_interleave_swiglu_layout(rng):
    w = rng.standard_normal((6, 4)).astype(F32)
    b = np.arange(6, dtype=F32)
    wi, bi = OM.interleave_swiglu(w, b, 3, 4)
    np.testing.assert_array_equal(wi[[0, 2, 4]], w[:3])
    np.testing.assert_array_equal(wi[[1, 3, 5]], w[3:])
    assert (wi[6:] == 0).all() and list(bi) == [0, 3, 1, 4, 2, 5, 0, 0]


def test_rotated_weights_preserve_products(rng):
    """W' = W H and x' = x H give x' W'^T = x W^T (H orthogonal): the rotation never changes the linear map."""
    x = rng.standard_normal((4, 1024))
    w = rng.standard_normal((8, 1024)) * 0.02
    h = OM.hadamard(1024)
    np.testing.assert_allclose((x @ h) @ (w @ h).T, x @ w.T, atol=1e-10)


def test_w8a8_linear_tracks_float(rng):
    """The single W8A8 linear of the plumbing configuration (scaled down) against float64."""
    x, qw, ws, b = OM.w8a8_linear_inputs(m=65, k=1024, n=256, seed=2)
    a8, rs = OR.rot_q8_1024(x)
    y = OG.gemm_s8(a8, qw, rs, ws, b, OG.EPI_BIAS_F16).astype(np.float64)
    w = np.random.default_rng(2)
    ref = x.astype(np.float64) @ (qw.astype(np.float64) * ws[:, None].astype(np.float64) @ OM.hadamard(1024)).T + b
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 0.02, rel


def test_int8_forward_tracks_float_forward():
    cfg = OM.Eva02Config(img_size=56, depth=2, tags=64)
    w = OM.synthetic_weights(cfg, seed=4)
    q = [OM.convert_block(b, cfg) for b in w.blocks]
    images = OM.synthetic_images(2, 56, seed=3)
    p8 = OM.forward_int8(images, w, q)
    pf = OM.forward_float(images, w)
    assert np.abs(p8 - pf).max() < 0.05 and np.abs(p8 - pf).mean() < 0.01


# ---------------- the CPU baseline's PyTorch restatement (oracle/float_torch.py) ----------------


def _float_torch_pair(seed=3):
    """A 2-block EVA02 at 56 px: the engine's float state dict (for float_torch) and the same weights as the numpy
    oracle's FloatWeights."""
    torch = pytest.importorskip("torch")
    from foidfinder_amd.engine import Eva02Config, eva02_rope_tables, synthetic_checkpoint
    from oracle import float_torch as FT

    cfg = Eva02Config(img_size=56, depth=2, tags=64)
    raw = synthetic_checkpoint(cfg, seed=seed)
    n = {k: v.numpy() for k, v in raw.items()}
    w = OM.FloatWeights(cfg=OM.Eva02Config(img_size=56, depth=2, tags=64), patch_w=n["patch_embed.weight"],
                        patch_b=n["patch_embed.bias"], cls=n["cls_token"], pos=n["pos_embed"], norm_w=n["norm.weight"],
                        norm_b=n["norm.bias"], head_w=n["head.weight"], head_b=n["head.bias"])
    names = {"norm1_w": "norm1.weight", "norm1_b": "norm1.bias", "qkv_w": "attn.qkv.weight", "qkv_b": "attn.qkv.bias",
             "proj_w": "attn.proj.weight", "proj_b": "attn.proj.bias", "norm2_w": "norm2.weight",
             "norm2_b": "norm2.bias", "fc1_w": "mlp.fc1.weight", "fc1_b": "mlp.fc1.bias",
             "mlp_norm_w": "mlp.norm.weight", "mlp_norm_b": "mlp.norm.bias", "fc2_w": "mlp.fc2.weight",
             "fc2_b": "mlp.fc2.bias"}
    for i in range(cfg.depth):
        w.blocks.append({k: n[f"blocks.{i}.{v}"] for k, v in names.items()})
    images = OM.synthetic_images(2, 56, seed=5)
    run = lambda: FT.forward_float(torch.from_numpy(images).float(), raw, cfg.depth, cfg.heads, cfg.patch,  # noqa
                                   cfg.hidden, eva02_rope_tables(cfg.grid, cfg.rope_ref), cfg.eps).numpy()
    return run, OM.head_logits(OM.forward_float_x(images, w), w)


def test_float_torch_forward_matches_float64_forward():
    """bench.py's CPU baseline workload: the fp32 PyTorch forward against the numpy float64 forward of the same
    weights (measured max |dlogit| 1.9e-3 at logits up to 3.4: fp32 rounding through two blocks)."""
    run, want = _float_torch_pair()
    got = run()
    assert np.abs(got - want).max() < 5e-3


def test_float_torch_check_catches_a_dropped_rope(monkeypatch):
    pytest.importorskip("torch")
    from oracle import float_torch as FT

    run, want = _float_torch_pair()
    monkeypatch.setattr(FT, "_rope", lambda x, cos, sin: x)
    assert np.abs(run() - want).max() > 5e-3


def test_float_torch_rot_q8_equals_the_oracle(rng):
    """The CPU baseline's rotation + quantization takes the reference's butterfly order and division sequence, so it
    reproduces the oracle's codes and fp32 scales bit for bit (1 % outlier channels x20, the plumbing config's
    activations)."""
    torch = pytest.importorskip("torch")
    from oracle import float_torch as FT

    x = OM.w8a8_linear_inputs(m=257, seed=7)[0]
    codes, scale = FT.rot_q8(torch.from_numpy(x))
    q, s = OR.rot_q8_1024(x)
    assert np.array_equal(codes.numpy().astype(np.int8), q)
    assert np.array_equal(scale.numpy().view(np.uint32), s.view(np.uint32))


def test_float_torch_w8a8_linear_within_one_fp16_ulp():
    """The plumbing config's W8A8 linear at full size (1025 x 1024 -> 3072) on the CPU against the oracle's
    rot_q8_1024 + gemm_s8(EPI_BIAS_F16): identical codes, and the dequant rounds `acc * rs * cs + bias` after each
    operation where the oracle (as the reference's compiler) fuses the last multiply-add: within one fp16 ulp."""
    torch = pytest.importorskip("torch")
    from oracle import float_torch as FT

    x, qw, ws, b = OM.w8a8_linear_inputs()
    got = FT.w8a8_linear(*(torch.from_numpy(a) for a in (x, qw, ws, b))).numpy().astype(np.float32)
    a8, rs = OR.rot_q8_1024(x)
    want = OG.gemm_s8(a8, qw, rs, ws, b, OG.EPI_BIAS_F16).astype(np.float32)
    ulp = np.spacing(np.maximum(np.abs(got), np.abs(want)).astype(np.float16)).astype(np.float32)
    assert (np.abs(got - want) <= ulp).all()


# ---------------- planted mistakes: the checks above must catch them ----------------


def test_checks_catch_a_wrong_butterfly_sign(rng, monkeypatch):
    def bad(v, bit):
        n = v.shape[-1]
        w = v.reshape(*v.shape[:-1], n >> (bit + 1), 2, 1 << bit)
        a, b = w[..., 0, :], w[..., 1, :]
        return np.stack([a + b, b - a], axis=-2).reshape(v.shape)

    monkeypatch.setattr(OR, "butterfly", bad)
    with pytest.raises(AssertionError):
        test_fwht_matches_hadamard_product(rng)


def test_checks_catch_truncation_instead_of_rounding(monkeypatch):
    monkeypatch.setattr(OR.np, "rint", np.trunc)
    with pytest.raises(AssertionError):
        test_quant_rows_ties_and_clamp()


def test_checks_catch_a_transposed_gemm_operand(rng, monkeypatch):
    monkeypatch.setattr(OG, "gemm_s8_i32", lambda a, w: (a.astype(np.float64) @ w.astype(np.float64).T).T[: a.shape[0], : w.shape[0]].astype(np.int32))
    with pytest.raises(Exception):
        test_gemm_s8_i32_brute_force(rng, 3, 5, 7)


def test_checks_catch_a_dropped_rope_term(monkeypatch):
    def bad(y, m0, cos, sin, rope_len):
        rows = (np.arange(y.shape[0]) + m0) % rope_len
        pair = np.arange(y.shape[1] // 2) % 32
        co = cos[rows][:, pair]
        out = y.copy()
        out[:, 0::2] = y[:, 0::2] * co  # the - y1 sin term dropped
        out[:, 1::2] = y[:, 1::2] * co
        return out

    monkeypatch.setattr(OG, "rope_pairs", bad)
    with pytest.raises(AssertionError):
        test_qkv_rope_epilogue_closed_forms(np.random.default_rng(0))


def test_checks_catch_a_wrong_layernorm_divisor(rng, monkeypatch):
    orig = OR._xor_tree

    def tree(s, masks):  # sums correct, but report a 1023-element mean/variance
        return orig(s, masks) * F32(1024.0 / 1023.0)

    monkeypatch.setattr(OR, "_xor_tree", tree)
    with pytest.raises(AssertionError):
        test_layer_norm_1024_matches_float64(rng)
