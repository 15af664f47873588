"""W8A8 GEMM with exact int32 accumulation and the fused fp16 epilogues, restated in numpy.

acc[m, n] = sum_k A[m, k] * W[n, k] (int8 x int8 -> int32, exact), then
y = fma(float(acc) * row_scale[m], col_scale[n], bias[n])   (one rounding for the product, one for the fused step:
    the reference's `acc * rs * cs + bias` as the CUDA compiler contracts it, gemm.cuh:135-136)
and per epilogue (reference: foidfinder/backends/cuda/csrc/gemm.cuh:119-171, Epi enum gemm.cuh:8-12):

  QKV_ROPE  interleaved-pair rotation on the q and k sections (n < 2C, C = N/3) with table row m % rope_len and pair
            index (n mod 64)/2: r0 = y0*cos - y1*sin, r1 = y0*sin + y1*cos (each product rounded, then the sum);
            q additionally x q_scale; fp16 out                                              (gemm.cuh:140-151)
  RESIDUAL  x <- fp16(fp16(y) + x)                                                         (gemm.cuh:163-169)
  GELU_F16  fp16(gelu_tanh(y))                                                  (gemm.cuh:137-139, common.cuh:50-56)
  SWIGLU    columns interleaved as (gate j, value j) pairs: h[j] = fp16(silu(y[2j]) * y[2j+1]), out [M, N/2];
            silu uses exp_cw below, a deterministic exp (the GPU uses its ~1-ulp transcendental units and lands within
            one fp16 ulp of this)
            (no CUDA counterpart; EVA02 SwiGLU of foidfinder/backends/mlx/kernels.py:45-49 with the gate-first fc1
            rows of foidfinder/haruka.py:59-60 interleaved at conversion)
  BIAS_F16  fp16(y)
  I32       the raw int32 accumulators (debug, pins the integer GEMM bit for bit)
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
EPI_QKV_ROPE, EPI_RESIDUAL, EPI_GELU_F16, EPI_SWIGLU, EPI_BIAS_F16, EPI_I32 = 0, 1, 2, 3, 4, 5


def gemm_s8_i32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """A int8 [M, K] x W int8 [N, K] -> int32 [M, N], exact.

    float64 BLAS is exact here: every partial sum is an integer below K * 127^2 < 2^53 for K < 5.5e8."""
    assert a.dtype == np.int8 and w.dtype == np.int8 and a.shape[1] == w.shape[1]
    acc = a.astype(np.float64) @ w.astype(np.float64).T
    return acc.astype(np.int64).astype(np.int32)


def fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded float32 a * b + c with a single rounding (the hardware's fused multiply-add).

    a * b is exact in float64 (24 + 24 significant bits); Knuth's TwoSum splits p + c exactly into s + e in float64.
    Rounding s to float32 is then the correct rounding of p + c unless s lies exactly halfway between two float32
    values and e != 0: the sign of e then decides (numpy's tie-to-even would ignore it). (No float32 midpoint can lie
    strictly between p + c and s, since it would be a float64 value nearer to p + c than s.)

    The midpoint test runs on the float64 bits: in float32's normal range a float32 midpoint has exactly bit 28 set
    among the 29 low fraction bits that float32 drops. Only such elements, and those outside the normal range
    (subnormal, overflowing, non-finite), take the TwoSum path."""
    a, b, c = np.broadcast_arrays(np.asarray(a, F32), np.asarray(b, F32), np.asarray(c, F32))
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    r = s.astype(F32)
    mag = np.abs(s)
    cand = ((s.view(np.int64) & ((1 << 29) - 1)) == (1 << 28)) | ~(mag >= 2.0**-125) | (mag >= 2.0**127)
    if not cand.any():
        return r
    idx = np.nonzero(cand)
    r[idx] = _fma32_twosum(p[idx], c64[idx], s[idx])
    return r


def _fma32_twosum(p: np.ndarray, c64: np.ndarray, s: np.ndarray) -> np.ndarray:
    """fma32's exact path on 1-D float64 operands: p = a * b exact, s = p + c rounded to float64."""
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(F32)
    d = s - r.astype(np.float64)  # exact: r is the float32 rounding of s
    toward = np.where(d > 0, F32(np.inf), F32(-np.inf)).astype(F32)
    other = np.nextafter(r, toward)  # the float32 neighbour on s's side of r
    with np.errstate(invalid="ignore", over="ignore"):
        mid = (r.astype(np.float64) + other.astype(np.float64)) * 0.5
    fix = (d != 0) & (s == mid) & (e != 0) & ((e > 0) == (d > 0))
    return np.where(fix, other, r).astype(F32)


def dequant(acc: np.ndarray, row_scale: np.ndarray, col_scale: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """y = fma(float(acc) * rs[m], cs[n], bias[n]) in float32 (gemm.cuh:135-136 as contracted by its compiler)."""
    t = acc.astype(F32) * row_scale.astype(F32)[:, None]
    return fma32(t, col_scale.astype(F32)[None, :], bias.astype(F32)[None, :])


def gelu_tanh(y: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in float32 (common.cuh:55-56's formula)."""
    y = y.astype(F32)
    return F32(0.5) * y * (F32(1.0) + np.tanh(F32(0.7978845608) * (y + F32(0.044715) * y * y * y)))


def exp_cw(x: np.ndarray) -> np.ndarray:
    """exp(x) in float32 from plain float32 operations in a fixed order: Cody-Waite range reduction x = n ln2 + r with
    ln2 split as 0.693145751953125 (16 significant bits, so n * head is exact for |n| < 256) + 1.428606765330187045e-6,
    a degree-6 Taylor polynomial for e^r on |r| <= ln2/2 in Horner form, then an exact scaling by 2^n: a
    deterministic exp with relative error below 3e-7 over [-80, 80] (checked against float64 exp in
    tests/test_oracle.py), so that the SwiGLU restatement does not depend on the host's libm. The kernel instead takes
    e^-g from v_exp_f32 and the quotient from v_rcp_f32 (about 1 ulp each), so its fp16 SwiGLU outputs agree with
    this restatement to within one fp16 ulp, not bit for bit; the SwiGLU parity tests allow exactly that."""
    x = np.asarray(x, F32)
    n = np.rint(x * F32(1.44269504088896341))
    r = (x - n * F32(0.693145751953125)) - n * F32(1.428606765330187045e-06)
    p = np.full_like(r, F32(1.0) / F32(720.0))
    for c in (F32(1.0) / F32(120.0), F32(1.0) / F32(24.0), F32(1.0) / F32(6.0), F32(0.5), F32(1.0), F32(1.0)):
        p = p * r + c
    e = np.clip(n, -300, 300).astype(np.int32)
    return np.ldexp(p, e).astype(F32)


def silu(g: np.ndarray) -> np.ndarray:
    """g / (1 + exp(-g)) in float32 with exp_cw (mlx/kernels.py:45-49 formula, deterministic exp)."""
    g = g.astype(F32)
    return g / (F32(1.0) + exp_cw(-g))


def rope_pairs(y: np.ndarray, m0: int, cos: np.ndarray, sin: np.ndarray, rope_len: int) -> np.ndarray:
    """Rotate interleaved column pairs of a [M, 64*k] block whose rows are tokens m0.. (gemm.cuh:141-151)."""
    M, n = y.shape
    rows = (np.arange(M) + m0) % rope_len
    pair = (np.arange(n // 2)) % 32
    co = cos[rows][:, pair].astype(F32)
    si = sin[rows][:, pair].astype(F32)
    y0, y1 = y[:, 0::2], y[:, 1::2]
    out = np.empty_like(y)
    out[:, 0::2] = y0 * co - y1 * si
    out[:, 1::2] = y0 * si + y1 * co
    return out


def epilogue(
    acc: np.ndarray,
    row_scale: np.ndarray,
    col_scale: np.ndarray,
    bias: np.ndarray,
    epi: int,
    *,
    residual: np.ndarray | None = None,
    rope_cos: np.ndarray | None = None,
    rope_sin: np.ndarray | None = None,
    q_scale: float = 1.0,
) -> np.ndarray:
    """int32 accumulators -> the epilogue's output (fp16, or int32 for EPI_I32)."""
    if epi == EPI_I32:
        return acc.astype(np.int32)
    y = dequant(acc, row_scale, col_scale, bias)
    if epi == EPI_QKV_ROPE:
        N = y.shape[1]
        assert N % 3 == 0 and (N // 3) % 64 == 0
        C = N // 3
        qk = rope_pairs(y[:, : 2 * C], 0, rope_cos, rope_sin, rope_cos.shape[0])
        qk[:, :C] = qk[:, :C] * F32(q_scale)
        y = np.concatenate([qk, y[:, 2 * C :]], axis=1)
        return y.astype(np.float16)
    if epi == EPI_RESIDUAL:
        assert residual is not None and residual.dtype == np.float16
        return (y.astype(np.float16).astype(F32) + residual.astype(F32)).astype(np.float16)
    if epi == EPI_GELU_F16:
        return gelu_tanh(y).astype(np.float16)
    if epi == EPI_SWIGLU:
        return (silu(y[:, 0::2]) * y[:, 1::2]).astype(np.float16)
    if epi == EPI_BIAS_F16:
        return y.astype(np.float16)
    raise ValueError(f"bad epilogue {epi}")


def gemm_s8(
    a: np.ndarray,
    w: np.ndarray,
    row_scale: np.ndarray,
    col_scale: np.ndarray,
    bias: np.ndarray,
    epi: int,
    **kw,
) -> np.ndarray:
    """The whole op: exact int32 GEMM then the epilogue (the reference op `gemm_s8`, kernels.cu:187-217)."""
    return epilogue(gemm_s8_i32(a, w), row_scale, col_scale, bias, epi, **kw)
