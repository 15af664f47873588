// Walsh-Hadamard rotation fused with per-token symmetric int8 quantization (gfx950, wave64).
//
// The rotation spreads activation outliers over all channels so one scale per token suffices; the weights carry the
// same rotation. Both kernels are HBM-bound in bytes (2 B read + 1 B written per element) and close to VALU-bound
// in instructions, so the cross-lane butterflies are single DPP operations:
//
//  * Gray-code lane order: lane l of a 16-lane DPP row owns the 16-byte column chunk gray(l) = l ^ (l >> 1) of its
//    128-column group. The butterfly partner for column bit 3, 4, 5, 6 is then lane l ^ 1, ^ 3, ^ 7, ^ 15: quad_perm,
//    quad_perm, row_half_mirror and row_mirror, each a DPP source modifier (no LDS traffic, no extra instruction).
//  * Sign tracking: with partner value p and own value u, every lane computes fma(p, s, u) with s = +1 if its column
//    bit is 0 and -1 if 1. The lower lane gets a + b; the upper gets b - a = -(a - b), i.e. the reference's a - b
//    negated. One instruction per value and stage; the accumulated sign (-1)^(number of set column bits) is folded
//    into the quantization multiplier and the absmax is sign-free, so codes and scales are unchanged bit for bit
//    (IEEE rounding is sign-symmetric and fma(p, +-1, u) rounds once, like the reference's add and subtract).
//
// The butterfly stage order, the LayerNorm reduction order and every rounding match oracle/rotq8.py bit for bit (this
// file is compiled with -ffp-contract=off and correctly rounded fp32 division and sqrt; the LayerNorm's variance
// accumulation and affine step are explicit fused multiply-adds, as the reference's compiler contracts them).
//
// Reference: foidfinder/backends/cuda/csrc/kernels.cu:13-160 (rot_q8_1024_kernel, rot_q8_h128_kernel).
#include <algorithm>

#include "common.h"

namespace ff {

// Sign-tracked butterfly across lanes, u = fma(p, s, u) with partner p, own u, s = +1 (column bit 0) or -1 (column
// bit 1), as one v_fmac_f32_dpp (DPP on the multiplicand: the partner's u). The compiler only emits it as
// v_mov_b32_dpp + v_fmac_f32, so it is written out; one stage is one call over all of a lane's values, which are
// distinct registers, so the only VALU-write -> DPP-read hazard (2 wait states) is with whatever wrote them before
// the stage: the leading s_nop covers it. DPP controls: l^1 quad_perm [1,0,3,2], l^3 quad_perm [3,2,1,0], l^7
// row_half_mirror, l^15 row_mirror (all partners are inside the 16-lane DPP row, so bound_ctrl never applies).
#define FF_FMAC_DPP(CTL) "v_fmac_f32_dpp %0, %0, %1 " CTL " row_mask:0xf bank_mask:0xf bound_ctrl:1"
template <int CTRL, int N>
__device__ __forceinline__ void bfly_stage(float (&v)[N], float s) {
  asm volatile("s_nop 1" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if constexpr (CTRL == DPP_XOR1)
      asm volatile(FF_FMAC_DPP("quad_perm:[1,0,3,2]") : "+v"(v[i]) : "v"(s));
    else if constexpr (CTRL == DPP_XOR3)
      asm volatile(FF_FMAC_DPP("quad_perm:[3,2,1,0]") : "+v"(v[i]) : "v"(s));
    else if constexpr (CTRL == DPP_XOR7)
      asm volatile(FF_FMAC_DPP("row_half_mirror") : "+v"(v[i]) : "v"(s));
    else
      asm volatile(FF_FMAC_DPP("row_mirror") : "+v"(v[i]) : "v"(s));
  }
}

__device__ __forceinline__ float gray_sign(int bit) { return bit ? -1.f : 1.f; }

// Code of t in [-inf, inf]: clamp to [-127, 127], round half to even, low byte. Adding 1.5 * 2^23 rounds to an
// integer with ties to even (the ulp there is 1 and 1.5 * 2^23 is even), and the low byte of the sum's bit pattern is
// the code in two's complement.
__device__ __forceinline__ uint32_t q8_word(float t) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_fmed3f(t, -127.f, 127.f) + 12582912.f);
}

// The four codes, a in the low byte: two byte permutes gather the low bytes of (a, b) and (c, d), a third joins them.
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
  const uint32_t ab = __builtin_amdgcn_perm(q8_word(b), q8_word(a), 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(q8_word(d), q8_word(c), 0x0c0c0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// fp16 inputs folded into their first fp32 operation with v_fma_mix_f32, whose f16 sources convert exactly and whose
// result rounds once, so each equals the fp32 operation on the converted value: half HI of h2 plus s; and the first
// butterfly of an (even, odd) column pair held in one register: (lo + hi, lo - hi).
template <int HI>
__device__ __forceinline__ float add_h(uint32_t h2, float s) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s));
  return r;
}
// 0 + the low half of h2 (a sum's first term, as the reference's sum starting from 0), with 0 an inline constant: a
// register operand holding 0 would be hoisted out of the row loop and hold a register through it.
__device__ __forceinline__ float add_h_zero(uint32_t h2) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2));
  return r;
}
__device__ __forceinline__ void bfly0_h(uint32_t h2, float& lo_plus_hi, float& lo_minus_hi) {
  asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(lo_plus_hi) : "v"(h2));
  asm("v_fma_mix_f32 %0, %1, -1.0, %1 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(lo_minus_hi) : "v"(h2));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m; m >>= 1) v = fmaxf(v, xor_shuffle(v, m));
  return v;
}

// The LayerNorm reduction of the reference (kernels.cu:73, common.cuh:58-62) pairs reference lanes L ^ 16, ^ 8, ^ 4,
// ^ 2, ^ 1. With the Gray lane order those partners are physical lanes l ^ 16, ^ 15, ^ 7, ^ 3, ^ 1.
__device__ __forceinline__ float ref_tree_sum(float v) {
  v = v + swz_xor16(v);
  v = v + dpp<DPP_XOR15>(v);
  v = v + dpp<DPP_XOR7>(v);
  v = v + dpp<DPP_XOR3>(v);
  v = v + dpp<DPP_XOR1>(v);
  return v;
}

__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, swz_xor16(v));
  v = fmaxf(v, dpp<DPP_XOR15>(v));
  v = fmaxf(v, dpp<DPP_XOR7>(v));
  v = fmaxf(v, dpp<DPP_XOR3>(v));
  v = fmaxf(v, dpp<DPP_XOR1>(v));
  return v;
}

// One row of 1024 per 32-lane half-wave. Reference lane L = 16 c7 + gray(l & 15) of the half owns columns
// j*256 + L*8 + e (j 0..3, e 0..7), the reference's column layout (kernels.cu:11-12), held by physical lane
// l = 16 c7 + gray^-1(L & 15). Stage order: column bits 0, 1, 2 (registers e), 8, 9 (registers j), 3..7 (lanes; the
// last one, bit 7 = lane bit 4, through ds_swizzle). 256-thread workgroups of 8 half-waves stride over the rows;
// LayerNorm's gamma and beta sit in LDS, loaded once per workgroup.
template <bool NORM>
__global__ __launch_bounds__(256) void rot_q8_1024_kernel(const half_t* __restrict__ x, const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps, int64_t T,
                                                          int8_t* __restrict__ out, float* __restrict__ row_scale) {
  __shared__ float4_t gb[NORM ? 512 : 1];  // gamma as 256 float4, then beta
  if constexpr (NORM) {
    for (int i = threadIdx.x; i < 512; i += 256)
      gb[i] = i < 256 ? reinterpret_cast<const float4_t*>(gamma)[i] : reinterpret_cast<const float4_t*>(beta)[i - 256];
    __syncthreads();
  }
  const int lane = threadIdx.x & 31;
  const int l16 = lane & 15, gl = l16 ^ (l16 >> 1);
  const int L = (lane & 16) | gl;  // reference lane = column bits 3..7
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 8;
  int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  // whole half-waves share a row; cross-lane operations below stay inside the half
  // The row is loaded at the top of its own iteration, not prefetched during the previous one: without the 16
  // registers of a row in flight the kernel fits 7-8 waves per SIMD instead of 5-7, and the other waves hide the
  // load better than the prefetch did (measured 10-15 % faster).
  half8_t nxt[4];
  auto load = [&](int64_t r) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) nxt[j] = *reinterpret_cast<const half8_t*>(x + r * 1024 + j * 256 + L * 8);
  };
  const float s3 = gray_sign(L & 1), s4 = gray_sign(L & 2), s5 = gray_sign(L & 4), s6 = gray_sign(L & 8);
  const float s7 = gray_sign(L & 16);
  for (; row < T; row += stride) {
    float v[32];
    uint32_t w[4][4];  // the row's fp16 pairs (column e in half e & 1 of word e / 2)
    load(row);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) w[j][k] = __builtin_bit_cast(uint32_t, half2_t{nxt[j][2 * k], nxt[j][2 * k + 1]});
    auto hv = [&](int i, float s) __attribute__((always_inline)) {  // element i (= 8j + e) + s, one rounding
      return (i & 1) ? add_h<1>(w[i >> 3][(i & 7) >> 1], s) : add_h<0>(w[i >> 3][(i & 7) >> 1], s);
    };
    if constexpr (NORM) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) s = hv(i, s);
      const float mean = ref_tree_sum(s) * (1.f / 1024.f);
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        v[i] = hv(i, -mean);
        sq = __builtin_fmaf(v[i], v[i], sq);
      }
      const float var = ref_tree_sum(sq) * (1.f / 1024.f);
      const float rstd = 1.f / sqrtf(var + eps);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c4 = (j * 256 + L * 8) >> 2;  // float4 index of the lane's 8 columns
        const float4_t g0 = gb[c4], g1 = gb[c4 + 1], b0 = gb[256 + c4], b1 = gb[256 + c4 + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[j * 8 + e] = __builtin_fmaf(v[j * 8 + e] * rstd, g0[e], b0[e]);
          v[j * 8 + 4 + e] = __builtin_fmaf(v[j * 8 + 4 + e] * rstd, g1[e], b1[e]);
        }
      }
    }
    // column bits 0, 1, 2 (registers e); without the norm, bit 0 straight from the fp16 pairs
    if constexpr (!NORM) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) bfly0_h(w[j][k], v[j * 8 + 2 * k], v[j * 8 + 2 * k + 1]);
    }
#pragma unroll
    for (int h = NORM ? 1 : 2; h < 8; h <<= 1)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (!(e & h)) {
            const float a = v[j * 8 + e], b = v[j * 8 + e + h];
            v[j * 8 + e] = a + b;
            v[j * 8 + e + h] = a - b;
          }
    // column bits 8, 9 (registers j)
#pragma unroll
    for (int h = 1; h < 4; h <<= 1)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (!(j & h))
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float a = v[j * 8 + e], b = v[(j + h) * 8 + e];
            v[j * 8 + e] = a + b;
            v[(j + h) * 8 + e] = a - b;
          }
    // column bits 3..7 (lanes)
    bfly_stage<DPP_XOR1>(v, s3);
    bfly_stage<DPP_XOR3>(v, s4);
    bfly_stage<DPP_XOR7>(v, s5);
    bfly_stage<DPP_XOR15>(v, s6);
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = __builtin_fmaf(swz_xor16(v[i]), s7, v[i]);
    // v now holds (-1)^popcount(L) times the unnormalized rotation; x 1/32 is exact, so it joins the multiplier
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = half_wave_max(amax) * 0.03125f;
    const float scale = fmaxf(amax, 1e-12f) / 127.f;
    const float inv = 1.f / scale;
    const float mul = (__builtin_popcount(L) & 1 ? -inv : inv) * 0.03125f;
    int8_t* orow = out + row * 1024;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 pk;
      pk.x = pack4(v[j * 8] * mul, v[j * 8 + 1] * mul, v[j * 8 + 2] * mul, v[j * 8 + 3] * mul);
      pk.y = pack4(v[j * 8 + 4] * mul, v[j * 8 + 5] * mul, v[j * 8 + 6] * mul, v[j * 8 + 7] * mul);
      *reinterpret_cast<uint2*>(orow + j * 256 + L * 8) = pk;
    }
    if (lane == 0) row_scale[row] = scale;
  }
}

// One row of C = 128*nb columns per G groups of 16 lanes: G = 4 (a 64-lane wave per row) or G = 2 (a 32-lane
// half-wave per row, two rows per wave), chosen so that no group idles (h128_groups). Lane 16g + l of a row owns,
// for i = 0..NI-1, the 8 columns (G i + g)*128 + 8*gray(l) + e of block G i + g: column bits 0-2 in registers, bits
// 3-6 across the 16 lanes of a DPP row. Stages run over column bits 0..6 in ascending order, as in
// kernels.cu:125-135. 256-thread workgroups stride over the rows.
// LayerNorm (new; EVA02's norm after SwiGLU): gamma/beta are [C] with zeros past c_real, held in LDS (dynamic, 2C
// floats) for the workgroup's rows; sums over the real columns run per lane sequentially in (i, e) order, then over
// the row's lanes by the xor tree 32 (G = 4 only), 16, 15, 7, 3, 1.
// Rows are loaded at the top of their own iteration, not prefetched: the registers of a row in flight (8 NI per lane)
// would cost occupancy, and more waves per SIMD hide the load better (at EVA02's 2816 columns, NI = 11, three waves
// fit instead of two: 5-8 % faster; Haruka's rows 0-6 %).
template <int NI, bool NORM, int G, bool FULL, int TAIL>
__global__ __launch_bounds__(256, NI > 8 ? 3 : 1) void rot_q8_h128_kernel(const half_t* __restrict__ x, int64_t T, int C, int c_real,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps,
                                                          int8_t* __restrict__ out, float* __restrict__ row_scale) {
  static_assert(G == 2 || G == 4, "a row spans 2 or 4 groups of 16 lanes");
  constexpr int RPW = 4 / G;  // rows per wave
  extern __shared__ float4_t gbh[];  // NORM: gamma as C/4 float4, then beta
  const int nb = C >> 7;
  if constexpr (NORM) {
    const int n4 = C >> 2;
    for (int i = threadIdx.x; i < 2 * n4; i += 256)
      gbh[i] = i < n4 ? reinterpret_cast<const float4_t*>(gamma)[i] : reinterpret_cast<const float4_t*>(beta)[i - n4];
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int g = (lane >> 4) & (G - 1), l16 = lane & 15, gl = l16 ^ (l16 >> 1);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4 * RPW;
  // whole groups of 16 G lanes share a row; cross-lane operations below stay inside them
  int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RPW + (G == 2 ? lane >> 5 : 0);
  half8_t nxt[NI];
  auto load = [&](int64_t r) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int b = G * i + g;  // lanes of blocks past the row end hold zeros
      nxt[i] = (FULL || b < nb) ? *reinterpret_cast<const half8_t*>(x + r * C + b * 128 + 8 * gl) : half8_t{};
    }
  };
  const float s3 = gray_sign(gl & 1), s4 = gray_sign(gl & 2), s5 = gray_sign(gl & 4), s6 = gray_sign(gl & 8);
  // Block groups that can hold padding or lie past c_real: TAIL 2 none, 1 only the last one, 0 any (a uniform
  // run-time test). With TAIL 1 or 2 the LayerNorm loop is straight-line code; the per-group branches of TAIL 0 cost
  // 6-10 % at EVA02's 2816 columns and Haruka's 768 and 2048.
  auto padded = [&](int i) __attribute__((always_inline)) {
    if constexpr (TAIL == 2)
      return false;
    else if constexpr (TAIL == 1)
      return i == NI - 1;
    else
      return (G * i + G) * 128 > c_real;
  };
  auto tree_sum = [](float t) __attribute__((always_inline)) {
    if constexpr (G == 4) t = t + xor_shuffle(t, 32);
    t = t + swz_xor16(t);
    t = t + dpp<DPP_XOR15>(t);
    t = t + dpp<DPP_XOR7>(t);
    t = t + dpp<DPP_XOR3>(t);
    return t + dpp<DPP_XOR1>(t);
  };
  for (; row < T; row += stride) {
    float v[NI * 8];
    uint32_t w[NI][4];  // the row's fp16 pairs (column e in half e & 1 of word e / 2)
    load(row);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) w[i][k] = __builtin_bit_cast(uint32_t, half2_t{nxt[i][2 * k], nxt[i][2 * k + 1]});
    auto hv = [&](int i, int e, float s) __attribute__((always_inline)) {  // column (i, e) + s, one rounding
      return (e & 1) ? add_h<1>(w[i][e >> 1], s) : add_h<0>(w[i][e >> 1], s);
    };
    if constexpr (NORM) {
      // Only the padded() block groups can hold padding or the row end: the others skip the masks. Real columns
      // among the lane's 8 of block G i + g (a prefix): clamp(lb - 128 G i, 0, 8), with lb = c_real minus the lane's
      // first column of block g; blocks past the row end get 0 from the same formula (c_real <= 128 nb). lb is
      // recomputed each row from an opaque copy of the lane index (a few VALU), so that the compiler neither hoists
      // 8 NI loop-invariant lane masks into scalar registers nor holds counts through the loop: held, at NI = 11
      // they spilled, and a spill reload, queued behind the row's loads in the in-order memory counter, made the
      // wave wait for nearly the whole row before its first add.
      int ln = static_cast<int>(threadIdx.x);
      asm volatile("" : "+v"(ln));
      const int ls = ln & 15;
      const int lb = c_real - (((ln >> 4) & (G - 1)) * 128 + 8 * (ls ^ (ls >> 1)));
      int nr[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) nr[i] = min(max(lb - 128 * G * i, 0), 8);
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if (padded(i)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            // evaluated on every lane, then selected (no branch around the asm)
            const float t = i == 0 && e == 0 ? add_h_zero(w[0][0]) : hv(i, e, sum);
            sum = e < nr[i] ? t : sum;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) sum = i == 0 && e == 0 ? add_h_zero(w[0][0]) : hv(i, e, sum);
        }
      }
      const float fr = static_cast<float>(c_real);
      const float mean = tree_sum(sum) / fr;
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if (padded(i)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float t = hv(i, e, -mean);
            const float d = e < nr[i] ? t : 0.f;
            v[i * 8 + e] = d;
            sq = __builtin_fmaf(d, d, sq);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = hv(i, e, -mean);
            v[i * 8 + e] = d;
            sq = __builtin_fmaf(d, d, sq);
          }
        }
      }
      const float var = tree_sum(sq) / fr;
      const float rstd = 1.f / sqrtf(var + eps);
      const int n4 = C >> 2;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int b = G * i + g;
        if (!FULL && b >= nb) continue;  // lanes past the row end keep zeros (they take part in the row's absmax)
        const int c4 = (b * 128 + 8 * gl) >> 2;  // gamma/beta are zero past c_real: no masking inside the row
        const float4_t g0 = gbh[c4], g1 = gbh[c4 + 1], b0 = gbh[n4 + c4], b1 = gbh[n4 + c4 + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[i * 8 + e] = __builtin_fmaf(v[i * 8 + e] * rstd, g0[e], b0[e]);
          v[i * 8 + 4 + e] = __builtin_fmaf(v[i * 8 + 4 + e] * rstd, g1[e], b1[e]);
        }
      }
    }
    // column bits 0, 1, 2 (registers); without the norm, bit 0 straight from the fp16 pairs
    if constexpr (!NORM) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) bfly0_h(w[i][k], v[i * 8 + 2 * k], v[i * 8 + 2 * k + 1]);
    }
#pragma unroll
    for (int h = NORM ? 1 : 2; h < 8; h <<= 1)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (!(e & h)) {
            const float a = v[i * 8 + e], b = v[i * 8 + e + h];
            v[i * 8 + e] = a + b;
            v[i * 8 + e + h] = a - b;
          }
    // column bits 3..6 (lanes, Gray order)
    bfly_stage<DPP_XOR1>(v, s3);
    bfly_stage<DPP_XOR3>(v, s4);
    bfly_stage<DPP_XOR7>(v, s5);
    bfly_stage<DPP_XOR15>(v, s6);
    // x fp32(1/sqrt(128)) is a rounded multiply (kernels.cu:138); rounding is sign-symmetric, so it may act on the
    // sign-tracked values
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NI * 8; ++i) {
      v[i] = v[i] * 0.08838834764831845f;
      amax = fmaxf(amax, fabsf(v[i]));
    }
    if constexpr (G == 4)
      amax = wave_max(amax);
    else
      amax = half_wave_max(amax);
    const float scale = fmaxf(amax, 1e-12f) / 127.f;
    const float inv = 1.f / scale;
    const float mul = __builtin_popcount(gl) & 1 ? -inv : inv;
    int8_t* orow = out + row * C;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int b = G * i + g;
      if (FULL || b < nb) {
        uint2 pk;
        pk.x = pack4(v[i * 8] * mul, v[i * 8 + 1] * mul, v[i * 8 + 2] * mul, v[i * 8 + 3] * mul);
        pk.y = pack4(v[i * 8 + 4] * mul, v[i * 8 + 5] * mul, v[i * 8 + 6] * mul, v[i * 8 + 7] * mul);
        *reinterpret_cast<uint2*>(orow + b * 128 + 8 * gl) = pk;
      }
    }
    if ((lane & (16 * G - 1)) == 0) row_scale[row] = scale;
  }
}

// Grid of a grid-stride rotation kernel: one workgroup per `rows` rows, capped at what the device holds resident
// (every workgroup then streams rows, and no workgroup waits for a slot).
static dim3 stride_grid(const void* kernel, size_t smem, int64_t T, int rows) {
  int64_t cap = resident_blocks(kernel, 256, smem);
  if (cap <= 0) cap = 2048;
  return dim3(static_cast<unsigned>(std::min<int64_t>((T + rows - 1) / rows, cap)));
}

// 16-lane groups per row: 2 when the block count is even but not a multiple of 4 (768, 2816: no idle group), else 4
static int h128_groups(int nb) { return nb % 2 == 0 && nb % 4 != 0 && nb / 2 <= 12 ? 2 : 4; }

template <int NI, int G, bool FULL, int TAIL>
static void launch_h128_norm(hipStream_t st, const half_t* x, int64_t T, int C, int c_real, const float* g,
                             const float* b, float eps, int8_t* out, float* rs) {
  const size_t smem = 2 * C * sizeof(float);
  const dim3 grid = stride_grid(reinterpret_cast<const void*>(&rot_q8_h128_kernel<NI, true, G, FULL, TAIL>), smem, T,
                                4 * (4 / G));
  rot_q8_h128_kernel<NI, true, G, FULL, TAIL><<<grid, 256, smem, st>>>(x, T, C, c_real, g, b, eps, out, rs);
}
template <int NI, int G, bool FULL>
static void launch_h128_rows(hipStream_t st, const half_t* x, int64_t T, int C, int c_real, const float* g,
                             const float* b, float eps, int8_t* out, float* rs) {
  if (g) {
    // TAIL (see the kernel): whole rows of real columns need no masks, and when every block group but the last
    // holds real columns only, only the last one does
    if constexpr (FULL) {
      if (c_real == C)
        launch_h128_norm<NI, G, FULL, 2>(st, x, T, C, c_real, g, b, eps, out, rs);
      else if (c_real >= (NI - 1) * G * 128)
        launch_h128_norm<NI, G, FULL, 1>(st, x, T, C, c_real, g, b, eps, out, rs);
      else
        launch_h128_norm<NI, G, FULL, 0>(st, x, T, C, c_real, g, b, eps, out, rs);
    } else {
      launch_h128_norm<NI, G, FULL, 0>(st, x, T, C, c_real, g, b, eps, out, rs);
    }
  } else {
    const dim3 grid = stride_grid(reinterpret_cast<const void*>(&rot_q8_h128_kernel<NI, false, G, FULL, 0>), 0, T,
                                  4 * (4 / G));
    rot_q8_h128_kernel<NI, false, G, FULL, 0><<<grid, 256, 0, st>>>(x, T, C, c_real, g, b, eps, out, rs);
  }
}
// FULL: the row's nb blocks fill all NI G lane groups, so every load is unconditional (straight-line loads let the
// compiler wait for each block group as it arrives instead of for the whole row before the first add). Half-wave
// rows (G = 2) are always full; wave rows are full when 4 divides nb.
template <int NI, int G>
static void launch_h128(hipStream_t st, const half_t* x, int64_t T, int C, int c_real, const float* g, const float* b,
                        float eps, int8_t* out, float* rs) {
  if constexpr (G == 2) {
    launch_h128_rows<NI, G, true>(st, x, T, C, c_real, g, b, eps, out, rs);
  } else {
    if ((C >> 7) == NI * G)
      launch_h128_rows<NI, G, true>(st, x, T, C, c_real, g, b, eps, out, rs);
    else
      launch_h128_rows<NI, G, false>(st, x, T, C, c_real, g, b, eps, out, rs);
  }
}

}  // namespace ff

using namespace ff;

static bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

extern "C" int ff_rot_q8_1024(const void* x, const float* gamma, const float* beta, float eps, int64_t T, int8_t* out,
                              float* row_scale, void* stream) {
  clear_error();
  if (T < 0) return fail(FF_EINVAL, "rot_q8_1024: T must be >= 0");
  if (T == 0) return FF_OK;
  if (!x || !out || !row_scale) return fail(FF_EINVAL, "rot_q8_1024: null pointer");
  if ((gamma == nullptr) != (beta == nullptr)) return fail(FF_EINVAL, "rot_q8_1024: gamma and beta go together");
  if (gamma && !(eps > 0.f)) return fail(FF_EINVAL, "rot_q8_1024: eps must be > 0");
  if (!aligned(x, 16) || !aligned(out, 8) || !aligned(row_scale, 4) || (gamma && (!aligned(gamma, 16) || !aligned(beta, 16))))
    return fail(FF_EINVAL, "rot_q8_1024: misaligned pointer");
  // grid-stride: each half-wave takes every (8 * grid)-th row
  const half_t* px = static_cast<const half_t*>(x);
  if (gamma) {
    const dim3 grid = stride_grid(reinterpret_cast<const void*>(&rot_q8_1024_kernel<true>), 0, T, 8);
    rot_q8_1024_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(px, gamma, beta, eps, T, out, row_scale);
  } else {
    const dim3 grid = stride_grid(reinterpret_cast<const void*>(&rot_q8_1024_kernel<false>), 0, T, 8);
    rot_q8_1024_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(px, nullptr, nullptr, eps, T, out, row_scale);
  }
  return check_launch("rot_q8_1024");
}

extern "C" int ff_rot_q8_h128(const void* x, int64_t T, int64_t C, int64_t c_real, const float* gamma,
                              const float* beta, float eps, int8_t* out, float* row_scale, void* stream) {
  clear_error();
  if (T < 0) return fail(FF_EINVAL, "rot_q8_h128: T must be >= 0");
  if (C <= 0 || C % 128 != 0) return fail(FF_EINVAL, "rot_q8_h128: C must be a positive multiple of 128");
  if (C > 6144) return fail(FF_EINVAL, "rot_q8_h128: C > 6144 is not supported");
  if ((gamma == nullptr) != (beta == nullptr)) return fail(FF_EINVAL, "rot_q8_h128: gamma and beta go together");
  if (gamma && (c_real <= 0 || c_real > C)) return fail(FF_EINVAL, "rot_q8_h128: need 0 < c_real <= C");
  if (gamma && !(eps > 0.f)) return fail(FF_EINVAL, "rot_q8_h128: eps must be > 0");
  if (T == 0) return FF_OK;
  if (!x || !out || !row_scale) return fail(FF_EINVAL, "rot_q8_h128: null pointer");
  if (!aligned(x, 16) || !aligned(out, 8) || !aligned(row_scale, 4) || (gamma && (!aligned(gamma, 16) || !aligned(beta, 16))))
    return fail(FF_EINVAL, "rot_q8_h128: misaligned pointer");
  const int nb = static_cast<int>(C / 128);
  const int G = h128_groups(nb);
  const int ni = (nb + G - 1) / G;
  const int cr = gamma ? static_cast<int>(c_real) : static_cast<int>(C);
  const half_t* px = static_cast<const half_t*>(x);
  hipStream_t st = as_stream(stream);
  const int Ci = static_cast<int>(C);
#define FF_H128_CASE(N, GG) \
  case N: launch_h128<N, GG>(st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
  if (G == 2) {
    switch (ni) {
      FF_H128_CASE(1, 2) FF_H128_CASE(3, 2) FF_H128_CASE(5, 2) FF_H128_CASE(7, 2) FF_H128_CASE(9, 2)
      FF_H128_CASE(11, 2)
      default: return fail(FF_EINVAL, "rot_q8_h128: unsupported C");
    }
  } else {
    switch (ni) {
      FF_H128_CASE(1, 4) FF_H128_CASE(2, 4) FF_H128_CASE(3, 4) FF_H128_CASE(4, 4) FF_H128_CASE(5, 4)
      FF_H128_CASE(6, 4) FF_H128_CASE(7, 4) FF_H128_CASE(8, 4) FF_H128_CASE(9, 4) FF_H128_CASE(10, 4)
      FF_H128_CASE(11, 4) FF_H128_CASE(12, 4)
      default: return fail(FF_EINVAL, "rot_q8_h128: unsupported C");
    }
  }
#undef FF_H128_CASE
  return check_launch("rot_q8_h128");
}
