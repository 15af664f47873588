// Walsh-Hadamard rotation fused with per-token symmetric int8 quantization (gfx950, wave64).
//
// The rotation spreads activation outliers over all channels so one scale per token suffices; the weights carry the
// same rotation. Both kernels are HBM-bound (2 B read + 1 B written per element). The butterfly stage order, the
// LayerNorm reduction order and every rounding match oracle/rotq8.py bit for bit (this file is compiled with
// -ffp-contract=off and correctly rounded fp32 division and sqrt).
//
// Reference: foidfinder/backends/cuda/csrc/kernels.cu:13-160 (rot_q8_1024_kernel, rot_q8_h128_kernel).
#include "common.h"

namespace ff {

// Sum over the 32 lanes of a half-wave, xor tree 16, 8, 4, 2, 1 (the order fixes the rounding).
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
  for (int m = 16; m; m >>= 1) v = v + xor_shuffle(v, m);
  return v;
}

__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
  for (int m = 16; m; m >>= 1) v = fmaxf(v, xor_shuffle(v, m));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m; m >>= 1) v = v + xor_shuffle(v, m);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m; m >>= 1) v = fmaxf(v, xor_shuffle(v, m));
  return v;
}

// Butterfly across lanes: the lane with bit `m` clear holds a, its partner b; results a + b (lower), a - b (upper).
__device__ __forceinline__ float lane_butterfly(float v, int m, bool upper) {
  const float o = xor_shuffle(v, m);
  return upper ? o - v : v + o;
}

// One row of 1024 per 32-lane half-wave; lane L of the half owns columns j*256 + L*8 + e (j 0..3, e 0..7), the
// reference's column layout (kernels.cu:11-12), which makes its stage order (column bits 0,1,2 | 8,9 | 3..7) and its
// LayerNorm reduction order natural here. 8 rows per 256-thread workgroup.
template <bool NORM>
__global__ __launch_bounds__(256) void rot_q8_1024_kernel(const half_t* __restrict__ x, const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps, int64_t T,
                                                          int8_t* __restrict__ out, float* __restrict__ row_scale) {
  const int lane = threadIdx.x & 31;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (row >= T) return;  // whole half-waves exit together; shuffles below stay inside the half
  const half_t* xr = x + row * 1024;
  float v[32];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const half8_t h = *reinterpret_cast<const half8_t*>(xr + j * 256 + lane * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j * 8 + e] = static_cast<float>(h[e]);
  }
  if constexpr (NORM) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s = s + v[i];
    const float mean = half_wave_sum(s) * (1.f / 1024.f);
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      v[i] = v[i] - mean;
      sq = sq + v[i] * v[i];
    }
    const float var = half_wave_sum(sq) * (1.f / 1024.f);
    const float rstd = 1.f / sqrtf(var + eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = j * 256 + lane * 8;
      const float4_t g0 = *reinterpret_cast<const float4_t*>(gamma + c);
      const float4_t g1 = *reinterpret_cast<const float4_t*>(gamma + c + 4);
      const float4_t b0 = *reinterpret_cast<const float4_t*>(beta + c);
      const float4_t b1 = *reinterpret_cast<const float4_t*>(beta + c + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[j * 8 + e] = v[j * 8 + e] * rstd * g0[e] + b0[e];
        v[j * 8 + 4 + e] = v[j * 8 + 4 + e] * rstd * g1[e] + b1[e];
      }
    }
  }
  // column bits 0, 1, 2 (registers e)
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
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
  // column bits 3..7 (lane bits 0..4)
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) {
    const bool upper = lane & m;
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = lane_butterfly(v[i], m, upper);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    v[i] = v[i] * 0.03125f;  // 1/sqrt(1024), exact
    amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = half_wave_max(amax);
  const float scale = fmaxf(amax, 1e-12f) / 127.f;
  const float inv = 1.f / scale;
  int8_t* orow = out + row * 1024;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint2 pk;
    pk.x = q8x4(v[j * 8] * inv, v[j * 8 + 1] * inv, v[j * 8 + 2] * inv, v[j * 8 + 3] * inv);
    pk.y = q8x4(v[j * 8 + 4] * inv, v[j * 8 + 5] * inv, v[j * 8 + 6] * inv, v[j * 8 + 7] * inv);
    *reinterpret_cast<uint2*>(orow + j * 256 + lane * 8) = pk;
  }
  if (lane == 0) row_scale[row] = scale;
}

// One row of C = 128*nb columns per 64-lane wave. Lane l = 16g + s owns, for i = 0..NI-1, the 8 columns
// (4i + g)*128 + 8s + e of block 4i + g: column bits 0-2 in registers, bits 3-6 across the 16 lanes of a DPP row.
// Stages run over column bits 0..6 in ascending order, as in kernels.cu:125-135. 4 rows per workgroup.
template <int NI, bool NORM>
__global__ __launch_bounds__(256) void rot_q8_h128_kernel(const half_t* __restrict__ x, int64_t T, int C, int c_real,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps,
                                                          int8_t* __restrict__ out, float* __restrict__ row_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= T) return;  // whole waves exit together
  const int g = lane >> 4, s = lane & 15;
  const int nb = C >> 7;
  const half_t* xr = x + row * C;
  float v[NI * 8];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int b = 4 * i + g;
    if (b < nb) {
      const half8_t h = *reinterpret_cast<const half8_t*>(xr + b * 128 + 8 * s);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i * 8 + e] = static_cast<float>(h[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i * 8 + e] = 0.f;
    }
  }
  if constexpr (NORM) {
    // LayerNorm over the first c_real columns; the rest are padding and stay zero. nreal[i] = how many of the
    // lane's 8 columns of block 4i + g are real (the prefix e < nreal[i]).
    int nreal[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int b = 4 * i + g;
      const int left = c_real - (b * 128 + 8 * s);
      nreal[i] = b < nb ? (left < 0 ? 0 : (left > 8 ? 8 : left)) : 0;
    }
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) sum = sum + (e < nreal[i] ? v[i * 8 + e] : 0.f);
    const float fr = static_cast<float>(c_real);
    const float mean = wave_sum(sum) / fr;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = e < nreal[i] ? v[i * 8 + e] - mean : 0.f;
        v[i * 8 + e] = d;
        sq = sq + d * d;
      }
    const float var = wave_sum(sq) / fr;
    const float rstd = 1.f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int col0 = (4 * i + g) * 128 + 8 * s;
      float gg[8], bb[8];
      if (nreal[i] == 8) {
        const float4_t g0 = *reinterpret_cast<const float4_t*>(gamma + col0);
        const float4_t g1 = *reinterpret_cast<const float4_t*>(gamma + col0 + 4);
        const float4_t b0 = *reinterpret_cast<const float4_t*>(beta + col0);
        const float4_t b1 = *reinterpret_cast<const float4_t*>(beta + col0 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gg[e] = g0[e];
          gg[e + 4] = g1[e];
          bb[e] = b0[e];
          bb[e + 4] = b1[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int cc = e < nreal[i] ? col0 + e : 0;  // never read gamma/beta past c_real
          gg[e] = gamma[cc];
          bb[e] = beta[cc];
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = v[i * 8 + e] * rstd * gg[e] + bb[e];
        v[i * 8 + e] = e < nreal[i] ? y : 0.f;
      }
    }
  }
  // column bits 0, 1, 2 (registers)
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!(e & h)) {
          const float a = v[i * 8 + e], b = v[i * 8 + e + h];
          v[i * 8 + e] = a + b;
          v[i * 8 + e + h] = a - b;
        }
  // column bits 3..6 (lane bits 0..3)
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    const bool upper = lane & m;
#pragma unroll
    for (int i = 0; i < NI * 8; ++i) v[i] = lane_butterfly(v[i], m, upper);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < NI * 8; ++i) {
    v[i] = v[i] * 0.08838834764831845f;  // fp32(1/sqrt(128)), kernels.cu:138
    amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max(amax);
  const float scale = fmaxf(amax, 1e-12f) / 127.f;
  const float inv = 1.f / scale;
  int8_t* orow = out + row * C;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int b = 4 * i + g;
    if (b < nb) {
      uint2 pk;
      pk.x = q8x4(v[i * 8] * inv, v[i * 8 + 1] * inv, v[i * 8 + 2] * inv, v[i * 8 + 3] * inv);
      pk.y = q8x4(v[i * 8 + 4] * inv, v[i * 8 + 5] * inv, v[i * 8 + 6] * inv, v[i * 8 + 7] * inv);
      *reinterpret_cast<uint2*>(orow + b * 128 + 8 * s) = pk;
    }
  }
  if (lane == 0) row_scale[row] = scale;
}

template <int NI>
static void launch_h128(dim3 grid, hipStream_t st, const half_t* x, int64_t T, int C, int c_real, const float* g,
                        const float* b, float eps, int8_t* out, float* rs) {
  if (g)
    rot_q8_h128_kernel<NI, true><<<grid, 256, 0, st>>>(x, T, C, c_real, g, b, eps, out, rs);
  else
    rot_q8_h128_kernel<NI, false><<<grid, 256, 0, st>>>(x, T, C, c_real, g, b, eps, out, rs);
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
  const int64_t blocks = (T + 7) / 8;
  if (blocks > 0x7fffffff) return fail(FF_EINVAL, "rot_q8_1024: T too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  const half_t* px = static_cast<const half_t*>(x);
  if (gamma)
    rot_q8_1024_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(px, gamma, beta, eps, T, out, row_scale);
  else
    rot_q8_1024_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(px, nullptr, nullptr, eps, T, out, row_scale);
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
  const int64_t blocks = (T + 3) / 4;
  if (blocks > 0x7fffffff) return fail(FF_EINVAL, "rot_q8_h128: T too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  const int nb = static_cast<int>(C / 128);
  const int ni = (nb + 3) / 4;
  const int cr = gamma ? static_cast<int>(c_real) : static_cast<int>(C);
  const half_t* px = static_cast<const half_t*>(x);
  hipStream_t st = as_stream(stream);
  const int Ci = static_cast<int>(C);
  switch (ni) {
    case 1: launch_h128<1>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 2: launch_h128<2>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 3: launch_h128<3>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 4: launch_h128<4>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 5: launch_h128<5>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 6: launch_h128<6>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 7: launch_h128<7>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 8: launch_h128<8>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 9: launch_h128<9>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 10: launch_h128<10>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 11: launch_h128<11>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    case 12: launch_h128<12>(grid, st, px, T, Ci, cr, gamma, beta, eps, out, row_scale); break;
    default: return fail(FF_EINVAL, "rot_q8_h128: unsupported C");
  }
  return check_launch("rot_q8_h128");
}
