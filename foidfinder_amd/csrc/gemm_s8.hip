// W8A8 GEMM with exact int32 accumulation on gfx950 int8 MFMA, and the fused fp16 epilogues.
//
// acc[m, n] = sum_k A[m, k] W[n, k]; A [M, K] and W [N, K] are int8 with K contiguous.
// y = ((float)acc * row_scale[m]) * col_scale[n] + bias[n] (three roundings; this file is built with
// -ffp-contract=off), then the epilogue. The integer part is exact, so the order of the k-sum is free: each lane
// feeds the MFMA 16 contiguous bytes of K and the A- and W-fragments use the same k slots.
//
// Tiling: a 256-thread workgroup (4 waves as 2 x 2) computes a BM x BN tile of C from BK = 64 byte K-slices,
// double-buffered in LDS (global -> registers -> LDS, so the next slice's loads are in flight during the MFMAs).
// Each wave owns a (BM/2) x (BN/2) sub-tile made of 32 x 32 blocks of v_mfma_i32_32x32x32_i8. The MFMA computes the
// transposed product D[n][m] (W fragment as the row operand), so each lane ends with one row m and runs of 4
// consecutive columns n: pair epilogues (RoPE, SwiGLU) stay inside a lane and stores are 8 bytes wide.
//
// Reference: foidfinder/backends/cuda/csrc/gemm.cuh:14-171 and kernels.cu:167-217.
#include "common.h"

namespace ff {

struct GemmArgs {
  const int8_t* A;
  const int8_t* W;
  int M, N, K;
  const float* row_scale;  // [M]
  const float* col_scale;  // [N]
  const float* bias;       // [N]
  void* out;               // fp16 [M, N] (or [M, N/2] for SWIGLU, int32 [M, N] for I32; the residual for RESIDUAL)
  const float* rope_cos;   // [rope_len, 32]
  const float* rope_sin;
  int rope_len;
  float q_scale;
};

constexpr int BK = 64;

// LDS rows of 64 bytes (4 chunks of 16 B); chunk index XOR-swizzled with bits 1-2 of the row so the 16-byte
// fragment reads of 8 consecutive rows hit distinct banks.
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 1) & 3)) << 4); }

// Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a contiguous run of tiles (n fastest) so
// the tiles sharing an A row-panel share one L2.
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
  const int q = nblocks >> 3, r = nblocks & 7;
  const int x = b & 7, k = b >> 3;
  return x * q + (x < r ? x : r) + k;
}

// exp(x) from plain fp32 operations in a fixed order (no fused multiply-add: this file is built with
// -ffp-contract=off), so the CPU oracle reproduces it bit for bit: Cody-Waite range reduction x = n ln2 + r with ln2
// split into a 16-bit head and a tail (n * head is exact for |n| < 256), a degree-6 Taylor polynomial for e^r on
// |r| <= ln2/2, then an exact scaling by 2^n; relative error below 3e-7 over [-80, 80].
__device__ __forceinline__ float exp_cw(float x) {
  const float n = __builtin_rintf(x * 1.44269504088896341f);
  const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187045e-06f;
  float p = 1.f / 720.f;
  p = p * r + 1.f / 120.f;
  p = p * r + 1.f / 24.f;
  p = p * r + 1.f / 6.f;
  p = p * r + 0.5f;
  p = p * r + 1.f;
  p = p * r + 1.f;
  const int e = static_cast<int>(fminf(fmaxf(n, -300.f), 300.f));
  return ldexpf(p, e);
}

__device__ __forceinline__ float silu(float g) { return g / (1.f + exp_cw(-g)); }

__device__ __forceinline__ float gelu_tanh(float y) {
  return 0.5f * y * (1.f + tanhf(0.7978845608f * (y + 0.044715f * y * y * y)));
}

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256) void gemm_s8_kernel(const GemmArgs args) {
  constexpr int WM = BM / 2, WN = BN / 2;     // wave sub-tile
  constexpr int MI = WM / 32, NI = WN / 32;   // 32x32 MFMA blocks per wave
  constexpr int A_LD = BM * (BK / 16) / 256;  // 16-byte chunks per thread per slice
  constexpr int W_LD = BN * (BK / 16) / 256;
  constexpr int STAGE = (BM + BN) * BK;
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = args.M, N = args.N, K = args.K;
  const int tiles_n = (N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
  const int KT = K / BK;

  int4_t ra[A_LD], rw[W_LD];
  auto gload = [&](int kt) {
    const int kb = kt * BK;
#pragma unroll
    for (int p = 0; p < A_LD; ++p) {
      const int q = tid + 256 * p, r = q >> 2, c = q & 3;
      const int m = min(m0 + r, M - 1);
      ra[p] = *reinterpret_cast<const int4_t*>(args.A + static_cast<int64_t>(m) * K + kb + c * 16);
    }
#pragma unroll
    for (int p = 0; p < W_LD; ++p) {
      const int q = tid + 256 * p, r = q >> 2, c = q & 3;
      const int n = min(n0 + r, N - 1);
      rw[p] = *reinterpret_cast<const int4_t*>(args.W + static_cast<int64_t>(n) * K + kb + c * 16);
    }
  };
  auto swrite = [&](int buf) {
    int8_t* sa = smem + buf * STAGE;
    int8_t* sw = sa + BM * BK;
#pragma unroll
    for (int p = 0; p < A_LD; ++p) {
      const int q = tid + 256 * p;
      *reinterpret_cast<int4_t*>(sa + swz(q >> 2, q & 3)) = ra[p];
    }
#pragma unroll
    for (int p = 0; p < W_LD; ++p) {
      const int q = tid + 256 * p;
      *reinterpret_cast<int4_t*>(sw + swz(q >> 2, q & 3)) = rw[p];
    }
  };

  int16_t_v acc[NI][MI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int fr = lane & 31, fk = lane >> 5;  // fragment row, k half
  auto compute = [&](int buf) {
    const int8_t* sa = smem + buf * STAGE;
    const int8_t* sw = sa + BM * BK;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      int4_t xw[NI], ya[MI];
#pragma unroll
      for (int i = 0; i < NI; ++i)
        xw[i] = *reinterpret_cast<const int4_t*>(sw + swz(wn * WN + i * 32 + fr, 2 * kk + fk));
#pragma unroll
      for (int j = 0; j < MI; ++j)
        ya[j] = *reinterpret_cast<const int4_t*>(sa + swz(wm * WM + j * 32 + fr, 2 * kk + fk));
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xw[i], ya[j], acc[i][j], 0, 0, 0);
    }
  };

  gload(0);
  swrite(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    compute(cur);
    if (kt + 1 < KT) swrite(cur ^ 1);
    __syncthreads();
  }

  // Epilogue from registers. acc[i][j][4q + t] is D[n][m] with m = m0 + wm*WM + 32j + (lane & 31) and
  // n = n0 + wn*WN + 32i + 8q + 4*(lane >> 5) + t.
  const int C3 = N / 3;  // QKV: section width
#pragma unroll
  for (int j = 0; j < MI; ++j) {
    const int m = m0 + wm * WM + 32 * j + fr;
    if (m >= M) continue;
    const float rs = args.row_scale[m];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WN + 32 * i + 8 * q + 4 * fk;
        if (n >= N) continue;
        if constexpr (EPI == FF_EPI_I32) {
          int4_t v;
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = acc[i][j][4 * q + t];
          *reinterpret_cast<int4_t*>(static_cast<int*>(args.out) + static_cast<int64_t>(m) * N + n) = v;
        } else {
          const float4_t cs = *reinterpret_cast<const float4_t*>(args.col_scale + n);
          const float4_t bi = *reinterpret_cast<const float4_t*>(args.bias + n);
          float y[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) y[t] = static_cast<float>(acc[i][j][4 * q + t]) * rs * cs[t] + bi[t];
          half_t* o16 = static_cast<half_t*>(args.out);
          if constexpr (EPI == FF_EPI_SWIGLU) {
            half2_t h;
            h[0] = static_cast<half_t>(silu(y[0]) * y[1]);
            h[1] = static_cast<half_t>(silu(y[2]) * y[3]);
            *reinterpret_cast<half2_t*>(o16 + static_cast<int64_t>(m) * (N / 2) + n / 2) = h;
          } else {
            if constexpr (EPI == FF_EPI_QKV_ROPE) {
              const int section = n / C3;
              if (section < 2) {
                const int trow = (m % args.rope_len) * 32 + ((n & 63) >> 1);
#pragma unroll
                for (int pr = 0; pr < 2; ++pr) {
                  const float co = args.rope_cos[trow + pr], si = args.rope_sin[trow + pr];
                  const float y0 = y[2 * pr], y1 = y[2 * pr + 1];
                  const float r0 = y0 * co - y1 * si, r1 = y0 * si + y1 * co;
                  const float qs = section == 0 ? args.q_scale : 1.f;
                  y[2 * pr] = section == 0 ? r0 * qs : r0;
                  y[2 * pr + 1] = section == 0 ? r1 * qs : r1;
                }
              }
            }
            if constexpr (EPI == FF_EPI_GELU_F16) {
#pragma unroll
              for (int t = 0; t < 4; ++t) y[t] = gelu_tanh(y[t]);
            }
            half4_t h;
#pragma unroll
            for (int t = 0; t < 4; ++t) h[t] = static_cast<half_t>(y[t]);
            half4_t* dst = reinterpret_cast<half4_t*>(o16 + static_cast<int64_t>(m) * N + n);
            if constexpr (EPI == FF_EPI_RESIDUAL) {
              const half4_t x = *dst;
#pragma unroll
              for (int t = 0; t < 4; ++t) h[t] = h[t] + x[t];
            }
            *dst = h;
          }
        }
      }
  }
}

template <int BM, int BN>
static int launch_epi(const GemmArgs& a, int epi, hipStream_t st) {
  const int64_t tiles = static_cast<int64_t>((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles > 0x7fffffff) return fail(FF_EINVAL, "gemm_s8: too many tiles");
  const dim3 grid(static_cast<unsigned>(tiles));
  switch (epi) {
    case FF_EPI_QKV_ROPE: gemm_s8_kernel<BM, BN, FF_EPI_QKV_ROPE><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_RESIDUAL: gemm_s8_kernel<BM, BN, FF_EPI_RESIDUAL><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_GELU_F16: gemm_s8_kernel<BM, BN, FF_EPI_GELU_F16><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_SWIGLU: gemm_s8_kernel<BM, BN, FF_EPI_SWIGLU><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_BIAS_F16: gemm_s8_kernel<BM, BN, FF_EPI_BIAS_F16><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_I32: gemm_s8_kernel<BM, BN, FF_EPI_I32><<<grid, 256, 0, st>>>(a); break;
    default: return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  }
  return check_launch("gemm_s8");
}

constexpr int kVariants = 2;  // 1: 256 x 128 tiles, 2: 128 x 128 tiles

}  // namespace ff

using namespace ff;

static bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

extern "C" int ff_gemm_s8_variants(void) { return kVariants; }

extern "C" int ff_gemm_s8(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* row_scale,
                          const float* col_scale, const float* bias, void* out, int epi, int variant,
                          const float* rope_cos, const float* rope_sin, int64_t rope_len, float q_scale,
                          void* stream) {
  clear_error();
  if (M < 0 || N <= 0 || K <= 0) return fail(FF_EINVAL, "gemm_s8: need M >= 0, N > 0, K > 0");
  if (K % 64 != 0) return fail(FF_EINVAL, "gemm_s8: K must be a multiple of 64");
  if (N % 16 != 0) return fail(FF_EINVAL, "gemm_s8: N must be a multiple of 16");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return fail(FF_EINVAL, "gemm_s8: dimension too large");
  if (epi < FF_EPI_QKV_ROPE || epi > FF_EPI_I32) return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  if (variant < 0 || variant > kVariants) return fail(FF_EINVAL, "gemm_s8: bad variant");
  if (epi == FF_EPI_QKV_ROPE) {
    if (N % 3 != 0 || (N / 3) % 64 != 0) return fail(FF_EINVAL, "gemm_s8: QKV epilogue needs N = 3C with C % 64 == 0");
    if (!rope_cos || !rope_sin || rope_len <= 0) return fail(FF_EINVAL, "gemm_s8: QKV epilogue needs RoPE tables");
  }
  if (M == 0) return FF_OK;
  if (!A || !W || !out) return fail(FF_EINVAL, "gemm_s8: null pointer");
  if (epi != FF_EPI_I32 && (!row_scale || !col_scale || !bias)) return fail(FF_EINVAL, "gemm_s8: null scale/bias");
  if (!aligned(A, 16) || !aligned(W, 16) || !aligned(out, 8) ||
      (epi != FF_EPI_I32 && (!aligned(col_scale, 16) || !aligned(bias, 16))))
    return fail(FF_EINVAL, "gemm_s8: misaligned pointer");
  if (epi == FF_EPI_I32 && !aligned(out, 16)) return fail(FF_EINVAL, "gemm_s8: misaligned pointer");
  GemmArgs a{};
  a.A = A;
  a.W = W;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.row_scale = row_scale;
  a.col_scale = col_scale;
  a.bias = bias;
  a.out = out;
  a.rope_cos = rope_cos;
  a.rope_sin = rope_sin;
  a.rope_len = static_cast<int>(rope_len);
  a.q_scale = q_scale;
  hipStream_t st = as_stream(stream);
  switch (variant) {
    case 1: return launch_epi<256, 128>(a, epi, st);
    case 0:
    case 2: return launch_epi<128, 128>(a, epi, st);
  }
  return fail(FF_EINVAL, "gemm_s8: bad variant");
}
