// The memory-bound steps of Haruka's slot-sigmoid tree pool (foidfinder/backends/mlx/haruka.py:101-133) on gfx950:
//
//  * layer_norm2: the backbone's final LayerNorm, rounded to fp16, then the pool's own LayerNorm, in one pass over
//    the tokens (the reference applies them one after the other, each returning fp16).
//  * slot_weights: per token and pool head, the weights of M competing queries, softmax over the queries times
//    sigmoid(logit + bias), written transposed (query-major rows over the tokens, the layout of the pooling product)
//    with per-block sums over the tokens (each query's mass).
#include <algorithm>

#include "common.h"

namespace ff {

// One wave per row of C (C % 64 == 0, C <= 2048): lane l holds columns l + 64 k. Means and variances are two-pass
// (sum, then squared deviations) in fp32, rstd = 1 / sqrt(var + eps).
template <int PER>
__global__ __launch_bounds__(256) void layer_norm2_kernel(const half_t* __restrict__ x, int64_t T, int C,
                                                          const half_t* __restrict__ g1, const half_t* __restrict__ b1,
                                                          const half_t* __restrict__ g2, const half_t* __restrict__ b2,
                                                          float eps, half_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  const half_t* xr = x + row * C;
  float v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) v[k] = 64 * k + lane < C ? static_cast<float>(xr[64 * k + lane]) : 0.f;
  const float inv_c = 1.f / static_cast<float>(C);
  auto norm = [&](const half_t* g, const half_t* b, bool round_fp16) __attribute__((always_inline)) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) s += v[k];
#pragma unroll
    for (int m = 32; m; m >>= 1) s += xor_shuffle(s, m);
    const float mean = s * inv_c;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const float d = 64 * k + lane < C ? v[k] - mean : 0.f;
      q += d * d;
    }
#pragma unroll
    for (int m = 32; m; m >>= 1) q += xor_shuffle(q, m);
    const float rstd = 1.f / sqrtf(q * inv_c + eps);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int c = 64 * k + lane;
      if (c < C) {
        const float y = (v[k] - mean) * rstd * static_cast<float>(g[c]) + static_cast<float>(b[c]);
        v[k] = round_fp16 ? static_cast<float>(static_cast<half_t>(y)) : y;
      }
    }
  };
  norm(g1, b1, true);
  norm(g2, b2, false);
  half_t* orow = out + row * C;
#pragma unroll
  for (int k = 0; k < PER; ++k)
    if (64 * k + lane < C) orow[64 * k + lane] = static_cast<half_t>(v[k]);
}

// The same two norms for C % 256 == 0 (Haruka's 768): lane l holds the 4 contiguous columns 4 (l + 64 k), so each
// load and store moves 8 bytes per lane, and each wave streams rows (row = wave id + k * waves in the grid) with the
// four affine vectors kept in registers. Same arithmetic as layer_norm2_kernel; only the order of the sums differs.
template <int CH>
__global__ __launch_bounds__(256) void layer_norm2_vec_kernel(const half_t* __restrict__ x, int64_t T, int C,
                                                              const half_t* __restrict__ g1,
                                                              const half_t* __restrict__ b1,
                                                              const half_t* __restrict__ g2,
                                                              const half_t* __restrict__ b2, float eps,
                                                              half_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
  const int nch = C / 256;  // chunks per lane (<= CH)
  half4_t ga[CH], ba[CH], gb[CH], bb[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k)
    if (k < nch) {
      const int c = 4 * (lane + 64 * k);
      ga[k] = *reinterpret_cast<const half4_t*>(g1 + c);
      ba[k] = *reinterpret_cast<const half4_t*>(b1 + c);
      gb[k] = *reinterpret_cast<const half4_t*>(g2 + c);
      bb[k] = *reinterpret_cast<const half4_t*>(b2 + c);
    }
  const float inv_c = 1.f / static_cast<float>(C);
  // the next row's loads are issued before the current row's reductions, so a wave always has a row in flight
  half4_t nxt[CH];
  auto load = [&](int64_t r) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < CH; ++k)
      nxt[k] = k < nch ? *reinterpret_cast<const half4_t*>(x + r * C + 4 * (lane + 64 * k)) : half4_t{};
  };
  int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row < T) load(row);
  for (; row < T; row += waves) {
    float v[CH][4];
#pragma unroll
    for (int k = 0; k < CH; ++k)
#pragma unroll
      for (int t = 0; t < 4; ++t) v[k][t] = static_cast<float>(nxt[k][t]);
    if (row + waves < T) load(row + waves);
    auto norm = [&](const half4_t (&g)[CH], const half4_t (&b)[CH], bool round_fp16) __attribute__((always_inline)) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < CH; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) s += v[k][t];
      s = wave_sum(s);
      const float mean = s * inv_c;
      float q = 0.f;
#pragma unroll
      for (int k = 0; k < CH; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float d = k < nch ? v[k][t] - mean : 0.f;
          q += d * d;
        }
      q = wave_sum(q);
      const float rstd = 1.f / sqrtf(q * inv_c + eps);
#pragma unroll
      for (int k = 0; k < CH; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float y = (v[k][t] - mean) * rstd * static_cast<float>(g[k][t]) + static_cast<float>(b[k][t]);
          v[k][t] = round_fp16 ? static_cast<float>(static_cast<half_t>(y)) : y;
        }
    };
    norm(ga, ba, true);
    norm(gb, bb, false);
    half_t* orow = out + row * C;
#pragma unroll
    for (int k = 0; k < CH; ++k)
      if (k < nch) {
        half4_t h;
#pragma unroll
        for (int t = 0; t < 4; ++t) h[t] = static_cast<half_t>(v[k][t]);
        *reinterpret_cast<half4_t*>(orow + 4 * (lane + 64 * k)) = h;
      }
  }
}

// Tokens per workgroup of slot_weights.
constexpr int SW_TOKENS = 32;

// Grid (token blocks of 32, batch). The block's logits [ntok][G*M] are one contiguous run: the workgroup first copies
// them into LDS (16-byte loads when G*M % 8 == 0 and the base is 16-byte aligned, else 2-byte ones). Thread t then
// handles pairs (token, head) p = t, t + 256, ... of the block's 32 x G: it reads the pair's M logits (+ c, the
// queries' key-bias terms) from LDS and computes the weights in fp32 from the hardware exp2 and reciprocal (each about
// 1 ulp), softmax over the queries times sigmoid(logit + bias), keeping them in registers. After a barrier the same
// LDS holds the weights as a tile [G*M][32] (transposed), which is written out row by row (32 contiguous tokens per
// query column, two columns per wave); each column's fp32 sum over the block's tokens goes to partial[b, block,
// column] (summed in token order by one thread per column). PMAX bounds the pairs per thread: the host allows G*M <= 496, i.e. 32 G <= 256 PMAX.
template <int M>
__global__ __launch_bounds__(256) void slot_weights_kernel(const half_t* __restrict__ logits, const float* __restrict__ c,
                                                           int64_t c_stride, const float* __restrict__ bias, int N,
                                                           int G, int vec, half_t* __restrict__ a_t,
                                                           float* __restrict__ partial) {
  constexpr int PMAX = M == 18 ? 4 : 8;
  constexpr float LOG2E = 1.4426950408889634f;
  extern __shared__ float tile[];  // first the logits block (fp16), then [G*M][SW_TOKENS + 1] fp32 weights
  half_t* lh = reinterpret_cast<half_t*>(tile);
  const int GM = G * M, b = blockIdx.y, n0 = blockIdx.x * SW_TOKENS;
  const int ntok = min(SW_TOKENS, N - n0);
  const half_t* lg = logits + (static_cast<int64_t>(b) * N + n0) * GM;
  const int nh = ntok * GM;
  if (vec) {
    for (int i = threadIdx.x; i < nh / 8; i += 256)
      reinterpret_cast<int4_t*>(lh)[i] = reinterpret_cast<const int4_t*>(lg)[i];
  } else {
    for (int i = threadIdx.x; i < nh; i += 256) lh[i] = lg[i];
  }
  const float* cb = c + b * c_stride;
  float bi[M];
#pragma unroll
  for (int m = 0; m < M; ++m) bi[m] = -bias[m] * LOG2E;
  __syncthreads();
  float w[PMAX][M];
#pragma unroll
  for (int k = 0; k < PMAX; ++k) {
    const int p = threadIdx.x + 256 * k, t = p / G, h = p % G;
    if (t < ntok) {
      float l[M];
      float mx = -INFINITY;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        l[m] = static_cast<float>(lh[p * M + m]) + cb[h * M + m];
        mx = fmaxf(mx, l[m]);
      }
      float s = 0.f;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        w[k][m] = __builtin_amdgcn_exp2f((l[m] - mx) * LOG2E);
        s += w[k][m];
      }
      const float inv = __builtin_amdgcn_rcpf(s);
#pragma unroll
      for (int m = 0; m < M; ++m)
        w[k][m] = w[k][m] * inv * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(__builtin_fmaf(-l[m], LOG2E, bi[m])));
    }
  }
  __syncthreads();  // every logit is read: the tile may overwrite them
#pragma unroll
  for (int k = 0; k < PMAX; ++k) {
    const int p = threadIdx.x + 256 * k, t = p / G, h = p % G;
    if (t < SW_TOKENS) {
#pragma unroll
      for (int m = 0; m < M; ++m) tile[(h * M + m) * (SW_TOKENS + 1) + t] = t < ntok ? w[k][m] : 0.f;
    }
  }
  __syncthreads();
  // each column's sum over the block's 32 tokens (zeros past ntok), one thread per column, in token order
  for (int j = threadIdx.x; j < GM; j += 256) {
    float s = 0.f;
#pragma unroll 8
    for (int t = 0; t < SW_TOKENS; ++t) s += tile[j * (SW_TOKENS + 1) + t];
    partial[(static_cast<int64_t>(b) * gridDim.x + blockIdx.x) * GM + j] = s;
  }
  // rows of the transposed tile: each half-wave takes every eighth query column, a lane per token
  const int half = threadIdx.x >> 5, lane = threadIdx.x & 31;
  if (lane < ntok) {
    half_t* orow = a_t + static_cast<int64_t>(b) * GM * N + n0 + lane;
#pragma unroll 4
    for (int j = half; j < GM; j += 8)
      orow[static_cast<int64_t>(j) * N] = static_cast<half_t>(tile[j * (SW_TOKENS + 1) + lane]);
  }
}

}  // namespace ff

using namespace ff;

extern "C" int ff_layer_norm2(const void* x, int64_t T, int64_t C, const void* g1, const void* b1, const void* g2,
                              const void* b2, float eps, void* out, void* stream) {
  clear_error();
  if (T < 0 || C <= 0 || C % 64 != 0 || C > 2048)
    return fail(FF_EINVAL, "layer_norm2: need T >= 0 and 0 < C <= 2048, C % 64 == 0");
  if (!(eps > 0.f)) return fail(FF_EINVAL, "layer_norm2: eps must be > 0");
  if (T == 0) return FF_OK;
  if (!x || !g1 || !b1 || !g2 || !b2 || !out) return fail(FF_EINVAL, "layer_norm2: null pointer");
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  const hipStream_t st = as_stream(stream);
  const auto* px = static_cast<const half_t*>(x);
  const auto *pg1 = static_cast<const half_t*>(g1), *pb1 = static_cast<const half_t*>(b1);
  const auto *pg2 = static_cast<const half_t*>(g2), *pb2 = static_cast<const half_t*>(b2);
  auto* po = static_cast<half_t*>(out);
  const int Ci = static_cast<int>(C);
  const auto aligned8 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 8 == 0; };
  const bool vec = C % 256 == 0 && C <= 1024 && aligned8(x) && aligned8(g1) && aligned8(b1) && aligned8(g2) &&
                   aligned8(b2) && aligned8(out);
  if (vec) {
    // a few waves per SIMD stream the rows, so the affine vectors are loaded once per wave
    const dim3 vgrid(static_cast<unsigned>(std::min<int64_t>((T + 3) / 4, 2048)));
    layer_norm2_vec_kernel<4><<<vgrid, 256, 0, st>>>(px, T, Ci, pg1, pb1, pg2, pb2, eps, po);
  } else if (C <= 768) {
    layer_norm2_kernel<12><<<grid, 256, 0, st>>>(px, T, Ci, pg1, pb1, pg2, pb2, eps, po);
  } else {
    layer_norm2_kernel<32><<<grid, 256, 0, st>>>(px, T, Ci, pg1, pb1, pg2, pb2, eps, po);
  }
  return check_launch("layer_norm2");
}

extern "C" int64_t ff_slot_weights_blocks(int64_t N) { return N > 0 ? (N + SW_TOKENS - 1) / SW_TOKENS : 0; }

extern "C" int ff_slot_weights(const void* logits, const float* c, int64_t c_stride, const float* bias, int64_t B,
                               int64_t N, int64_t G, int64_t M, void* a_t, float* partial, void* stream) {
  clear_error();
  if (B < 0 || N <= 0 || N > 0x7fffffff || G <= 0 || G > 64) return fail(FF_EINVAL, "slot_weights: bad B, N or G");
  if (M != 6 && M != 18) return fail(FF_EINVAL, "slot_weights: M must be 6 or 18 (the tree pool's query counts)");
  if (B > 65535) return fail(FF_EINVAL, "slot_weights: B > 65535");
  if (c_stride != 0 && c_stride < G * M) return fail(FF_EINVAL, "slot_weights: c_stride must be 0 or >= G*M");
  if (B == 0) return FF_OK;
  if (!logits || !c || !bias || !a_t || !partial) return fail(FF_EINVAL, "slot_weights: null pointer");
  const size_t smem = static_cast<size_t>(G * M) * (SW_TOKENS + 1) * sizeof(float);
  if (smem > 64 * 1024) return fail(FF_EINVAL, "slot_weights: G*M too large (LDS tile above 64 KB)");
  // the fp16 logits block (64 G M bytes) fits in the tile's LDS, and 32 G pairs fit the kernel's 256 PMAX
  const int vec = (G * M) % 8 == 0 && reinterpret_cast<uintptr_t>(logits) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(ff_slot_weights_blocks(N)), static_cast<unsigned>(B));
  const hipStream_t st = as_stream(stream);
  const auto* pl = static_cast<const half_t*>(logits);
  auto* pa = static_cast<half_t*>(a_t);
  const int Ni = static_cast<int>(N), Gi = static_cast<int>(G);
  if (M == 6)
    slot_weights_kernel<6><<<grid, 256, smem, st>>>(pl, c, c_stride, bias, Ni, Gi, vec, pa, partial);
  else
    slot_weights_kernel<18><<<grid, 256, smem, st>>>(pl, c, c_stride, bias, Ni, Gi, vec, pa, partial);
  return check_launch("slot_weights");
}
