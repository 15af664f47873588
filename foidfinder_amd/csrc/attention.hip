// Non-causal flash attention, head_dim 64, fp16 in / fp32 accumulate, on gfx950 fp16 MFMA.
//
// Input is the QKV GEMM's output: qkv fp16 [S*L, 3C] with q already rotated and scaled by softmax_scale*log2(e) and
// k rotated, so the softmax is in base 2. One 256-thread workgroup = 4 waves x 32 queries of one (sequence, head).
// K and V stream through LDS in 64-key tiles (double-buffered; V stored transposed so the PV product reads
// contiguous keys). Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_f16, which leaves one query per lane
// and 32 keys per lane-pair, so the online softmax (running max, exp2, running sum) stays in registers with a
// single cross-lane exchange, and P^T feeds the PV MFMA (O^T = V^T P^T) directly as its column operand.
// Tails: query rows >= L are computed but not stored; keys >= L are masked to -inf.
//
// Reference: foidfinder/backends/cuda/csrc/attention.cuh:19-157 (which accumulates each 64-key block in fp16;
// here every product and sum is fp32).
#include "common.h"

namespace ff {

constexpr int HD = 64;
constexpr int BQ = 128;         // queries per workgroup
constexpr int BKV = 64;         // keys per tile
constexpr int VT_STRIDE = 68;   // halves per transposed-V row: 64 keys + 4 pad (136 B rows spread the banks)

// K tile rows of 128 B (8 chunks of 16 B), chunk XOR bits 1-3 of the row: the 16 lanes of one 16-byte LDS read pass
// (64 banks, 256 B) read 16 rows -> 2 rows per 256-byte window, spread over 16 distinct slots.
__device__ __forceinline__ int k_swz(int row, int chunk) { return row * HD + ((chunk ^ ((row >> 1) & 7)) << 3); }

__global__ __launch_bounds__(256) void attention_kernel(const half_t* __restrict__ qkv, half_t* __restrict__ out,
                                                        int L, int H) {
  __shared__ __attribute__((aligned(16))) half_t sK[2][BKV * HD];
  __shared__ __attribute__((aligned(16))) half_t sV[2][HD * VT_STRIDE];

  const int C = H * HD, ROW = 3 * C;
  // 1-D grid over (sequence, head, query block), query block fastest, remapped so that all query blocks of one
  // (sequence, head) run on one XCD and read its K and V through one L2.
  const int nq = (L + BQ - 1) / BQ;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = t % nq, h = (t / nq) % H, seq = t / (nq * H);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  const int64_t tok0 = static_cast<int64_t>(seq) * L;
  const half_t* qbase = qkv + tok0 * ROW + h * HD;
  const half_t* kbase = qbase + C;
  const half_t* vbase = qbase + 2 * C;

  // Q fragments (column operand of S^T): lane holds query q0 + fr, d = 16s + 8fh + 0..7.
  const int q0 = qb * BQ + wave * 32;
  const int qrow = min(q0 + fr, L - 1);
  half8_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qf[s] = *reinterpret_cast<const half8_t*>(qbase + static_cast<int64_t>(qrow) * ROW + 16 * s + 8 * fh);

  // Tile loads: 64 keys x 8 chunks of 8 halves for K and for V, two chunks of each per thread.
  half8_t rk[2], rv[2];
  auto gload = [&](int tile) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int idx = tid + 256 * p, key = min(tile * BKV + (idx >> 3), L - 1), c = idx & 7;
      rk[p] = *reinterpret_cast<const half8_t*>(kbase + static_cast<int64_t>(key) * ROW + c * 8);
      rv[p] = *reinterpret_cast<const half8_t*>(vbase + static_cast<int64_t>(key) * ROW + c * 8);
    }
  };
  auto swrite = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int idx = tid + 256 * p, key = idx >> 3, c = idx & 7;
      *reinterpret_cast<half8_t*>(&sK[buf][k_swz(key, c)]) = rk[p];
#pragma unroll
      for (int i = 0; i < 8; ++i) sV[buf][(c * 8 + i) * VT_STRIDE + key] = rv[p][i];
    }
  };

  float16_t o[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int ntiles = (L + BKV - 1) / BKV;
  gload(0);
  swrite(0);
  __syncthreads();
  for (int tile = 0; tile < ntiles; ++tile) {
    const int cur = tile & 1;
    if (tile + 1 < ntiles) gload(tile + 1);

    // S^T[key][q] for the tile's two 32-key halves: lane holds q = q0 + fr and keys 8(r/4) + 4fh + r%4.
    float16_t sc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[kt][r] = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const half8_t kf = *reinterpret_cast<const half8_t*>(&sK[cur][k_swz(kt * 32 + fr, 2 * s + fh)]);
        sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], sc[kt], 0, 0, 0);
      }
    }
    if (tile == ntiles - 1) {  // mask keys past the sequence end
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = tile * BKV + kt * 32 + 8 * (r >> 2) + 4 * fh + (r & 3);
          if (key >= L) sc[kt][r] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[kt][r]);
    mx = fmaxf(mx, xor_shuffle(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float corr = exp2f(m_run - m_new);
    m_run = m_new;
    half8_t pf[2][2];
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(sc[kt][r] - m_new);
        psum += p;
        pf[kt][r >> 3][r & 7] = static_cast<half_t>(p);
      }
    l_run = l_run * corr + psum;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= corr;

    // O^T[d][q] += V^T[d][keys] P^T[keys][q]. MFMA slot u of lane half fh is key 16t + 8(u/4) + 4fh + u%4 of the
    // 32-key half kt, both for the P^T registers (S^T rows 8t..8t+7) and for the V^T reads below.
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const half_t* vr = &sV[cur][(dt * 32 + fr) * VT_STRIDE + kt * 32 + 16 * t + 4 * fh];
          const half4_t lo = *reinterpret_cast<const half4_t*>(vr);
          const half4_t hi = *reinterpret_cast<const half4_t*>(vr + 8);
          const half8_t vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[kt][t], o[dt], 0, 0, 0);
        }
    if (tile + 1 < ntiles) swrite(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + xor_shuffle(l_run, 32);
  const float inv = 1.f / l_tot;
  const int q = q0 + fr;
  if (q < L) {
    half_t* orow = out + (tok0 + q) * C + h * HD;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4_t v;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = static_cast<half_t>(o[dt][4 * g + t] * inv);
        *reinterpret_cast<half4_t*>(orow + dt * 32 + 8 * g + 4 * fh) = v;
      }
  }
}

}  // namespace ff

using namespace ff;

extern "C" int ff_attention(const void* qkv, void* out, int64_t T, int64_t heads, int64_t seq_len, void* stream) {
  clear_error();
  if (heads <= 0 || heads > 65535) return fail(FF_EINVAL, "attention: need 0 < heads <= 65535");
  if (seq_len <= 0 || seq_len > 0x7fffffff) return fail(FF_EINVAL, "attention: need seq_len > 0");
  if (T < 0 || T % seq_len != 0) return fail(FF_EINVAL, "attention: T must be a multiple of seq_len");
  if (heads * 3 * HD * seq_len > (int64_t(1) << 40)) return fail(FF_EINVAL, "attention: too large");
  const int64_t seqs = T / seq_len;
  if (T == 0) return FF_OK;
  if (!qkv || !out) return fail(FF_EINVAL, "attention: null pointer");
  if ((reinterpret_cast<uintptr_t>(qkv) & 15) || (reinterpret_cast<uintptr_t>(out) & 7))
    return fail(FF_EINVAL, "attention: misaligned pointer");
  const int64_t blocks = (seq_len + BQ - 1) / BQ * heads * seqs;
  if (blocks > 0x7fffffff) return fail(FF_EINVAL, "attention: too many blocks");
  const dim3 grid(static_cast<unsigned>(blocks));
  attention_kernel<<<grid, 256, 0, as_stream(stream)>>>(static_cast<const half_t*>(qkv), static_cast<half_t*>(out),
                                                        static_cast<int>(seq_len), static_cast<int>(heads));
  return check_launch("attention");
}
