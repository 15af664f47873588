// W8A8 GEMM with exact int32 accumulation on gfx950 int8 MFMA, and the fused fp16 epilogues.
//
// acc[m, n] = sum_k A[m, k] W[n, k]; A [M, K] and W [N, K] are int8 with K contiguous.
// y = fma((float)acc * row_scale[m], col_scale[n], bias[n]) - the reference's `acc * rs * cs + bias` as its CUDA
// compiler contracts it (gemm.cuh:135-136; this file is built with -ffp-contract=off, so every other operation rounds
// separately) - then the epilogue. The integer part is exact, so the order of the k-sum is free: each lane
// feeds the MFMA 16 contiguous bytes of K and the A- and W-fragments use the same k slots.
//
// Every variant computes the transposed product D[n][m] with v_mfma_i32_32x32x32_i8 (the W fragment is the row
// operand), each wave a 128 x 64 (or 64 x 64) sub-tile, so each lane ends with one output row m and runs of 4
// consecutive columns n: the pair epilogues (RoPE, SwiGLU) stay inside a lane, and the epilogue stages each wave's
// rows through LDS for 16-byte stores. K slices sit in LDS with their 16-byte chunks XOR-swizzled by row bits
// (conflict-free 16-byte fragment reads). The variant (the engine autotunes it per GEMM and batch size):
//
//  * 1, gemm_s8_kernel<128, 128>: 128 x 128 tiles, 4 waves, register-staged double buffering (small M).
//  * 2, gemm_s8_ring_kernel: 256 x 128 tiles, 4 waves, a 3-slot ring of K-64 slices filled by buffer loads straight
//    into LDS, two workgroups per CU.
//  * 3, gemm_s8_wide_kernel: 256 x 256 tiles, 8 waves (2 per SIMD), one workgroup per CU, a 2-slot ring of K-128
//    slices (4 slots of K 64 when K % 128 != 0).
//  * 4, gemm_s8_persist_kernel: variant 3's main loop on a persistent grid of one workgroup per CU whose ring runs on
//    across tiles; the rows past the last whole 256-row tile follow in 32 x 32 blocks, split-K (large M).
//  * 5, gemm_s8_wide_kernel<..., 128>: variant 3 on 256 x 128 tiles, each of its 8 waves a 64 x 64 sub-tile, with a
//    3-slot ring (narrow products at small M, where 256 x 256 tiles leave most CUs idle).
//  * 6, gemm_s8_ksplit_kernel: 64 x 64 blocks, each over all of K split across its 4 waves and summed through LDS
//    (small M, where even 256 x 128 tiles leave most CUs idle).
//
// Reference: foidfinder/backends/cuda/csrc/gemm.cuh:14-171 and kernels.cu:167-217.
#include <type_traits>

#include <algorithm>

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

constexpr uint32_t RSRC_WORD3 = 0x00020000;  // buffer descriptor word 3: raw dword access (gfx9 family)

// Raw buffer loads and stores through a descriptor over [base, base + nbytes): an access past the range reads zeros
// or is dropped, so bounds need no clamped addresses or branches, and the 32-bit lane offset plus a scalar base
// replaces 64-bit address arithmetic per access. Plain functions, so the descriptor type never appears in a
// template-dependent expression (the host pass of a template drops its kernel stubs otherwise). An offset of
// OOB_OFFSET is always out of range (nbytes <= INT32_MAX).
constexpr uint32_t OOB_OFFSET = 0x80000000u;
__device__ __forceinline__ int buf_bytes(int64_t bytes) {
  return static_cast<int>(bytes < 0 ? 0 : (bytes < 0x7fffffff ? bytes : 0x7fffffff));
}
__device__ __forceinline__ float4_t buf_load_f4(const void* base, int nbytes, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, RSRC_WORD3);
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ float buf_load_f1(const void* base, int nbytes, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, RSRC_WORD3);
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}
__device__ __forceinline__ half8_t buf_load_h8(const void* base, int nbytes, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, RSRC_WORD3);
  return __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ void buf_store_h8(half8_t v, void* base, int nbytes, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, nbytes, RSRC_WORD3);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4_t, v), r, voff, 0, 0);
}

// LDS rows of 64 bytes (4 chunks of 16 B); chunk index XOR-swizzled with bits 2-3 of the row. gfx950 serves a
// 16-byte-per-lane LDS read 16 lanes at a time from 64 four-byte banks (256 B), so the 16 rows read by 16 consecutive
// lanes must land in 16 distinct 16-byte slots of a 256-byte window: rows r..r+3 fill one window's 4 slots each, and
// the XOR with (r >> 2) & 3 spreads r, r+4, r+8, r+12 over the 4 chunk positions (measured: zero bank conflicts,
// where XOR with bits 1-2 doubles every read).
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 2) & 3)) << 4); }

// silu(g) = g / (1 + e^-g) from the hardware transcendental units: e^-g = v_exp_f32(-g log2 e) and the quotient as
// g * v_rcp_f32(1 + e^-g), each about 1 ulp, so silu(g) * value lands within one fp16 ulp of the correctly rounded
// result (the reference's own exp is a platform library call, mlx/kernels.py:45-49). Limits: g -> -inf gives
// e^-g = inf, rcp = 0, silu = -0; g -> +inf gives g.
__device__ __forceinline__ float silu(float g) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.f + e);
}

// The tanh GELU 0.5 y (1 + tanh(u)), u = sqrt(2/pi) (y + 0.044715 y^3), in the exactly equal form y / (1 + e^(-2u)),
// from the hardware exp2 and reciprocal (each about 1 ulp): within a few fp32 ulp of the exact value for every y (the
// form 0.5 y (1 + tanh(u)) cancels for negative y), where the reference itself evaluates tanh with a hardware
// approximation (common.cuh:50-56); ~8 instructions instead of a library tanhf with branches. Limits: y -> -inf
// gives e^(-2u) = inf, rcp = 0, gelu = -0; y -> +inf gives y.
__device__ __forceinline__ float gelu_tanh(float y) {
  constexpr float K1 = -2.f * 1.4426950408889634f * 0.7978845608f;  // -2 sqrt(2/pi) log2(e)
  constexpr float K3 = K1 * 0.044715f;
  const float t = __builtin_fmaf(K3, y * y, K1) * y;  // -2u log2(e)
  return y * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(t));
}

// Per-wave LDS staging area of store_epilogue: 32 rows of the wave's output columns, each row padded so that the
// writes of 32 lanes (32 rows, one column group) and the 16-byte row reads both spread over the 64 banks. fp16 rows
// (8-byte pad), except QKV, which stages the fp32 y (16-byte pad) and applies RoPE after the transpose to rows.
template <int EPI, int NI>
constexpr int stage_row_bytes() {
  if constexpr (EPI == FF_EPI_QKV_ROPE) return NI * 32 * 4 + 16;
  return (EPI == FF_EPI_SWIGLU ? NI * 16 : NI * 32) * 2 + 8;
}
template <int EPI, int NI>
constexpr int stage_bytes() {
  return 32 * stage_row_bytes<EPI, NI>();
}

// The epilogue of one wave: acc[i][j][4q + t] is D[n][m] with m = m_base + 32j + (lane & 31) and
// n = n_base + 32i + 8q + 4*(lane >> 5) + t. For each 32-row block j the wave computes y and the fp16 results in
// registers (pairs of columns are in-lane for SwiGLU), writes them to its LDS staging area, and then stores whole
// 16-byte row segments (for RESIDUAL: loads the matching residual segment and adds in fp16), so global stores are
// row-contiguous instead of 16 bytes per row. QKV stages y itself and rotates in the row layout, where the 8 lanes
// of a row read that row's RoPE table entries as 16-byte runs instead of 32 scattered rows per load. `stage` is this
// wave's private area of stage_bytes<EPI, NI>().
// Tile metadata staged in LDS (the persistent kernel): the tile's 256 column scales, 256 biases and 256 row scales,
// in that order, 1 KB each.
constexpr int META_BYTES = 3 * 1024;

template <int EPI, int NI, int MI>
__device__ __forceinline__ void store_epilogue(const int16_t_v (&acc)[NI][MI], int m_base, int n_base, int lane,
                                               const GemmArgs& args, uint8_t* stage, const uint8_t* meta = nullptr,
                                               int row0 = 0, int col0 = 0) {
  const int M = args.M, N = args.N;
  const int fr = lane & 31, fk = lane >> 5;
  if constexpr (EPI == FF_EPI_I32) {  // debug output: raw accumulators, stored from registers
#pragma unroll
    for (int j = 0; j < MI; ++j) {
      const int m = m_base + 32 * j + fr;
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n_base + 32 * i + 8 * q + 4 * fk;
          if (n >= N) continue;
          int4_t v;
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = acc[i][j][4 * q + t];
          *reinterpret_cast<int4_t*>(static_cast<int*>(args.out) + static_cast<int64_t>(m) * N + n) = v;
        }
    }
    return;
  } else {
    constexpr bool SWI = EPI == FF_EPI_SWIGLU;
    constexpr int RB = stage_row_bytes<EPI, NI>();
    constexpr int OUT_COLS = SWI ? NI * 16 : NI * 32;  // fp16 output columns of the wave
    constexpr int LANES_PER_ROW = OUT_COLS / 8;        // 16-byte segments per row
    constexpr int ROWS_PER_PASS = 64 / LANES_PER_ROW;
    const int out_ld = SWI ? N / 2 : N;
    const int out_n0 = SWI ? n_base / 2 : n_base;
    const int C3 = N / 3;  // QKV: section width
    // The wave's output rows m_base .. m_base + 32 MI - 1 through one descriptor that ends at row M: rows past M
    // (and the column-masked segments below) are dropped by the range check.
    half_t* o16 = static_cast<half_t*>(args.out) + static_cast<int64_t>(m_base) * out_ld;
    const int o_bytes = buf_bytes(static_cast<int64_t>(M - m_base) * out_ld * 2);
    // Scale and bias of the wave's 32 NI columns, loaded once per lane column group (i, q); past N they read zeros
    // (those columns are never stored).
    float4_t cs[NI][4], bi[NI][4];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t off = static_cast<uint32_t>(32 * i + 8 * q + 4 * fk) * 4;
        if (meta) {
          cs[i][q] = *reinterpret_cast<const float4_t*>(meta + col0 * 4 + off);
          bi[i][q] = *reinterpret_cast<const float4_t*>(meta + 1024 + col0 * 4 + off);
        } else {
          const int nb = buf_bytes(static_cast<int64_t>(N - n_base) * 4);
          cs[i][q] = buf_load_f4(args.col_scale + n_base, nb, off);
          bi[i][q] = buf_load_f4(args.bias + n_base, nb, off);
        }
      }
    // Per-row inputs are software-pipelined: the row scale of block j + 1 is loaded as soon as block j's results are
    // computed, and the residual rows (or RoPE table rows) of block j + 1 as soon as block j is stored, so their
    // latency hides behind the other phase. The staging area needs no barrier: one wave's LDS operations execute in
    // order.
    float rs = 0.f;
    half8_t xres[32 / ROWS_PER_PASS];
    float4_t tco[32 / ROWS_PER_PASS], tsi[32 / ROWS_PER_PASS];  // QKV: RoPE entries of the lane's 4 pairs
    // QKV store-phase geometry: the lane's 8 columns n .. n+7 hold pairs (n mod 64)/2 .. +3 of a q, k or v section
    const int seg_n = out_n0 + (lane % LANES_PER_ROW) * 8;
    const bool seg_rot = EPI == FF_EPI_QKV_ROPE && seg_n < 2 * C3;  // wave-uniform: sections are 64-aligned
    const bool seg_q = seg_n < C3;
    const int row_in_pass = lane / LANES_PER_ROW;
    // Byte offset of the lane's store segment in row r of the wave (r = 32 j + pass row); OOB_OFFSET masks segments
    // past the last column (N not a multiple of the wave's columns).
    const uint32_t seg_off = seg_n < out_ld ? static_cast<uint32_t>(seg_n) * 2 : OOB_OFFSET;
    auto row_off = [&](int r) __attribute__((always_inline)) {
      return seg_off == OOB_OFFSET ? OOB_OFFSET : static_cast<uint32_t>(r * out_ld) * 2 + seg_off;
    };
    auto load_row = [&](int j) __attribute__((always_inline)) {
      // rows past M read 0 (computed, never stored)
      if (meta)
        rs = *reinterpret_cast<const float*>(meta + 2048 + (row0 + 32 * j + fr) * 4);
      else
        rs = buf_load_f1(args.row_scale + m_base, buf_bytes(static_cast<int64_t>(M - m_base) * 4),
                         static_cast<uint32_t>(32 * j + fr) * 4);
    };
    // QKV: RoPE table row (m mod rope_len) of the lane's pass row, kept incrementally: the rows of block j, pass p
    // are rope_row0 + 32 j + p ROWS_PER_PASS (at most 32 MI - 1 past it), wrapped by at most one subtraction when
    // rope_len is larger than that span, else by a modulo.
    int rope_row0 = 0;
    if constexpr (EPI == FF_EPI_QKV_ROPE) rope_row0 = (m_base + row_in_pass) % args.rope_len;
    auto load_rope = [&](int j) __attribute__((always_inline)) {
      if constexpr (EPI == FF_EPI_QKV_ROPE) {
        if (seg_rot) {
          const int L = args.rope_len;
          const int tbytes = buf_bytes(static_cast<int64_t>(L) * 32 * 4);  // rope_len < 2^24 (checked on the host)
#pragma unroll
          for (int p = 0; p < 32 / ROWS_PER_PASS; ++p) {
            int r = rope_row0 + 32 * j + p * ROWS_PER_PASS;
            if (L >= 32 * MI)
              r = r >= L ? r - L : r;
            else
              r %= L;
            const uint32_t t = static_cast<uint32_t>(r * 32 + ((seg_n & 63) >> 1)) * 4;
            tco[p] = buf_load_f4(args.rope_cos, tbytes, t);
            tsi[p] = buf_load_f4(args.rope_sin, tbytes, t);
          }
        }
      }
    };
    auto load_residual = [&](int j) __attribute__((always_inline)) {
      if constexpr (EPI == FF_EPI_RESIDUAL) {
#pragma unroll
        for (int p = 0; p < 32 / ROWS_PER_PASS; ++p)
          xres[p] = buf_load_h8(o16, o_bytes, row_off(32 * j + p * ROWS_PER_PASS + row_in_pass));
      }
    };
    load_row(0);
    load_residual(0);
    load_rope(0);
#pragma unroll
    for (int j = 0; j < MI; ++j) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = 32 * i + 8 * q + 4 * fk;  // column within the wave's tile
          float y[4];
#pragma unroll
          for (int t = 0; t < 4; ++t)
            y[t] = __builtin_fmaf(static_cast<float>(acc[i][j][4 * q + t]) * rs, cs[i][q][t], bi[i][q][t]);
          if constexpr (SWI) {
            half2_t h;
            h[0] = static_cast<half_t>(silu(y[0]) * y[1]);
            h[1] = static_cast<half_t>(silu(y[2]) * y[3]);
            *reinterpret_cast<half2_t*>(stage + fr * RB + c) = h;  // output column c/2, 2 bytes each
          } else if constexpr (EPI == FF_EPI_QKV_ROPE) {
            *reinterpret_cast<float4_t*>(stage + fr * RB + 4 * c) = float4_t{y[0], y[1], y[2], y[3]};
          } else {
            if constexpr (EPI == FF_EPI_GELU_F16) {
#pragma unroll
              for (int t = 0; t < 4; ++t) y[t] = gelu_tanh(y[t]);
            }
            half4_t h;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              // y is rounded to fp32 first, then to fp16: opaque here, so the compiler cannot fold the last fma and
              // the conversion into one v_fma_mix (a single rounding straight to fp16, which differs in ~3e-5 of
              // the outputs from the two-step rounding of the reference)
              asm("" : "+v"(y[t]));
              h[t] = static_cast<half_t>(y[t]);
            }
            *reinterpret_cast<half4_t*>(stage + fr * RB + 2 * c) = h;
          }
        }
      if (j + 1 < MI) load_row(j + 1);
#pragma unroll
      for (int p = 0; p < 32 / ROWS_PER_PASS; ++p) {
        const int r = p * ROWS_PER_PASS + lane / LANES_PER_ROW;
        const int seg = lane % LANES_PER_ROW;
        half8_t h;
        if constexpr (EPI == FF_EPI_QKV_ROPE) {
          const float4_t ya = *reinterpret_cast<const float4_t*>(stage + r * RB + seg * 32);
          const float4_t yb = *reinterpret_cast<const float4_t*>(stage + r * RB + seg * 32 + 16);
          float v[8] = {ya[0], ya[1], ya[2], ya[3], yb[0], yb[1], yb[2], yb[3]};
          if (seg_rot) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const float y0 = v[2 * k], y1 = v[2 * k + 1], co = tco[p][k], si = tsi[p][k];
              v[2 * k] = y0 * co - y1 * si;
              v[2 * k + 1] = y0 * si + y1 * co;
            }
            if (seg_q) {  // q is scaled after the rotation; k is not (wave-uniform)
#pragma unroll
              for (int t = 0; t < 8; ++t) v[t] = v[t] * args.q_scale;
            }
          }
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            asm("" : "+v"(v[t]));  // two roundings (fp32, then fp16), never one fused v_fma_mix
            h[t] = static_cast<half_t>(v[t]);
          }
        } else {
          h = *reinterpret_cast<const half8_t*>(stage + r * RB + seg * 16);
        }
        if constexpr (EPI == FF_EPI_RESIDUAL) {
#pragma unroll
          for (int t = 0; t < 8; ++t) h[t] = h[t] + xres[p][t];
        }
        buf_store_h8(h, o16, o_bytes, row_off(32 * j + r));
      }
      if (j + 1 < MI) {
        load_residual(j + 1);
        load_rope(j + 1);
      }
    }
  }
}

typedef __attribute__((address_space(3))) void lds_void;

// ---------------- variant 2: 256 x 128 tiles, 3-stage buffer->LDS ring, 2 workgroups per CU ----------------
//
// Sized for gfx950's feeds: an L2->CU load rate of ~55 B/clk per CU against 8192 int8 ops/clk per CU asks for
// >= ~150 ops per loaded byte (a 256 x 128 tile gives 171), and each wave's 128 x 64 sub-tile needs 96 B/clk of the
// ~240 B/clk LDS read rate. 72 KB of LDS and <= 256 registers per lane let two workgroups share a CU, so one
// workgroup's epilogue runs while the other's MFMAs do. Loads are buffer loads straight into LDS whose descriptors
// end at row M (or N): rows past the matrix read as zeros and need no clamping, and the per-slice offset lives in
// the scalar descriptor, so the main loop spends no VALU on addresses.

constexpr int R_BM = 256, R_BN = 128;
constexpr int R_GROUP_M = 8;                 // m-tiles per tile group

// LDS row layout of a K slice of RK bytes (64: 4 chunks of 16 B, 32: 2 chunks). A 16-byte-per-lane read pass covers
// 16 rows and 64 banks: with 64-byte rows the chunk XOR bits 2-3 of the row spreads rows r, r+4, r+8, r+12; with
// 32-byte rows (8 rows per 256 B) the chunk XOR bit 3 of the row separates r from r+8.
template <int RK>
__device__ __forceinline__ int rswz(int row, int chunk) {
  if constexpr (RK == 64)
    return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
  else
    return row * 32 + ((chunk ^ ((row >> 3) & 1)) << 4);
}

// One 16-byte-per-lane buffer load into LDS through a raw descriptor of `nbytes` bytes at `base` (loads past it read
// zeros). A plain function, so the descriptor type never appears in a template-dependent expression: the host pass
// of HIP cannot instantiate those and would silently drop the kernel's launch stub.
__device__ __forceinline__ void buffer_to_lds(const void* base, int nbytes, uint8_t* lds_dst, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, RSRC_WORD3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_dst, 16, voff, 0, 0, 0);
}

// RK: K bytes per ring slot, S: ring depth (variant 2 runs RK = 64, S = 3: 72 KB). The prefetch distance is S - 2
// slots plus half a slot.
template <int EPI, int RK, int S>
__global__ __launch_bounds__(256, 2) void gemm_s8_ring_kernel(const GemmArgs args) {
  constexpr int WM = R_BM / 2, WN = R_BN / 2, MI = WM / 32, NI = WN / 32;
  constexpr int STAGE = (R_BM + R_BN) * RK;      // bytes per ring slot (24 KB or 12 KB)
  constexpr int LOADS = STAGE / (256 * 16);      // 16-byte loads per thread per slot (6 or 3)
  constexpr int A_BLOCKS = R_BM * RK / 1024;     // 1 KB blocks of A per slot; W blocks follow
  constexpr int CPR = RK / 16;                   // 16-byte chunks per row
  constexpr int HALVES = RK / 32;                // 32-byte MFMA k-steps per slot
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (args.M + R_BM - 1) / R_BM, tiles_n = (args.N + R_BN - 1) / R_BN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int per_group = R_GROUP_M * tiles_n;
  const int g = t / per_group, in_g = t % per_group;
  const int gm = min(R_GROUP_M, tiles_m - g * R_GROUP_M);
  const int tm = g * R_GROUP_M + in_g % gm, tn = in_g / gm;
  const int m0 = tm * R_BM, n0 = tn * R_BN;
  const int K = args.K, KT = K / RK;

  // Slot layout: A_BLOCKS blocks of 1 KB (A rows) then the W blocks. Wave w issues blocks w*LOADS .. +LOADS-1; lane
  // l of a block writes LDS bytes 16 l, i.e. row l / CPR, slot l % CPR, and fetches the chunk rswz() puts there.
  uint32_t voff[LOADS];
#pragma unroll
  for (int p = 0; p < LOADS; ++p) {
    const int blk = wave * LOADS + p;
    const int brow = (blk < A_BLOCKS ? blk : blk - A_BLOCKS) * (1024 / RK);
    const int row = brow + lane / CPR, slot = lane % CPR;
    voff[p] = static_cast<uint32_t>(row * K + ((rswz<RK>(row, slot) - row * RK)));
  }
  // descriptor sizes: the bytes from the tile's first row to the end of the matrix (capped; in-tile offsets are
  // below 256 K, far under the cap)
  const int64_t a_rows = static_cast<int64_t>(args.M - m0) * K, w_rows = static_cast<int64_t>(args.N - n0) * K;
  auto nrec = [](int64_t bytes) { return static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff); };
  auto issue = [&](int kt) __attribute__((always_inline)) {
    uint8_t* st = smem + (kt % S) * STAGE;
    const int kb = kt * RK;
    const int8_t* abase = args.A + static_cast<int64_t>(m0) * K + kb;
    const int8_t* wbase = args.W + static_cast<int64_t>(n0) * K + kb;
    const int an = nrec(a_rows - kb), wn_ = nrec(w_rows - kb);
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      const int blk = wave * LOADS + p;  // wave-uniform
      if (blk < A_BLOCKS)
        buffer_to_lds(abase, an, st + blk * 1024, voff[p]);
      else
        buffer_to_lds(wbase, wn_, st + blk * 1024, voff[p]);
    }
  };

  int16_t_v acc[NI][MI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < KT) issue(s);

  const int fr = lane & 31, fk = lane >> 5;
  int4_t xw0[NI], ya0[MI], xw1[NI], ya1[MI];
  // fragments of 32-byte k-step kk of slot kt
  auto read_frags = [&](int kt, int kk, int4_t (&xw)[NI], int4_t (&ya)[MI]) __attribute__((always_inline)) {
    const uint8_t* sa = smem + (kt % S) * STAGE;
    const uint8_t* sw = sa + R_BM * RK;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      xw[i] = *reinterpret_cast<const int4_t*>(sw + rswz<RK>(wn * WN + i * 32 + fr, 2 * kk + fk));
#pragma unroll
    for (int j = 0; j < MI; ++j)
      ya[j] = *reinterpret_cast<const int4_t*>(sa + rswz<RK>(wm * WM + j * 32 + fr, 2 * kk + fk));
  };
  auto mfmas = [&](const int4_t (&xw)[NI], const int4_t (&ya)[MI]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < MI; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xw[i], ya[j], acc[i][j], 0, 0, 0);
  };
  auto interleave = [] __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < NI + MI; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NI * MI - (NI + MI), 0);
  };
  // Slot kt + 1 has landed once at most the loads of the newer slots are outstanding; lgkmcnt(0): this thread's
  // fragment reads of older slots are complete, so after the barrier any of them may be refilled.
  auto wait_next = [&](auto steady) __attribute__((always_inline)) {
    if constexpr (decltype(steady)::value)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((S - 2) * LOADS) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };

  if (KT >= S - 1)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 2) * LOADS) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  read_frags(0, 0, xw0, ya0);

  // One slot per step. STEADY: slot kt + S - 1 exists and is issued into the ring position of slot kt - 1, whose
  // fragments every wave finished reading before the previous barrier. With RK = 64 the second k-step of slot kt is
  // read while the first one's MFMAs run, and the first k-step of slot kt + 1 (after its barrier) while the second
  // one's run; with RK = 32, slot kt + 1 is read while slot kt's MFMAs run. On the last slot the read-ahead hits a
  // stale ring position and is never used.
  auto step = [&](int kt, auto steady) __attribute__((always_inline)) {
    if constexpr (decltype(steady)::value) issue(kt + S - 1);
    if constexpr (HALVES == 2) {
      read_frags(kt, 1, xw1, ya1);
      mfmas(xw0, ya0);
      interleave();
      wait_next(steady);
      read_frags(kt + 1, 0, xw0, ya0);
      mfmas(xw1, ya1);
      interleave();
    } else {
      wait_next(steady);
      read_frags(kt + 1, 0, xw1, ya1);
      mfmas(xw0, ya0);
      interleave();
#pragma unroll
      for (int i = 0; i < NI; ++i) xw0[i] = xw1[i];
#pragma unroll
      for (int j = 0; j < MI; ++j) ya0[j] = ya1[j];
    }
  };
  int kt = 0;
  for (; kt + S - 1 < KT; ++kt) step(kt, std::true_type{});
  for (; kt < KT; ++kt) step(kt, std::false_type{});
  __syncthreads();  // every wave is done with the ring; reuse it as the epilogue staging area
  static_assert(4 * stage_bytes<FF_EPI_QKV_ROPE, NI>() <= S * STAGE, "staging must fit in the ring");
  store_epilogue<EPI, NI, MI>(acc, m0 + wm * WM, n0 + wn * WN, lane, args, smem + wave * stage_bytes<EPI, NI>());
}

template <int RK, int S>
static int launch_ring(const GemmArgs& a, int epi, hipStream_t st) {
  if (a.K % RK != 0) return fail(FF_EINVAL, "gemm_s8: K must be a multiple of the slice");
  const int64_t tiles = static_cast<int64_t>((a.M + R_BM - 1) / R_BM) * ((a.N + R_BN - 1) / R_BN);
  if (tiles > 0x7fffffff) return fail(FF_EINVAL, "gemm_s8: too many tiles");
  const dim3 grid(static_cast<unsigned>(tiles));
  switch (epi) {
    case FF_EPI_QKV_ROPE: gemm_s8_ring_kernel<FF_EPI_QKV_ROPE, RK, S><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_RESIDUAL: gemm_s8_ring_kernel<FF_EPI_RESIDUAL, RK, S><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_GELU_F16: gemm_s8_ring_kernel<FF_EPI_GELU_F16, RK, S><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_SWIGLU: gemm_s8_ring_kernel<FF_EPI_SWIGLU, RK, S><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_BIAS_F16: gemm_s8_ring_kernel<FF_EPI_BIAS_F16, RK, S><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_I32: gemm_s8_ring_kernel<FF_EPI_I32, RK, S><<<grid, 256, 0, st>>>(a); break;
    default: return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  }
  return check_launch("gemm_s8");
}

// ---------------- variant 3: 256 x 256 tiles, 8 waves, buffer->LDS ring ----------------
//
// Halves the load traffic per MFMA of the 256 x 128 ring (the CU's vector-memory path, not the MFMA, bounds that
// kernel): 8 waves (2 per SIMD, each a 128 x 64 sub-tile as before) share one 256 x 256 tile, one workgroup per CU
// with a 128 KB ring. RK = 128 reads whole 128-byte lines per row and slot (2 slots); RK = 64 keeps 4 slots.

template <int RK>
__device__ __forceinline__ int wswz(int row, int chunk) {
  if constexpr (RK == 128)
    return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);  // 8 rows per read pass window pair: rows r, r+2, ...
  else
    return rswz<RK>(row, chunk);
}

// BN_ = 256: each wave a 128 x 64 sub-tile (waves 2 x 4). BN_ = 128 (variant 5): each wave 64 x 64 (waves 4 x 2),
// one fragment read per MFMA instead of 0.75 but twice the tiles, for narrow products whose 256 x 256 tiles leave
// most CUs idle (PixAI's fc2 and proj at M = 5185, N = 1024: 84 tiles of 256 x 256, 168 of 256 x 128). Its 48 KB
// slots leave room for a third (144 KB), so the next two slices load while one computes: at small M the weights
// arrive cold from HBM, and one slice of prefetch does not cover that latency.
template <int EPI, int RK, int S, int BN_ = 256>
__global__ __launch_bounds__(512, 1) void gemm_s8_wide_kernel(const GemmArgs args) {
  constexpr int BM = 256, BN = BN_, WM = BN == 256 ? 128 : 64, WN = 64, MI = WM / 32, NI = WN / 32;
  constexpr int WCOLS = BN / WN;  // waves across the tile's columns
  constexpr int STAGE = (BM + BN) * RK;       // bytes per ring slot (64 KB or 32 KB)
  constexpr int LOADS = STAGE / (512 * 16);   // 16-byte loads per thread per slot (8 or 4)
  constexpr int A_BLOCKS = BM * RK / 1024;    // 1 KB blocks of A per slot; W blocks follow
  constexpr int CPR = RK / 16;                // 16-byte chunks per row
  constexpr int KSTEPS = RK / 32;             // 32-byte MFMA k-steps per slot
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WCOLS, wn = wave % WCOLS;
  const int tiles_m = (args.M + BM - 1) / BM, tiles_n = (args.N + BN - 1) / BN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int per_group = R_GROUP_M * tiles_n;
  const int g = t / per_group, in_g = t % per_group;
  const int gm = min(R_GROUP_M, tiles_m - g * R_GROUP_M);
  const int tm = g * R_GROUP_M + in_g % gm, tn = in_g / gm;
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = args.K, KT = K / RK;

  uint32_t voff[LOADS];
#pragma unroll
  for (int p = 0; p < LOADS; ++p) {
    const int blk = wave * LOADS + p;
    const int brow = (blk < A_BLOCKS ? blk : blk - A_BLOCKS) * (1024 / RK);
    const int row = brow + lane / CPR, slot = lane % CPR;
    voff[p] = static_cast<uint32_t>(row * K + ((wswz<RK>(row, slot) - row * RK)));
  }
  const int64_t a_rows = static_cast<int64_t>(args.M - m0) * K, w_rows = static_cast<int64_t>(args.N - n0) * K;
  auto nrec = [](int64_t bytes) { return static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff); };
  auto issue = [&](int kt) __attribute__((always_inline)) {
    uint8_t* st = smem + (kt % S) * STAGE;
    const int kb = kt * RK;
    const int8_t* abase = args.A + static_cast<int64_t>(m0) * K + kb;
    const int8_t* wbase = args.W + static_cast<int64_t>(n0) * K + kb;
    const int an = nrec(a_rows - kb), wn_ = nrec(w_rows - kb);
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      const int blk = wave * LOADS + p;  // wave-uniform
      if (blk < A_BLOCKS)
        buffer_to_lds(abase, an, st + blk * 1024, voff[p]);
      else
        buffer_to_lds(wbase, wn_, st + blk * 1024, voff[p]);
    }
  };

  int16_t_v acc[NI][MI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < KT) issue(s);

  const int fr = lane & 31, fk = lane >> 5;
  int4_t xw[2][NI], ya[2][MI];
  auto read_frags = [&](int kt, int kk, int b) __attribute__((always_inline)) {
    const uint8_t* sa = smem + (kt % S) * STAGE;
    const uint8_t* sw = sa + BM * RK;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      xw[b][i] = *reinterpret_cast<const int4_t*>(sw + wswz<RK>(wn * WN + i * 32 + fr, 2 * kk + fk));
#pragma unroll
    for (int j = 0; j < MI; ++j)
      ya[b][j] = *reinterpret_cast<const int4_t*>(sa + wswz<RK>(wm * WM + j * 32 + fr, 2 * kk + fk));
  };
  auto mfmas = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < MI; ++j)
#pragma unroll
      for (int i = 0; i < NI; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xw[b][i], ya[b][j], acc[i][j], 0, 0, 0);
  };
  auto interleave = [] __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < NI + MI; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NI * MI - (NI + MI), 0);
  };
  auto wait_next = [&](auto steady) __attribute__((always_inline)) {
    if constexpr (decltype(steady)::value)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((S - 2) * LOADS) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };

  if (KT >= S - 1)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 2) * LOADS) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  read_frags(0, 0, 0);

  // One slot per step: the k-steps of slot kt are computed in order, each while the next one's fragments are read;
  // before the last k-step, slot kt + 1 is waited for (and the barrier passed), so its first k-step is read while
  // slot kt's last one computes. STEADY: slot kt + S - 1 is issued first, into the ring position of slot kt - 1.
  auto step = [&](int kt, auto steady) __attribute__((always_inline)) {
    if constexpr (decltype(steady)::value) issue(kt + S - 1);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const int b = kk & 1;
      if (kk + 1 < KSTEPS) {
        read_frags(kt, kk + 1, b ^ 1);
      } else {
        wait_next(steady);
        read_frags(kt + 1, 0, b ^ 1);
      }
      mfmas(b);
      interleave();
    }
  };
  int kt = 0;
  for (; kt + S - 1 < KT; ++kt) step(kt, std::true_type{});
  for (; kt < KT; ++kt) step(kt, std::false_type{});
  __syncthreads();  // every wave is done with the ring; reuse it as the epilogue staging area
  static_assert(8 * stage_bytes<FF_EPI_QKV_ROPE, NI>() <= S * STAGE, "staging must fit in the ring");
  store_epilogue<EPI, NI, MI>(acc, m0 + wm * WM, n0 + wn * WN, lane, args, smem + wave * stage_bytes<EPI, NI>());
}

template <int RK, int S, int BN = 256>
static int launch_wide(const GemmArgs& a, int epi, hipStream_t st) {
  if (a.K % RK != 0) return fail(FF_EINVAL, "gemm_s8: K must be a multiple of the slice");
  const int64_t tiles = static_cast<int64_t>((a.M + 255) / 256) * ((a.N + BN - 1) / BN);
  if (tiles > 0x7fffffff) return fail(FF_EINVAL, "gemm_s8: too many tiles");
  const dim3 grid(static_cast<unsigned>(tiles));
  switch (epi) {
    case FF_EPI_QKV_ROPE: gemm_s8_wide_kernel<FF_EPI_QKV_ROPE, RK, S, BN><<<grid, 512, 0, st>>>(a); break;
    case FF_EPI_RESIDUAL: gemm_s8_wide_kernel<FF_EPI_RESIDUAL, RK, S, BN><<<grid, 512, 0, st>>>(a); break;
    case FF_EPI_GELU_F16: gemm_s8_wide_kernel<FF_EPI_GELU_F16, RK, S, BN><<<grid, 512, 0, st>>>(a); break;
    case FF_EPI_SWIGLU: gemm_s8_wide_kernel<FF_EPI_SWIGLU, RK, S, BN><<<grid, 512, 0, st>>>(a); break;
    case FF_EPI_BIAS_F16: gemm_s8_wide_kernel<FF_EPI_BIAS_F16, RK, S, BN><<<grid, 512, 0, st>>>(a); break;
    case FF_EPI_I32: gemm_s8_wide_kernel<FF_EPI_I32, RK, S, BN><<<grid, 512, 0, st>>>(a); break;
    default: return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  }
  return check_launch("gemm_s8");
}

// ---------------- the rows past the last whole 256-row tile (variant 4) ----------------
//
// M = 32 800 leaves 32 rows past 128 whole row tiles. As one more 256-row tile per column tile they would take a
// whole extra round of the persistent grid (4 tiles on 4 CUs for N = 1024, each with the full K loop: ~24 us of
// fc2's ~113 us). Instead, before its tiles, workgroup b of the persistent grid takes blocks b, b + G, ... of
// 32 of those rows x 32 columns (a separate launch would cost a launch gap and a ramp per GEMM), and splits K over its
// 8 waves in 128-byte chunks (wave w: chunks w, w + 8, ...). A wave stages each chunk of its 32 A rows and 32 W rows in its own two LDS
// buffers with buffer->LDS loads (whole 128-byte rows per 8 lanes, the next chunk loading while the current one is
// multiplied; rows past M or N read as zeros), the waves' int32 partial products are summed exactly through LDS, and
// wave 0 applies the same epilogue as the main kernel. No barrier until the sum: each wave touches only its buffers.
constexpr int T_CHUNK = 64 * 128;  // one staged chunk: 32 A rows + 32 W rows x 128 K bytes

template <int EPI>
__device__ __forceinline__ void tail_block(const GemmArgs& args, int m_first, int bx, int by, uint8_t* lds) {
  // lds: 8 * 2 * T_CHUNK bytes, [wave][2 buffers][64 rows x 128 B]
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 31, fk = lane >> 5;
  const int M = args.M, N = args.N, K = args.K, nch = K / 128;
  const int m0 = m_first + 32 * by, n0 = 32 * bx;
  const int a_bytes = buf_bytes(static_cast<int64_t>(M - m0) * K), w_bytes = buf_bytes(static_cast<int64_t>(N - n0) * K);
  const int8_t* abase = args.A + static_cast<int64_t>(m0) * K;
  const int8_t* wbase = args.W + static_cast<int64_t>(n0) * K;
  uint8_t* mine = lds + wave * 2 * T_CHUNK;
  // Load p of a chunk fills LDS rows 8p .. 8p + 7 (rows 0-31: A, 32-63: W); lane l writes physical 16-byte slot l % 8
  // of row 8p + l / 8, so it fetches the global chunk that the swizzle of wswz<128> puts there.
  auto load_chunk = [&](int c, uint8_t* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int row = 8 * p + (lane >> 3), slot = lane & 7;
      const uint32_t voff =
          static_cast<uint32_t>((row & 31) * K + c * 128 + ((slot ^ ((row >> 1) & 7)) << 4));
      if (p < 4)
        buffer_to_lds(abase, a_bytes, dst + p * 1024, voff);
      else
        buffer_to_lds(wbase, w_bytes, dst + p * 1024, voff);
    }
  };
  int16_t_v acc[1][1] = {};
  int b = 0;
  if (wave < nch) load_chunk(wave, mine);
  for (int c = wave; c < nch; c += 8, b ^= 1) {
    if (c + 8 < nch) {
      load_chunk(c + 8, mine + (b ^ 1) * T_CHUNK);  // that buffer's last reads finished in the previous chunk
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // chunk c has landed (only chunk c + 8's loads outstanding)
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const uint8_t* sb = mine + b * T_CHUNK;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int4_t ya = *reinterpret_cast<const int4_t*>(sb + wswz<128>(fr, 2 * kk + fk));
      const int4_t xw = *reinterpret_cast<const int4_t*>(sb + wswz<128>(32 + fr, 2 * kk + fk));
      acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xw, ya, acc[0][0], 0, 0, 0);
    }
  }
  // partial products: each wave into the start of its own buffers (its chunk reads are done)
  int* part = reinterpret_cast<int*>(mine) + lane * 16;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<int4_t*>(part + 4 * q) =
        int4_t{acc[0][0][4 * q], acc[0][0][4 * q + 1], acc[0][0][4 * q + 2], acc[0][0][4 * q + 3]};
  __syncthreads();
  if (wave != 0) return;
#pragma unroll 1
  for (int w = 1; w < 8; ++w) {
    const int* theirs = reinterpret_cast<const int*>(lds + w * 2 * T_CHUNK) + lane * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int4_t v = *reinterpret_cast<const int4_t*>(theirs + 4 * q);
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[0][0][4 * q + t] += v[t];
    }
  }
  // every partial product is in wave 0's registers now: its own buffers are the epilogue's staging area
  static_assert(stage_bytes<FF_EPI_QKV_ROPE, 1>() <= 2 * T_CHUNK, "staging must fit in wave 0's buffers");
  store_epilogue<EPI, 1, 1>(acc, m0, n0, lane, args, lds);
}

// ---------------- variant 6: 64 x 64 blocks, K split over the workgroup's 4 waves ----------------
//
// For products too small to fill the GPU with 256-wide tiles (EVA02-L at batch 1: fc2 at M = 1025, N = 1024 is 40
// tiles of 256 x 128 for 256 CUs): the tail blocks' scheme at 64 x 64 over the whole matrix, 272 blocks there. Wave w
// of the block's WV waves multiplies the 64-byte K chunks w, w + WV, ... of its 64 A rows and 64 W rows, each chunk
// staged in the wave's own 8 KB of LDS by buffer->LDS loads (rows past M or N read as zeros; the chunk's fragments go
// to registers before the wave's next chunk loads into the buffer). The int32 partial tiles are then summed exactly in
// two steps through the same LDS (the upper half of the waves hands theirs to the lower half, then each of waves 0-3
// sums one 32 x 32 quadrant over those) and each of waves 0-3 applies the epilogue to its quadrant. With WV = 4 a
// block takes 32 KB and at most 128 VGPRs, so four share a CU and 1024 are resident (EVA02-L's qkv at batch 1 is 816
// blocks). Measured at batch 1 (fc2 / proj / qkv): 11.1 / 6.5 / 11.2 us; the same kernel with 8 waves per block (64
// KB, two per CU) ran 12.8 / 7.8 / 13.8.
constexpr int KS_CHUNK = 128 * 64;     // one staged chunk: 64 A rows + 64 W rows x 64 K bytes
constexpr int KS_PART = 64 * 64 * 4;   // one wave's 64 x 64 int32 partial tile

template <int EPI>
__global__ __launch_bounds__(256, 4) void gemm_s8_ksplit_kernel(const GemmArgs args) {
  constexpr int WV = 4;          // waves per block
  constexpr int SLOTS = WV / 2;  // partial slots in the chunk buffers
  static_assert(stage_bytes<EPI, 1>() <= KS_CHUNK, "a quadrant's staging fits its wave's chunk buffer");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[WV * KS_CHUNK];  // chunks, then partials, then staging
  static_assert(WV * KS_CHUNK == SLOTS * KS_PART, "the partial slots fill the chunk buffers");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 31, fk = lane >> 5;
  const int M = args.M, N = args.N, K = args.K, nch = K / 64;
  const int tiles_n = (N + 63) / 64;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (t / tiles_n) * 64, n0 = (t % tiles_n) * 64;
  const int a_bytes = buf_bytes(static_cast<int64_t>(M - m0) * K), w_bytes = buf_bytes(static_cast<int64_t>(N - n0) * K);
  const int8_t* abase = args.A + static_cast<int64_t>(m0) * K;
  const int8_t* wbase = args.W + static_cast<int64_t>(n0) * K;
  uint8_t* mine = lds + wave * KS_CHUNK;
  // Load p of a chunk fills LDS rows 16p .. 16p + 15 (rows 0-63: A, 64-127: W); lane l writes physical 16-byte slot
  // l % 4 of row 16p + l / 4, so it fetches the global chunk that the swizzle of rswz<64> puts there.
  auto load_chunk = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int row = 16 * p + (lane >> 2), slot = lane & 3;
      const uint32_t voff = static_cast<uint32_t>((row & 63) * K + c * 64 + ((slot ^ ((row >> 2) & 3)) << 4));
      if (p < 4)
        buffer_to_lds(abase, a_bytes, mine + p * 1024, voff);
      else
        buffer_to_lds(wbase, w_bytes, mine + p * 1024, voff);
    }
  };
  int16_t_v acc[2][2] = {};
  if (wave < nch) load_chunk(wave);
  for (int c = wave; c < nch; c += WV) {
    // the chunk's fragments into registers, then the buffer takes the wave's next chunk while these multiply
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int4_t xw[2][2], ya[2][2];  // [k-step][block]
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        xw[kk][i] = *reinterpret_cast<const int4_t*>(mine + rswz<64>(64 + 32 * i + fr, 2 * kk + fk));
#pragma unroll
      for (int j = 0; j < 2; ++j) ya[kk][j] = *reinterpret_cast<const int4_t*>(mine + rswz<64>(32 * j + fr, 2 * kk + fk));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (c + WV < nch) load_chunk(c + WV);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xw[kk][i], ya[kk][j], acc[i][j], 0, 0, 0);
  }
  // A partial tile in slot s: quadrant (i, j) at 4 KB (2 i + j), 16-byte chunk q of lane l at 1 KB q + 16 l.
  auto put = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<int4_t*>(lds + s * KS_PART + (2 * i + j) * 4096 + q * 1024 + lane * 16) =
              int4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
  };
  __syncthreads();  // every wave is done with its chunk buffer
  // step 1: the upper half of the waves hands its partials to the lower half
  if (wave >= SLOTS) put(wave - SLOTS);
  __syncthreads();
  if (wave < SLOTS) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int4_t v = *reinterpret_cast<const int4_t*>(lds + wave * KS_PART + (2 * i + j) * 4096 + q * 1024 + lane * 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
        }
  }
  __syncthreads();  // the lower half has read the slots it now overwrites
  // step 2: the lower half's sums into the slots; waves 0-3 each sum one quadrant over them
  if (wave < SLOTS) put(wave);
  __syncthreads();
  const int qi = (wave >> 1) & 1, qj = wave & 1;  // waves 0-3: the quadrant, column block qi, row block qj
  int16_t_v sum[1][1] = {};
  if (wave < 4) {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4_t v = *reinterpret_cast<const int4_t*>(lds + s * KS_PART + (2 * qi + qj) * 4096 + q * 1024 + lane * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[0][0][4 * q + e] += v[e];
      }
  }
  __syncthreads();  // every quadrant is read: the chunk buffers become the epilogue's staging areas
  if (wave >= 4) return;
  store_epilogue<EPI, 1, 1>(sum, m0 + 32 * qj, n0 + 32 * qi, lane, args, lds + wave * KS_CHUNK);
}

static int launch_ksplit(const GemmArgs& a, int epi, hipStream_t st) {
  const int64_t blocks = static_cast<int64_t>((a.M + 63) / 64) * ((a.N + 63) / 64);
  if (blocks > 0x7fffffff) return fail(FF_EINVAL, "gemm_s8: too many tiles");
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (epi) {
    case FF_EPI_QKV_ROPE: gemm_s8_ksplit_kernel<FF_EPI_QKV_ROPE><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_RESIDUAL: gemm_s8_ksplit_kernel<FF_EPI_RESIDUAL><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_GELU_F16: gemm_s8_ksplit_kernel<FF_EPI_GELU_F16><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_SWIGLU: gemm_s8_ksplit_kernel<FF_EPI_SWIGLU><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_BIAS_F16: gemm_s8_ksplit_kernel<FF_EPI_BIAS_F16><<<grid, 256, 0, st>>>(a); break;
    case FF_EPI_I32: gemm_s8_ksplit_kernel<FF_EPI_I32><<<grid, 256, 0, st>>>(a); break;
    default: return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  }
  return check_launch("gemm_s8");
}

// ---------------- variant 4: persistent 256 x 256, 8 waves, one workgroup per CU ----------------
//
// The variant-3 main loop (two 64 KB slots of K 128), with the ring running on across tiles: the grid holds one
// workgroup per CU, each takes every G-th tile of the grouped order, and slices are one stream, so the next tile's
// first slice loads under the current tile's last MFMAs and its first fragments are read before the epilogue. No
// workgroup starts cold, and row tiles that reach past M are ordered last (their rows past M load as zeros, and
// MFMAs on zeros draw less power, so the partial last round runs at a higher clock). A tile's column scales, biases
// and row scales load into LDS with its first slice (buffer->LDS, three waves, 1 KB each), so the epilogue reads
// them from LDS instead of waiting ~2000 cycles for global loads issued at its start. The epilogue stages through
// the ring slot of the tile's last slice, which no load targets until the barrier after the epilogue; when eight
// staging areas do not fit in one slot (QKV), the last ones use a spare area past the ring. SwiGLU's small staging
// areas (18 KB for eight waves) sit past the ring instead, so its waves skip that barrier: a wave that finishes its
// epilogue early starts the next tile's products while slower waves finish theirs, and the next slice barrier
// joins them (measured per wave with s_memtime at fc1's batch-32 shape: the barrier had cost ~2000 cycles per tile
// of waiting for the slowest wave).

template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_s8_persist_kernel(const GemmArgs args, int m_full) {
  constexpr int RK = 128, BM = 256, BN = 256, WM = 128, WN = 64, MI = WM / 32, NI = WN / 32;
  constexpr int STAGE = (BM + BN) * RK;      // 64 KB per ring slot, two slots
  constexpr int LOADS = STAGE / (512 * 16);  // 16-byte loads per thread per slot
  constexpr int A_BLOCKS = BM * RK / 1024;   // 1 KB blocks of A per slot; W blocks follow
  constexpr int CPR = RK / 16;               // 16-byte chunks per row
  constexpr int KSTEPS = RK / 32;            // 32-byte MFMA k-steps per slot (even: a slot starts in buffer 0)
  constexpr int SB = stage_bytes<EPI, NI>();
  // The tile metadata (column scales, biases, row scales) loads into LDS with the tile's first slice, into one of
  // two buffers by tile parity. SwiGLU's staging areas fit beside the ring, so its waves need not wait for each other
  // after the epilogue; the other epilogues stage through the free ring slot (the last slots past the ring when
  // eight areas do not fit in it).
  constexpr bool META = EPI != FF_EPI_I32;
  constexpr bool OWN_STAGE = EPI == FF_EPI_SWIGLU;
  constexpr int FIT = OWN_STAGE ? 0 : (STAGE / SB < 8 ? STAGE / SB : 8);
  constexpr int META_OFF = 2 * STAGE;
  constexpr int STAGE_OFF = META_OFF + 2 * META_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGE_OFF + (8 - FIT) * SB];
  static_assert(STAGE_OFF + (8 - FIT) * SB <= 160 * 1024, "LDS");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int M = args.M, N = args.N, K = args.K, KT = K / RK;
  const int tiles_n = (N + BN - 1) / BN, full_m = M / BM, tiles_m = (M + BM - 1) / BM;
  const int ntiles = tiles_m * tiles_n, G = gridDim.x;
  const int first = xcd_remap(blockIdx.x, G);  // this workgroup's tiles: first, first + G, ...
  const int my_tiles = first < ntiles ? (ntiles - 1 - first) / G + 1 : 0;
  const int total = my_tiles * KT;             // slices this workgroup streams
  // Tile r of this workgroup: full row tiles in groups of R_GROUP_M row tiles (column-major inside a group), then
  // the partial row tile.
  auto coords = [&](int r, int& m0, int& n0) __attribute__((always_inline)) {
    const int L = first + r * G;
    if (L < full_m * tiles_n) {
      const int per_group = R_GROUP_M * tiles_n;
      const int g = L / per_group, in_g = L % per_group;
      const int gm = min(R_GROUP_M, full_m - g * R_GROUP_M);
      m0 = (g * R_GROUP_M + in_g % gm) * BM;
      n0 = (in_g / gm) * BN;
    } else {
      m0 = full_m * BM;
      n0 = (L - full_m * tiles_n) * BN;
    }
  };

  auto nrec = [](int64_t bytes) { return static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff); };
  // Load side: slice `ig` (kt `ikt` of tile `ir`, at rows im0 / columns in0) goes to ring slot ig & 1.
  int ig = 0, ir = 0, ikt = 0, im0 = 0, in0 = 0;
  if (my_tiles > 0) coords(0, im0, in0);
  auto issue = [&]() __attribute__((always_inline)) {
    uint8_t* st = smem + (ig & 1) * STAGE;
    const int kb = ikt * RK;
    const int8_t* abase = args.A + static_cast<int64_t>(im0) * K + kb;
    const int8_t* wbase = args.W + static_cast<int64_t>(in0) * K + kb;
    const int an = nrec(static_cast<int64_t>(M - im0) * K - kb), wn_ = nrec(static_cast<int64_t>(N - in0) * K - kb);
    // Lane offsets are recomputed per slice from an opaque copy of the lane index (a few VALU per load) instead of
    // being held in registers, which would stay live through the epilogue.
    int l = lane;
    asm volatile("" : "+v"(l));
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      const int blk = wave * LOADS + p;  // wave-uniform
      const int row = (blk < A_BLOCKS ? blk : blk - A_BLOCKS) * (1024 / RK) + l / CPR, chunk = l % CPR;
      const uint32_t voff = static_cast<uint32_t>(row * K + ((wswz<RK>(row, chunk) - row * RK)));
      if (blk < A_BLOCKS)
        buffer_to_lds(abase, an, st + blk * 1024, voff);
      else
        buffer_to_lds(wbase, wn_, st + blk * 1024, voff);
    }
    if constexpr (META) {
      if (ikt == 0 && wave < 3) {  // the tile's metadata, 1 KB per wave: column scales, biases, row scales
        uint8_t* md = smem + META_OFF + (ir & 1) * META_BYTES + wave * 1024;
        const int nb = nrec(static_cast<int64_t>(N - in0) * 4);
        if (wave == 0)
          buffer_to_lds(args.col_scale + in0, nb, md, static_cast<uint32_t>(lane) * 16);
        else if (wave == 1)
          buffer_to_lds(args.bias + in0, nb, md, static_cast<uint32_t>(lane) * 16);
        else
          buffer_to_lds(args.row_scale + im0, nrec(static_cast<int64_t>(M - im0) * 4), md,
                        static_cast<uint32_t>(lane) * 16);
      }
    }
    ++ig;
    if (++ikt == KT) {
      ikt = 0;
      if (++ir < my_tiles) coords(ir, im0, in0);
    }
  };

  // No zero fill: a tile's first k-step writes the accumulators from an inline-constant zero C operand.
  int16_t_v acc[NI][MI];

  const int fr = lane & 31, fk = lane >> 5;
  int4_t xw[2][NI], ya[2][MI];
  auto read_frags = [&](int g, int kk, int b) __attribute__((always_inline)) {
    const uint8_t* sa = smem + (g & 1) * STAGE;
    const uint8_t* sw = sa + BM * RK;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      xw[b][i] = *reinterpret_cast<const int4_t*>(sw + wswz<RK>(wn * WN + i * 32 + fr, 2 * kk + fk));
#pragma unroll
    for (int j = 0; j < MI; ++j)
      ya[b][j] = *reinterpret_cast<const int4_t*>(sa + wswz<RK>(wm * WM + j * 32 + fr, 2 * kk + fk));
  };

  // The rows M .. m_full - 1 past the whole row tiles, in 32 x 32 blocks over the grid (see tail_block), before the
  // tiles: after them, a block's first wait on its loads would also wait for the stores of the workgroup's last
  // tile (a wave's memory operations complete in order), i.e. for the drain of every CU's last output burst.
  if (m_full > M) {
    GemmArgs ta = args;
    ta.M = m_full;
    const int gx = (N + 31) / 32, nb = gx * ((m_full - M + 31) / 32);
    if (static_cast<int>(blockIdx.x) < nb) {
      for (int t = static_cast<int>(blockIdx.x); t < nb; t += G) {
        __syncthreads();  // every wave is past its last reads of the LDS that tail_block now fills
        tail_block<EPI>(ta, M, t % gx, t / gx, smem);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();  // the tail's LDS buffers overlap the ring's first slot
    }
  }
  if (total > 0) {
    issue();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    read_frags(0, 0, 0);
  }
  int r = 0, m0 = 0, n0 = 0;
  coords(0, m0, n0);
  // Slice g: slice g + 1 is issued into the other slot (free: every wave passed the barrier after reading it);
  // the k-steps run in order, each while the next one's fragments are read; before the last one, slice g + 1 is
  // waited for (and the barrier passed), so its first fragments are read while slice g's last k-step computes.
  // After a tile's last slice they are read once more after the epilogue; after the final slice the reads hit a
  // stale slot and are never used. FIRST: the tile's first slice, whose first k-step starts from C = 0.
  auto slice = [&](int g, auto first_c) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_c)::value;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const int b = kk & 1;
      if (kk + 1 < KSTEPS) {
        read_frags(g, kk + 1, b ^ 1);
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        read_frags(g + 1, 0, b ^ 1);
      }
      const int16_t_v zero = {};
#pragma unroll
      for (int j = 0; j < MI; ++j)
#pragma unroll
        for (int i = 0; i < NI; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xw[b][i], ya[b][j], FIRST && kk == 0 ? zero : acc[i][j],
                                                            0, 0, 0);
#pragma unroll
      for (int x = 0; x < NI + MI; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, NI * MI - (NI + MI), 0);
    }
  };
  for (int g = 0; g < total;) {
    // one tile: KT slices, the first one peeled (it starts the accumulators from zero)
    if (g + 1 < total) issue();
    slice(g, std::true_type{});
    ++g;
    for (int kt = 1; kt < KT; ++kt, ++g) {
      if (g + 1 < total) issue();
      slice(g, std::false_type{});
    }
    // Every wave has read all of the tile's last slice g - 1 (barrier above): its slot is the staging area until
    // the barrier below, after which slice g + 1 may load into it.
    uint8_t* stage = wave < FIT ? smem + ((g - 1) & 1) * STAGE + wave * SB : smem + STAGE_OFF + (wave - FIT) * SB;
    // An opaque lane index keeps the epilogue's lane-derived offsets from being hoisted out of the tile loop,
    // where they would hold registers through the main loop.
    int el = lane;
    asm volatile("" : "+v"(el));
    const uint8_t* md = META ? smem + META_OFF + (r & 1) * META_BYTES : nullptr;
    store_epilogue<EPI, NI, MI>(acc, m0 + wm * WM, n0 + wn * WN, el, args, stage, md, wm * WM, wn * WN);
    // Staging in the ring slot: every wave must be done with it before the next slice loads into it. With their own
    // staging areas the waves go on (the next tile's first slice barrier joins them), except for one-slice tiles,
    // whose next metadata load could overwrite the buffer a slower wave still reads.
    if (!OWN_STAGE || KT < 2) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
    }
    // The next slice's first fragments again: the copies read above are dead on this path, so they do not stay
    // live through the epilogue.
    read_frags(g, 0, 0);
    if (++r < my_tiles) coords(r, m0, n0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

static int launch_persist(const GemmArgs& args, int epi, hipStream_t st) {
  if (args.K % 128 != 0) return fail(FF_EINVAL, "gemm_s8: K must be a multiple of the slice");
  // Whole 256-row tiles on the persistent grid; the rows past them (if any) in 32-row blocks after its tiles.
  const int whole = args.M / 256 * 256;
  const bool split = whole > 0 && whole < args.M;
  GemmArgs a = args;
  if (split) a.M = whole;
  const int m_full = args.M;
  const int64_t tiles = static_cast<int64_t>((a.M + 255) / 256) * ((a.N + 255) / 256);
  if (tiles > 0x7fffffff) return fail(FF_EINVAL, "gemm_s8: too many tiles");
  const void* kernels[] = {
      reinterpret_cast<const void*>(&gemm_s8_persist_kernel<FF_EPI_QKV_ROPE>),
      reinterpret_cast<const void*>(&gemm_s8_persist_kernel<FF_EPI_RESIDUAL>),
      reinterpret_cast<const void*>(&gemm_s8_persist_kernel<FF_EPI_GELU_F16>),
      reinterpret_cast<const void*>(&gemm_s8_persist_kernel<FF_EPI_SWIGLU>),
      reinterpret_cast<const void*>(&gemm_s8_persist_kernel<FF_EPI_BIAS_F16>),
      reinterpret_cast<const void*>(&gemm_s8_persist_kernel<FF_EPI_I32>),
  };
  int64_t resident = resident_blocks(kernels[epi - FF_EPI_QKV_ROPE], 512, 0);
  if (resident <= 0) resident = 256;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(tiles, resident)));
  switch (epi) {
    case FF_EPI_QKV_ROPE: gemm_s8_persist_kernel<FF_EPI_QKV_ROPE><<<grid, 512, 0, st>>>(a, m_full); break;
    case FF_EPI_RESIDUAL: gemm_s8_persist_kernel<FF_EPI_RESIDUAL><<<grid, 512, 0, st>>>(a, m_full); break;
    case FF_EPI_GELU_F16: gemm_s8_persist_kernel<FF_EPI_GELU_F16><<<grid, 512, 0, st>>>(a, m_full); break;
    case FF_EPI_SWIGLU: gemm_s8_persist_kernel<FF_EPI_SWIGLU><<<grid, 512, 0, st>>>(a, m_full); break;
    case FF_EPI_BIAS_F16: gemm_s8_persist_kernel<FF_EPI_BIAS_F16><<<grid, 512, 0, st>>>(a, m_full); break;
    case FF_EPI_I32: gemm_s8_persist_kernel<FF_EPI_I32><<<grid, 512, 0, st>>>(a, m_full); break;
    default: return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  }
  return check_launch("gemm_s8");
}

// ---------------- variant 1: 128 x 128 tiles, register-staged double buffering ----------------

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256) void gemm_s8_kernel(const GemmArgs args) {
  constexpr int WM = BM / 2, WN = BN / 2;     // wave sub-tile
  constexpr int MI = WM / 32, NI = WN / 32;   // 32x32 MFMA blocks per wave
  constexpr int A_LD = BM * (BK / 16) / 256;  // 16-byte chunks per thread per slice
  constexpr int W_LD = BN * (BK / 16) / 256;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int SMEM = 2 * STAGE > 4 * stage_bytes<FF_EPI_QKV_ROPE, NI>() ? 2 * STAGE : 4 * stage_bytes<FF_EPI_QKV_ROPE, NI>();
  __shared__ __attribute__((aligned(16))) int8_t smem[SMEM];

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
  store_epilogue<EPI, NI, MI>(acc, m0 + wm * WM, n0 + wn * WN, lane, args,
                              reinterpret_cast<uint8_t*>(smem) + wave * stage_bytes<EPI, NI>());
}

template <int BM, int BN>
static int launch_staged(const GemmArgs& a, int epi, hipStream_t st) {
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

// 1: 128 x 128 register-staged; 2: 256 x 128 buffer->LDS ring (3 slots of K 64), two workgroups per CU;
// 3: 256 x 256, 8 waves, one workgroup per CU (2 slots of K 128, or 4 slots of K 64 when K % 128 != 0);
// 4: variant 3 as a persistent grid, the ring streaming across tiles (4 slots of K 64, not persistent, when
// K % 128 != 0); 5: variant 3 on 256 x 128 tiles of 64 x 64 per wave, 3 slots of K 128; 6: 64 x 64 blocks with K
// split over 4 waves. These are the variants the engine's autotune picks at the served shapes (1, 5 and 6
// for small M, 2, 3 and 5 for mid-sized M and the narrower GEMMs, 4 for large M).
constexpr int kVariants = 6;

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
  // offsets inside a tile's 256 rows of A or W (and of the output) are 32-bit byte offsets
  if (K > (int64_t(1) << 22) || N > (int64_t(1) << 21))
    return fail(FF_EINVAL, "gemm_s8: K above 2^22 or N above 2^21 is not supported");
  if (epi < FF_EPI_QKV_ROPE || epi > FF_EPI_I32) return fail(FF_EINVAL, "gemm_s8: bad epilogue");
  if (variant < 0 || variant > kVariants) return fail(FF_EINVAL, "gemm_s8: bad variant");
  if (epi == FF_EPI_QKV_ROPE) {
    if (N % 3 != 0 || (N / 3) % 64 != 0) return fail(FF_EINVAL, "gemm_s8: QKV epilogue needs N = 3C with C % 64 == 0");
    if (!rope_cos || !rope_sin || rope_len <= 0) return fail(FF_EINVAL, "gemm_s8: QKV epilogue needs RoPE tables");
    if (rope_len >= (int64_t(1) << 24)) return fail(FF_EINVAL, "gemm_s8: rope_len >= 2^24 is not supported");
    if (!aligned(rope_cos, 16) || !aligned(rope_sin, 16)) return fail(FF_EINVAL, "gemm_s8: misaligned RoPE tables");
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
  // The default follows the autotune's usual picks: K-split 64 x 64 blocks while they fill the GPU, 256 x 256 tiles
  // for mid-size M, the persistent grid from a few tiles per CU on.
  if (variant == 0) variant = M < 4096 ? 6 : (M < 16384 ? 3 : 4);
  switch (variant) {
    case 1: return launch_staged<128, 128>(a, epi, st);
    case 2: return launch_ring<64, 3>(a, epi, st);
    case 3: return a.K % 128 == 0 ? launch_wide<128, 2>(a, epi, st) : launch_wide<64, 4>(a, epi, st);
    case 4: return a.K % 128 == 0 ? launch_persist(a, epi, st) : launch_wide<64, 4>(a, epi, st);
    case 5: return a.K % 128 == 0 ? launch_wide<128, 3, 128>(a, epi, st) : launch_wide<64, 4, 128>(a, epi, st);
    case 6: return launch_ksplit(a, epi, st);
  }
  return fail(FF_EINVAL, "gemm_s8: bad variant");
}
