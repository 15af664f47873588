// Shared host and device helpers for the gfx950 kernels (wave64, MFMA, LDS).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "foidfinder_rocm.h"

namespace ff {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef int int16_t_v __attribute__((ext_vector_type(16)));

// ---- host-side error reporting (thread-local, read through ff_last_error) ----
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
int check_launch(const char* what);
// Workgroups of `kernel` (launched with `block` threads and `smem` dynamic LDS bytes) that the current device holds
// resident at once, over all CUs; cached per kernel, device and shape. 0 if the runtime cannot tell.
int64_t resident_blocks(const void* kernel, int block, size_t smem);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device helpers ----

// Workgroups are dispatched round-robin over the 8 XCDs (block b runs on XCD b % 8), each with its own L2. This
// bijection gives XCD x the contiguous run of logical work items [x*q + min(x, r), ...), so work items that share
// operands (GEMM tiles of one panel, query blocks of one attention head) share one L2.
__device__ __forceinline__ int xcd_remap(int b, int nblocks) {
  const int q = nblocks >> 3, r = nblocks & 7;
  const int x = b & 7, k = b >> 3;
  return x * q + (x < r ? x : r) + k;
}

// Value of lane (lane ^ mask) within the wave (ds_bpermute).
__device__ __forceinline__ float xor_shuffle(float v, int mask) { return __shfl_xor(v, mask, 64); }

// DPP controls: partner lane l ^ 1, l ^ 3 (quad_perm), l ^ 7 (row_half_mirror), l ^ 15 (row_mirror).
constexpr int DPP_XOR1 = 0xB1, DPP_XOR3 = 0x1B, DPP_XOR7 = 0x141, DPP_XOR15 = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Value of lane l ^ 16 within a 32-lane group (ds_swizzle bitmask mode: and 0x1F, or 0, xor 0x10).
__device__ __forceinline__ float swz_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

// Sum over the 64 lanes, in every lane: within each 32-lane half by one swizzle and four DPP steps (partners l ^ 16,
// ^ 15, ^ 7, ^ 3, ^ 1 cover all 32), then across the halves by one permute.
__device__ __forceinline__ float wave_sum(float v) {
  v = v + swz_xor16(v);
  v = v + dpp<DPP_XOR15>(v);
  v = v + dpp<DPP_XOR7>(v);
  v = v + dpp<DPP_XOR3>(v);
  v = v + dpp<DPP_XOR1>(v);
  return v + xor_shuffle(v, 32);
}

}  // namespace ff
