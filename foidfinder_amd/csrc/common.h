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

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device helpers ----

// Round to nearest even, clamp to [-127, 127], and keep the low byte (two's complement).
__device__ __forceinline__ uint32_t q8(float v) {
  int q = static_cast<int>(__builtin_rintf(v));
  q = q < -127 ? -127 : (q > 127 ? 127 : q);
  return static_cast<uint32_t>(q) & 0xffu;
}

// Four codes packed little-endian into one dword.
__device__ __forceinline__ uint32_t q8x4(float a, float b, float c, float d) {
  return q8(a) | (q8(b) << 8) | (q8(c) << 16) | (q8(d) << 24);
}

// Value of lane (lane ^ mask) within the wave (ds_bpermute).
__device__ __forceinline__ float xor_shuffle(float v, int mask) { return __shfl_xor(v, mask, 64); }

}  // namespace ff
