// Shared helpers for the gfx950 KV-path kernels and their C-ABI wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "prism_kv.h"

namespace prism {

// ---------------------------------------------------------------- host side

void set_error(const char* fmt, ...);
void clear_error();

// Returns PRISM_ERR_HIP and records the message when `err` is an error.
int check_hip(hipError_t err, const char* what);

// Launch-error check after a kernel launch.
inline int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

// Per source file: load its code object on the current device (see prism_preload).
int preload_kv_store();
int preload_kv_compaction();
int preload_paged_prefill();
int preload_paged_decode();

int device_cu_count();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

inline bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

inline int dtype_size(int dtype) {
  switch (dtype) {
    case PRISM_DTYPE_F32: return 4;
    case PRISM_DTYPE_BF16: return 2;
    case PRISM_DTYPE_F16: return 2;
    case PRISM_DTYPE_FP8_E4M3FN: return 1;
    default: return 0;
  }
}

// ---------------------------------------------------------------- device side

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 / fp16 bit patterns -> fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16));
  return static_cast<float>(h);
}

// fp32 -> bf16 bits, round to nearest even (used for outputs only).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

// NaN-propagating max/min (IEEE 754-2019 maximum/minimum), matching
// torch.amax / torch.clamp on NaN inputs.
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float nan_min(float a, float b) { return __builtin_elementwise_minimum(a, b); }

// Four fp32 values -> four E4M3FN bytes (byte i from value i), round to
// nearest even with the native gfx950 conversion.  Magnitudes above 464 (the
// rounding midpoint between 448 and the NaN code) and NaNs become 0x7F with
// the input's sign bit: the same bytes torch's float8_e4m3fn cast produces.
__device__ __forceinline__ uint32_t fp8_encode4(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  int both = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
  uint32_t r = static_cast<uint32_t>(both);
  float v[4] = {a, b, c, d};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t bits = __float_as_uint(v[i]);
    bool to_nan = (bits & 0x7FFFFFFFu) > 0x43E80000u;  // |x| > 464, inf or NaN
    uint32_t nanb = 0x7Fu | ((bits >> 24) & 0x80u);
    uint32_t mask = 0xFFu << (8 * i);
    r = to_nan ? ((r & ~mask) | (nanb << (8 * i))) : r;
  }
  return r;
}

// Wave64 lane id.
__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace prism
