// MFMA-side helpers shared by the paged attention kernels (gfx950): exact
// fp8 -> bf16/f16 conversions in MFMA operand order, the transposed LDS read
// that feeds V to the PV MFMA, and the cross-group max of a 16-lane column.
#pragma once

#include "common.h"

namespace prism {

// Two fp8 bytes (the selected 16-bit half of `w`) -> bf16x2, exact.
template <bool HI>
__device__ __forceinline__ bf16x2 fp8x2_to_bf16x2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
}

template <bool HI>
__device__ __forceinline__ f16x2 fp8x2_to_f16x2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI);
}

// 8 fp8 bytes (two dwords) -> 8 bf16 in order.  Assembled from whole dwords
// (see fp8x4_to_bf16x4_bits for why lanes are not extracted one by one).
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
  const u32x4 r = {__builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<false>(w0)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<true>(w0)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<false>(w1)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<true>(w1))};
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ f16x8 fp8x8_to_f16x8(uint32_t w0, uint32_t w1) {
  const u32x4 r = {__builtin_bit_cast(uint32_t, fp8x2_to_f16x2<false>(w0)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_f16x2<true>(w0)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_f16x2<false>(w1)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_f16x2<true>(w1))};
  return __builtin_bit_cast(f16x8, r);
}

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void*)p));
}

// Four ds_read_b64_tr_b8 issued back to back with one lgkmcnt wait.  Written
// as asm because the compiler's waitcnt pass cannot tell this LDS read from
// the in-flight load-to-LDS of other stages and would drain the whole
// prefetch (vmcnt(0)) before it.
__device__ __forceinline__ void lds_read_tr8_x4(const uint32_t (&ad)[4], uint64_t (&out)[4]) {
  asm volatile(
      "ds_read_b64_tr_b8 %0, %4\n\t"
      "ds_read_b64_tr_b8 %1, %5\n\t"
      "ds_read_b64_tr_b8 %2, %6\n\t"
      "ds_read_b64_tr_b8 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3])
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3])
      : "memory");
}

// Eight transposed reads: the four addresses at byte offsets OFF0 and OFF1
// (immediates), one wait for all of them.
template <int OFF0, int OFF1>
__device__ __forceinline__ void lds_read_tr8_x8(const uint32_t (&ad)[4], uint64_t (&o0)[4], uint64_t (&o1)[4]) {
  static_assert(OFF0 >= 0 && OFF1 >= 0 && OFF0 < 65536 && OFF1 < 65536, "ds offsets are 16-bit");
  asm volatile(
      "ds_read_b64_tr_b8 %0, %8 offset:%12\n\t"
      "ds_read_b64_tr_b8 %1, %9 offset:%12\n\t"
      "ds_read_b64_tr_b8 %2, %10 offset:%12\n\t"
      "ds_read_b64_tr_b8 %3, %11 offset:%12\n\t"
      "ds_read_b64_tr_b8 %4, %8 offset:%13\n\t"
      "ds_read_b64_tr_b8 %5, %9 offset:%13\n\t"
      "ds_read_b64_tr_b8 %6, %10 offset:%13\n\t"
      "ds_read_b64_tr_b8 %7, %11 offset:%13\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(o0[0]), "=&v"(o0[1]), "=&v"(o0[2]), "=&v"(o0[3]), "=&v"(o1[0]), "=&v"(o1[1]), "=&v"(o1[2]),
        "=&v"(o1[3])
      : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "i"(OFF0), "i"(OFF1)
      : "memory");
}

// Max over the four 16-lane groups (lanes l, l^16, l^32, l^48) with the
// gfx950 lane-swap instructions (VALU, no LDS round trip).
__device__ __forceinline__ float wave_max_across_groups(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// The same with IEEE-754 maximum (NaN-propagating, v_maximum_f32): unlike
// fmaxf it needs no canonicalisation of values that arrive through lane
// swaps, so a kernel compiled in IEEE mode pays one instruction per step.
__device__ __forceinline__ float wave_maximum_across_groups(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

typedef short shortx4 __attribute__((ext_vector_type(4)));

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// 4 fp8 bytes (one dword) -> 4 f16, exact; assembled from whole dwords like
// fp8x4_to_bf16x4_bits below.
__device__ __forceinline__ f16x4 fp8x4_to_f16x4(uint32_t w) {
  const u32x2 r = {__builtin_bit_cast(uint32_t, fp8x2_to_f16x2<false>(w)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_f16x2<true>(w))};
  return __builtin_bit_cast(f16x4, r);
}

// 4 fp8 bytes (one dword) -> 4 bf16 bit patterns, exact.  Built from whole
// dwords: extracting single bf16 lanes of the converted pairs (bit_cast of
// element [1] to short) was lowered by this compiler (ROCm 7.2 clang) to a
// v_perm that duplicates element [0].
__device__ __forceinline__ shortx4 fp8x4_to_bf16x4_bits(uint32_t w) {
  const u32x2 r = {__builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<false>(w)),
                   __builtin_bit_cast(uint32_t, fp8x2_to_bf16x2<true>(w))};
  return __builtin_bit_cast(shortx4, r);
}

// Four fp32 values -> NT E4M3FN terms per value (largest first; one packed
// dword per term), each the round-to-nearest of what the previous terms
// left: four significant bits per term.  The fp8 MFMA's products of these
// with fp8 operands are exact in fp32, so the sum over the terms carries y.
// Every term lies on E4M3FN's grid, whose finest step is the subnormal
// 2^-9: whatever the number of terms, the error per value is at most 2^-10
// once the remainder falls below the normal range, and zero before.
template <int NT>
__device__ __forceinline__ void fp8_split(const float (&y)[4], uint32_t (&out)[NT]) {
  float r[4] = {y[0], y[1], y[2], y[3]};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], w, true);
    out[t] = static_cast<uint32_t>(w);
    if (t + 1 < NT) {
      const floatx2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
      const floatx2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
      r[0] -= lo[0];
      r[1] -= lo[1];
      r[2] -= hi[0];
      r[3] -= hi[1];
    }
  }
}

__device__ __forceinline__ void fp8_split3(const float (&y)[4], uint32_t (&out)[3]) { fp8_split<3>(y, out); }

}  // namespace prism
