// KV store: bf16/fp16/fp32 K and V -> paged cache slots.
//
// Scaled FP8 (the hot path) restates the per-(token, kv head) quantiser of
// prism_infer/ops/kv_cache_store.py:81-167 (Triton) / :205-227 (eager):
//     s = max(amax|x| / 448, 1e-6)      fp32, IEEE division
//     q = e4m3fn(clamp(x / s, -448, 448))
// bit-exactly against the eager path (correctly rounded division, native RNE
// conversion, NaN propagation as torch's amax/clamp/cast do).
//
// The division is evaluated as one reciprocal per row plus two fused steps
// per element (quantize8), which gives the same correctly rounded quotient.
//
// Work layout.  A "unit" is one (token, K|V, head) row of D elements, handled
// by D/8 lanes that each load 8 consecutive elements (16 bytes for bf16/fp16),
// reduce |x| max across the unit, and write 8 FP8 bytes.
// * Token path (a token's heads fill whole waves, e.g. 8 heads x 128): one
//   wave per token issues all of the token's K and V loads at once and
//   writes through buffer resources that drop the stores of skipped slots.
// * Vector path (other power-of-two D): one thread group per unit.
// * Scalar path: anything else (any D, alignment or cache dtype).
#include "common.h"

#include <type_traits>

namespace prism {
namespace {

constexpr float kFp8Max = 448.0f;
constexpr float kScaleFloor = 1.0e-6f;  // the Python float 1e-6 rounded to fp32

template <int IN_DTYPE>
struct InVec8;  // 8 input elements -> 8 floats

template <>
struct InVec8<PRISM_DTYPE_BF16> {
  __device__ static void load(const void* p, float (&x)[8]) {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};

template <>
struct InVec8<PRISM_DTYPE_F16> {
  __device__ static void load(const void* p, float (&x)[8]) {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = f16_bits_to_f32(w[i] & 0xFFFFu);
      x[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
};

template <>
struct InVec8<PRISM_DTYPE_F32> {
  __device__ static void load(const void* p, float (&x)[8]) {
    const floatx4* f = reinterpret_cast<const floatx4*>(p);
    floatx4 a = f[0], b = f[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  }
};

__device__ __forceinline__ float load_scalar(const void* base, int dtype, int64_t idx) {
  if (dtype == PRISM_DTYPE_F32) return static_cast<const float*>(base)[idx];
  uint32_t bits = static_cast<const uint16_t*>(base)[idx];
  return dtype == PRISM_DTYPE_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

// Four finite values of magnitude at most 448 (1 + 2^-22) -> E4M3FN bytes
// (the native RNE conversion, which saturates: values above 448 and below
// 464 give 448 either way; fp8_encode4's NaN and overflow handling cannot
// apply).
__device__ __forceinline__ uint32_t fp8_cvt4_in_range(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// Eight elements of one (token, head) row -> E4M3FN bytes of
// clamp(x / s, -448, 448), where x / s is the correctly rounded fp32
// quotient, as IEEE division gives it.
//
// One division per row gives y = RN(1 / s).  Per element, q0 = RN(x * y) is
// within one ulp of x / s, so the residual e' = q0 * s - x is exact in fp32
// and one fused step q = RN(q0 - e' * y) is the correctly rounded quotient
// (Markstein's theorem on division by a correctly rounded reciprocal).  The
// quotients here are at most 448 (1 + 2^-22) in magnitude and s >= 1e-6, so
// nothing overflows; a quotient below 2^-126 may lose the theorem's
// guarantee but keeps its sign and is far below 2^-10, so its fp8 byte (a
// signed zero) is unaffected.  Signs of zeros: x = -0 gives q0 = -0,
// e' = -0 * s + 0 = +0 and q = -0 - (+0 * y) = -0; x = +0 gives +0 (with the
// residual of the other sign, x - q0 * s, the sum of opposite zeros would
// round -0 up to +0).  No clamp: s is amax / 448 rounded (or the 1e-6 floor
// above it), so |x / s| <= 448 (1 + 2^-22), which the native conversion
// rounds to 448 like the clamped value.  Rows whose scale is infinite or
// NaN (an infinite or NaN element) take the division itself.
__device__ __forceinline__ u32x2 quantize8(const float (&x)[8], float s) {
  float q[8];
  if (s < 0x1p125f) {
    const float y = 1.0f / s;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float q0 = x[i] * y;
      const float en = __builtin_fmaf(q0, s, -x[i]);
      q[i] = __builtin_fmaf(-en, y, q0);
    }
    u32x2 out;
    out[0] = fp8_cvt4_in_range(q[0], q[1], q[2], q[3]);
    out[1] = fp8_cvt4_in_range(q[4], q[5], q[6], q[7]);
    return out;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = nan_min(nan_max(x[i] / s, -kFp8Max), kFp8Max);
  u32x2 out;
  out[0] = fp8_encode4(q[0], q[1], q[2], q[3]);
  out[1] = fp8_encode4(q[4], q[5], q[6], q[7]);
  return out;
}

// Vector path: LANES = D / 8 lanes per unit, power of two <= 64.
template <int IN_DTYPE, int LANES, bool SCALED>
__global__ void __launch_bounds__(256)
kv_store_vec_kernel(const char* __restrict__ key, const char* __restrict__ value,
                    int64_t key_tok_stride_bytes, int64_t value_tok_stride_bytes,
                    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
                    float* __restrict__ k_scale, float* __restrict__ v_scale,
                    const int32_t* __restrict__ slot_mapping, int64_t num_units, int num_heads,
                    int64_t num_slots) {
  constexpr int IN_BYTES = (IN_DTYPE == PRISM_DTYPE_F32) ? 4 : 2;
  constexpr int D = LANES * 8;
  const int64_t unit = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / LANES;
  const int sub = threadIdx.x % LANES;
  if (unit >= num_units) return;  // whole units leave together
  const int two_h = 2 * num_heads;
  const int64_t token = unit / two_h;
  const int rem = static_cast<int>(unit - token * two_h);
  const int which = rem >= num_heads;  // 0 = K, 1 = V
  const int head = rem - which * num_heads;
  const int32_t slot = slot_mapping[token];
  if (slot < 0 || slot >= num_slots) return;

  const char* src = which ? value : key;
  const int64_t tok_stride = which ? value_tok_stride_bytes : key_tok_stride_bytes;
  const char* row = src + token * tok_stride + static_cast<int64_t>(head) * D * IN_BYTES;
  float x[8];
  InVec8<IN_DTYPE>::load(row + sub * 8 * IN_BYTES, x);

  uint8_t* cache = which ? v_cache : k_cache;
  uint8_t* dst = cache + (static_cast<int64_t>(slot) * num_heads + head) * D + sub * 8;
  u32x2 packed;
  if constexpr (SCALED) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = nan_max(amax, fabsf(x[i]));
#pragma unroll
    for (int off = 1; off < LANES; off <<= 1) amax = nan_max(amax, __shfl_xor(amax, off, LANES));
    float s = amax / kFp8Max;
    s = (s < kScaleFloor) ? kScaleFloor : s;  // clamp(min=) keeping NaN
    packed = quantize8(x, s);
    if (sub == 0) {
      float* scales = which ? v_scale : k_scale;
      scales[static_cast<int64_t>(slot) * num_heads + head] = s;
    }
  } else {
    packed[0] = fp8_encode4(x[0], x[1], x[2], x[3]);
    packed[1] = fp8_encode4(x[4], x[5], x[6], x[7]);
  }
  *reinterpret_cast<u32x2*>(dst) = packed;
}

// Max over each aligned group of LANES lanes (LANES <= 16 by DPP row
// operations inside a 16-lane row; wider groups finish with shuffles).
// NaN-propagating like nan_max.
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  if constexpr (LANES >= 2) v = nan_max(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  if constexpr (LANES >= 4) v = nan_max(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  if constexpr (LANES >= 8) v = nan_max(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  if constexpr (LANES >= 16) v = nan_max(v, dpp(v, std::integral_constant<int, 0x140>{})); // row_mirror
#pragma unroll
  for (int off = 16; off < LANES; off <<= 1) v = nan_max(v, __shfl_xor(v, off, LANES));
  return v;
}

// A raw buffer resource over [base, base + bytes); accesses at or past
// `bytes` are dropped by the hardware (stores) or read as zero (loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(bytes), 0x00020000);
}

// Cache-policy operand of the token path's buffer stores: non-temporal.  The
// cache rows are written once here and read back by a later decode, so
// they need not occupy the caches on the way (the input rows are read with
// non-temporal loads for the same reason).
constexpr int kNtPolicy = 2;

// Token path: one wave per token, no branches on the slot.  Every lane
// issues all of its 2 * PASSES 16-byte input loads (K passes, then V passes)
// together with the slot load, so a wave has the token's whole K and V rows
// in flight at once.  The slot selects the destination rows through buffer
// resources whose extent is zero when the slot is -1 or out of range, so
// those stores are dropped by the hardware.  Pass p of a tensor covers heads
// [p * 64 / LANES, (p + 1) * 64 / LANES): consecutive lanes read consecutive
// 16-byte chunks of the token row and write consecutive 8-byte chunks of the
// slot row.  Quantisation is quantize8, as on the vector path.
template <int IN_DTYPE, int LANES, int PASSES, bool SCALED>
__global__ void __launch_bounds__(256)
kv_store_token_kernel(const char* __restrict__ key, const char* __restrict__ value,
                      int64_t key_tok_stride_bytes, int64_t value_tok_stride_bytes,
                      uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
                      float* __restrict__ k_scale, float* __restrict__ v_scale,
                      const int32_t* __restrict__ slot_mapping, int64_t num_tokens, int64_t num_slots) {
  constexpr int IN_BYTES = (IN_DTYPE == PRISM_DTYPE_F32) ? 4 : 2;
  constexpr int D = LANES * 8;
  constexpr int HEADS_PER_PASS = 64 / LANES;
  constexpr int H = HEADS_PER_PASS * PASSES;
  constexpr uint32_t kRowBytes = H * D;          // one token's payload row
  constexpr uint32_t kScaleBytes = H * 4;         // one token's scale row
  const int64_t token = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
  if (token >= num_tokens) return;  // wave-uniform
  const int lane = threadIdx.x % 64;
  const int sub = lane % LANES;

  using Raw = typename std::conditional<IN_BYTES == 4, u32x4[2], u32x4[1]>::type;
  Raw raw[2][PASSES];
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const char* row = (which ? value + token * value_tok_stride_bytes : key + token * key_tok_stride_bytes) +
                      static_cast<int64_t>(lane) * 8 * IN_BYTES;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const u32x4* src = reinterpret_cast<const u32x4*>(row + p * 64 * 8 * IN_BYTES);
#pragma unroll
      for (int c = 0; c < IN_BYTES / 2; ++c) raw[which][p][c] = __builtin_nontemporal_load(src + c);
    }
  }
  const int32_t slot = __builtin_amdgcn_readfirstlane(slot_mapping[token]);
  const bool valid = slot >= 0 && slot < num_slots;
  const int64_t row_slot = valid ? slot : 0;

#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const __amdgpu_buffer_rsrc_t out_row =
        buffer_over((which ? v_cache : k_cache) + row_slot * kRowBytes, valid ? kRowBytes : 0u);
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      float x[8];
      InVec8<IN_DTYPE>::load(&raw[which][p][0], x);
      const int head = p * HEADS_PER_PASS + lane / LANES;
      u32x2 packed;
      if constexpr (SCALED) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = nan_max(amax, fabsf(x[i]));
        amax = group_max<LANES>(amax);
        float s = amax / kFp8Max;
        s = (s < kScaleFloor) ? kScaleFloor : s;  // clamp(min=) keeping NaN
        packed = quantize8(x, s);
        if (sub == 0) {
          const __amdgpu_buffer_rsrc_t scale_row =
              buffer_over((which ? v_scale : k_scale) + row_slot * H, valid ? kScaleBytes : 0u);
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s), scale_row, head * 4, 0, kNtPolicy);
        }
      } else {
        packed[0] = fp8_encode4(x[0], x[1], x[2], x[3]);
        packed[1] = fp8_encode4(x[4], x[5], x[6], x[7]);
      }
      __builtin_amdgcn_raw_buffer_store_b64(packed, out_row, (p * 64 + lane) * 8, 0, kNtPolicy);
    }
  }
}

// Scalar path: one thread per unit (any head_dim, any alignment, any cache
// dtype).  Used for shapes the vector path does not cover.
__global__ void __launch_bounds__(256)
kv_store_scalar_kernel(const void* __restrict__ key, const void* __restrict__ value, int in_dtype,
                       int64_t k_st, int64_t k_sh, int64_t k_sd, int64_t v_st, int64_t v_sh,
                       int64_t v_sd, void* __restrict__ k_cache, void* __restrict__ v_cache,
                       int cache_dtype, float* __restrict__ k_scale, float* __restrict__ v_scale,
                       const int32_t* __restrict__ slot_mapping, int64_t num_units, int num_heads,
                       int head_dim, int64_t num_slots) {
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (unit >= num_units) return;
  const int two_h = 2 * num_heads;
  const int64_t token = unit / two_h;
  const int rem = static_cast<int>(unit - token * two_h);
  const int which = rem >= num_heads;
  const int head = rem - which * num_heads;
  const int32_t slot = slot_mapping[token];
  if (slot < 0 || slot >= num_slots) return;
  const void* src = which ? value : key;
  const int64_t base = which ? (token * v_st + head * v_sh) : (token * k_st + head * k_sh);
  const int64_t sd = which ? v_sd : k_sd;
  void* cache = which ? v_cache : k_cache;
  const int64_t out_base = (static_cast<int64_t>(slot) * num_heads + head) * head_dim;
  const bool scaled = k_scale != nullptr;
  float s = 1.0f;
  if (scaled) {
    float amax = 0.0f;
    for (int d = 0; d < head_dim; ++d) amax = nan_max(amax, fabsf(load_scalar(src, in_dtype, base + d * sd)));
    s = amax / kFp8Max;
    s = (s < kScaleFloor) ? kScaleFloor : s;
    float* scales = which ? v_scale : k_scale;
    scales[static_cast<int64_t>(slot) * num_heads + head] = s;
  }
  for (int d = 0; d < head_dim; ++d) {
    float x = load_scalar(src, in_dtype, base + d * sd);
    if (cache_dtype == PRISM_DTYPE_FP8_E4M3FN) {
      if (scaled) x = nan_min(nan_max(x / s, -kFp8Max), kFp8Max);
      static_cast<uint8_t*>(cache)[out_base + d] = static_cast<uint8_t>(fp8_encode4(x, 0.f, 0.f, 0.f) & 0xFFu);
    } else if (cache_dtype == PRISM_DTYPE_F32) {
      static_cast<float*>(cache)[out_base + d] = x;
    } else if (cache_dtype == PRISM_DTYPE_BF16) {
      // Inputs of the cache's own dtype are copied bit for bit.
      uint16_t bits = (in_dtype == PRISM_DTYPE_BF16)
                          ? static_cast<const uint16_t*>(src)[base + d * sd]
                          : f32_to_bf16_bits(x);
      static_cast<uint16_t*>(cache)[out_base + d] = bits;
    } else {
      uint16_t bits = (in_dtype == PRISM_DTYPE_F16)
                          ? static_cast<const uint16_t*>(src)[base + d * sd]
                          : f32_to_f16_bits(x);
      static_cast<uint16_t*>(cache)[out_base + d] = bits;
    }
  }
}

template <int IN_DTYPE, int LANES, int PASSES>
int launch_token(const void* key, const void* value, int64_t k_tok_bytes, int64_t v_tok_bytes,
                 void* k_cache, void* v_cache, float* k_scale, float* v_scale, const int32_t* slots,
                 int64_t num_tokens, int64_t num_slots, hipStream_t stream) {
  const int64_t blocks = ceil_div(num_tokens, 4);  // four waves (tokens) per block
  if (blocks > INT32_MAX) {
    set_error("prism_kv_store: too many tokens for one launch");
    return PRISM_ERR_INVALID;
  }
  const char* k = static_cast<const char*>(key);
  const char* v = static_cast<const char*>(value);
  uint8_t* kc = static_cast<uint8_t*>(k_cache);
  uint8_t* vc = static_cast<uint8_t*>(v_cache);
  if (k_scale) {
    hipLaunchKernelGGL((kv_store_token_kernel<IN_DTYPE, LANES, PASSES, true>), dim3(blocks), dim3(256), 0, stream,
                       k, v, k_tok_bytes, v_tok_bytes, kc, vc, k_scale, v_scale, slots, num_tokens, num_slots);
  } else {
    hipLaunchKernelGGL((kv_store_token_kernel<IN_DTYPE, LANES, PASSES, false>), dim3(blocks), dim3(256), 0, stream,
                       k, v, k_tok_bytes, v_tok_bytes, kc, vc, nullptr, nullptr, slots, num_tokens, num_slots);
  }
  return check_launch("kv_store_token_kernel launch");
}

template <int IN_DTYPE, int LANES>
int launch_vec(const void* key, const void* value, int64_t k_tok_bytes, int64_t v_tok_bytes,
               void* k_cache, void* v_cache, float* k_scale, float* v_scale, const int32_t* slots,
               int64_t num_units, int num_heads, int64_t num_slots, hipStream_t stream) {
  // A token's heads fill whole waves: one wave per token.
  if constexpr (LANES >= 4) {
    if (num_heads * LANES % 64 == 0) {
      const int64_t tokens = num_units / (2 * num_heads);
      switch (num_heads * LANES / 64) {
        case 1: return launch_token<IN_DTYPE, LANES, 1>(key, value, k_tok_bytes, v_tok_bytes, k_cache, v_cache,
                                                        k_scale, v_scale, slots, tokens, num_slots, stream);
        case 2: return launch_token<IN_DTYPE, LANES, 2>(key, value, k_tok_bytes, v_tok_bytes, k_cache, v_cache,
                                                        k_scale, v_scale, slots, tokens, num_slots, stream);
        case 4: return launch_token<IN_DTYPE, LANES, 4>(key, value, k_tok_bytes, v_tok_bytes, k_cache, v_cache,
                                                        k_scale, v_scale, slots, tokens, num_slots, stream);
        default: break;
      }
    }
  }
  const int64_t threads = num_units * LANES;
  const int64_t blocks = ceil_div(threads, 256);
  if (blocks > INT32_MAX) {
    set_error("prism_kv_store: too many tokens for one launch");
    return PRISM_ERR_INVALID;
  }
  if (k_scale) {
    hipLaunchKernelGGL((kv_store_vec_kernel<IN_DTYPE, LANES, true>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const char*>(key), static_cast<const char*>(value), k_tok_bytes,
                       v_tok_bytes, static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache),
                       k_scale, v_scale, slots, num_units, num_heads, num_slots);
  } else {
    hipLaunchKernelGGL((kv_store_vec_kernel<IN_DTYPE, LANES, false>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const char*>(key), static_cast<const char*>(value), k_tok_bytes,
                       v_tok_bytes, static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache),
                       nullptr, nullptr, slots, num_units, num_heads, num_slots);
  }
  return check_launch("kv_store_vec_kernel launch");
}

template <int IN_DTYPE>
int dispatch_lanes(int lanes, const void* key, const void* value, int64_t kb, int64_t vb, void* kc,
                   void* vc, float* ks, float* vs, const int32_t* slots, int64_t units, int heads,
                   int64_t num_slots, hipStream_t stream) {
  switch (lanes) {
    case 1: return launch_vec<IN_DTYPE, 1>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    case 2: return launch_vec<IN_DTYPE, 2>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    case 4: return launch_vec<IN_DTYPE, 4>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    case 8: return launch_vec<IN_DTYPE, 8>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    case 16: return launch_vec<IN_DTYPE, 16>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    case 32: return launch_vec<IN_DTYPE, 32>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    case 64: return launch_vec<IN_DTYPE, 64>(key, value, kb, vb, kc, vc, ks, vs, slots, units, heads, num_slots, stream);
    default: return PRISM_ERR_LAYOUT;
  }
}

}  // namespace

// Loads this file's code object now rather than at its first kernel launch.
int preload_kv_store() {
  hipFuncAttributes attr;
  return check_hip(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&kv_store_scalar_kernel)), "preload_kv_store");
}

}  // namespace prism

extern "C" int prism_kv_store(const void* key, const void* value, int in_dtype,
                              const int64_t key_strides[3], const int64_t value_strides[3],
                              void* k_cache, void* v_cache, int cache_dtype, float* k_scale,
                              float* v_scale, const int32_t* slot_mapping, int64_t num_tokens,
                              int num_heads, int head_dim, int64_t num_slots, void* stream_ptr) {
  using namespace prism;
  clear_error();
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || num_slots < 0) {
    set_error("prism_kv_store: invalid geometry tokens=%lld heads=%d head_dim=%d slots=%lld",
              static_cast<long long>(num_tokens), num_heads, head_dim, static_cast<long long>(num_slots));
    return PRISM_ERR_INVALID;
  }
  if (in_dtype != PRISM_DTYPE_F32 && in_dtype != PRISM_DTYPE_BF16 && in_dtype != PRISM_DTYPE_F16) {
    set_error("prism_kv_store: unsupported input dtype code %d", in_dtype);
    return PRISM_ERR_INVALID;
  }
  if (dtype_size(cache_dtype) == 0) {
    set_error("prism_kv_store: unsupported cache dtype code %d", cache_dtype);
    return PRISM_ERR_INVALID;
  }
  if ((k_scale == nullptr) != (v_scale == nullptr)) {
    set_error("prism_kv_store: K/V scale caches must be provided together");
    return PRISM_ERR_INVALID;
  }
  if (k_scale && cache_dtype != PRISM_DTYPE_FP8_E4M3FN) {
    set_error("prism_kv_store: token-head scales require FP8 K/V payload caches");
    return PRISM_ERR_INVALID;
  }
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !key_strides || !value_strides) {
    if (num_tokens == 0) return PRISM_OK;
    set_error("prism_kv_store: null pointer argument");
    return PRISM_ERR_INVALID;
  }
  if (num_tokens == 0) return PRISM_OK;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const int64_t units = num_tokens * 2 * num_heads;
  const int in_bytes = dtype_size(in_dtype);
  const int lanes = head_dim / 8;
  const bool dense_rows = key_strides[2] == 1 && value_strides[2] == 1 && key_strides[1] == head_dim &&
                          value_strides[1] == head_dim;
  const bool pow2_lanes = head_dim % 8 == 0 && lanes >= 1 && lanes <= 64 && (lanes & (lanes - 1)) == 0;
  const int64_t kb = key_strides[0] * in_bytes;
  const int64_t vb = value_strides[0] * in_bytes;
  const bool vec_aligned = aligned(key, 16) && aligned(value, 16) && kb % 16 == 0 && vb % 16 == 0 &&
                           aligned(k_cache, 8) && aligned(v_cache, 8);
  if (cache_dtype == PRISM_DTYPE_FP8_E4M3FN && dense_rows && pow2_lanes && vec_aligned) {
    switch (in_dtype) {
      case PRISM_DTYPE_BF16:
        return dispatch_lanes<PRISM_DTYPE_BF16>(lanes, key, value, kb, vb, k_cache, v_cache, k_scale, v_scale,
                                                slot_mapping, units, num_heads, num_slots, stream);
      case PRISM_DTYPE_F16:
        return dispatch_lanes<PRISM_DTYPE_F16>(lanes, key, value, kb, vb, k_cache, v_cache, k_scale, v_scale,
                                               slot_mapping, units, num_heads, num_slots, stream);
      default:
        return dispatch_lanes<PRISM_DTYPE_F32>(lanes, key, value, kb, vb, k_cache, v_cache, k_scale, v_scale,
                                               slot_mapping, units, num_heads, num_slots, stream);
    }
  }
  const int64_t blocks = ceil_div(units, 256);
  hipLaunchKernelGGL(kv_store_scalar_kernel, dim3(blocks), dim3(256), 0, stream, key, value, in_dtype,
                     key_strides[0], key_strides[1], key_strides[2], value_strides[0], value_strides[1],
                     value_strides[2], k_cache, v_cache, cache_dtype, k_scale, v_scale, slot_mapping, units,
                     num_heads, head_dim, num_slots);
  return check_launch("kv_store_scalar_kernel launch");
}
