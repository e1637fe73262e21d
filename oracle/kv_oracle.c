/*
 * CPU oracle for the scaled-FP8 paged KV path.  TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference algorithms; it is the
 * checker that the HIP product path is compared against.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * Nothing in the product (prism-infer_amd/) links, loads or calls it.
 *
 * Functions and the reference code they restate (paths relative to the
 * Prism-Infer source tree):
 *
 *   oracle_e4m3fn_from_f32 / oracle_e4m3fn_to_f32
 *       OCP 8-bit floating point spec, E4M3 "FN" variant (no infinities, one
 *       NaN code S.1111.111, max finite 448), round-to-nearest-even.  The
 *       reference obtains this rounding from torch's Tensor.to(float8_e4m3fn)
 *       (prism_infer/ops/kv_cache_store.py:216-225).  Pinned exhaustively
 *       against torch's cast in tests/test_oracle_fp8.py.
 *
 *   oracle_store_scaled
 *       prism_infer/ops/kv_cache_store.py:170-230 (_store_kvcache_eager, scaled
 *       branch :205-227) with the constants of
 *       prism_infer/engine/kv_quantization.py:9-12.  Per (token, kv head):
 *         scale = clamp(amax(|x|) / 448, min=1e-6)     (fp32, IEEE divide)
 *         q     = clamp(x / scale, -448, 448) -> e4m3fn (RNE)
 *       slot < 0 is skipped; untouched slots keep their contents.  Slots
 *       >= num_slots are skipped too (the reference would write out of
 *       bounds; the HIP path and this oracle share the skip contract).
 *
 *   oracle_store_unit
 *       prism_infer/ops/kv_cache_store.py:228-230 (dense branch: plain cast of
 *       the input into an FP8 cache, no scale).
 *
 *   oracle_compact_slots
 *       prism_infer/ops/kv_compaction.py:93-112: cache[:, :, dst[i]] receives
 *       the bytes of cache[:, :, src[i]] as they were BEFORE the call
 *       (index_select(...).clone() then index_copy_).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fp32 -> E4M3FN, round to nearest even.  Values whose rounded magnitude
 * exceeds 448 (|x| > 464, and inf) become NaN, as do NaNs; the sign bit is
 * kept in all cases (this is also what torch's cast produces). */
uint8_t oracle_e4m3fn_from_f32(float f) {
    uint32_t u = f32_bits(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return sign | 0x7Fu; /* inf / NaN -> NaN */
    int exp_field = (int)(a >> 23);
    if (exp_field == 0) return sign; /* fp32 subnormal: |x| < 2^-126 -> 0 */
    int e = exp_field - 127;          /* unbiased exponent */
    uint32_t mant24 = (a & 0x7FFFFFu) | 0x800000u; /* 1.m as a 24-bit integer */
    if (e >= -6) {
        /* normal range of E4M3: keep 1 implicit + 3 explicit mantissa bits */
        uint32_t keep = mant24 >> 20;          /* 8..15 */
        uint32_t rem = mant24 & 0xFFFFFu;
        uint32_t half = 0x80000u;
        if (rem > half || (rem == half && (keep & 1u))) keep += 1;
        int biased = e + 7;
        if (keep == 16) { keep = 8; biased += 1; }
        if (biased > 15 || (biased == 15 && (keep & 7u) == 7u)) return sign | 0x7Fu;
        return sign | (uint8_t)((biased << 3) | (keep & 7u));
    }
    /* subnormal range of E4M3: integer multiples of 2^-9 */
    int shift = 14 - e; /* value / 2^-9 = mant24 >> shift (with rounding) */
    if (shift > 24) return sign; /* |x| < 2^-10: rounds to zero */
    uint32_t keep = mant24 >> shift;
    uint32_t rem = mant24 & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (keep & 1u))) keep += 1;
    /* keep == 8 is exactly the smallest normal (exponent field 1, mantissa 0),
     * which the same bit pattern encodes. */
    return sign | (uint8_t)keep;
}

float oracle_e4m3fn_to_f32(uint8_t b) {
    int sign = (b >> 7) & 1;
    int exp_field = (b >> 3) & 0xF;
    int mant = b & 7;
    float v;
    if (exp_field == 15 && mant == 7) {
        v = bits_f32(0x7FC00000u);
    } else if (exp_field == 0) {
        v = ldexpf((float)mant, -9);
    } else {
        v = ldexpf((float)(8 + mant), exp_field - 7 - 3);
    }
    return sign ? -v : v;
}

/* Encode n floats (used by the exhaustive check against torch). */
void oracle_e4m3fn_encode_array(const float* in, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3fn_from_f32(in[i]);
}

/* Encode every fp32 bit pattern in [lo, hi) (as uint32) into out. */
void oracle_e4m3fn_encode_bit_range(uint32_t lo, uint32_t hi, uint8_t* out) {
    for (uint64_t u = lo; u < hi; ++u) out[u - lo] = oracle_e4m3fn_from_f32(bits_f32((uint32_t)u));
}

enum { ORACLE_IN_F32 = 0, ORACLE_IN_BF16 = 1, ORACLE_IN_F16 = 2 };

static float half_to_f32(uint16_t h) {
    int sign = (h >> 15) & 1;
    int e = (h >> 10) & 0x1F;
    int m = h & 0x3FF;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? bits_f32(0x7FC00000u) : INFINITY;
    else v = ldexpf((float)(1024 + m), e - 25);
    return sign ? -v : v;
}

static float load_elem(const void* base, int dtype, int64_t index) {
    if (dtype == ORACLE_IN_F32) return ((const float*)base)[index];
    if (dtype == ORACLE_IN_BF16) return bits_f32((uint32_t)((const uint16_t*)base)[index] << 16);
    return half_to_f32(((const uint16_t*)base)[index]);
}

/* torch.amax propagates NaN; torch.clamp(min=...) propagates NaN too. */
static float amax_abs(const void* x, int dtype, int64_t base, int64_t stride_d, int d) {
    float m = 0.0f;
    int nan = 0;
    for (int i = 0; i < d; ++i) {
        float v = fabsf(load_elem(x, dtype, base + (int64_t)i * stride_d));
        if (v != v) nan = 1;
        else if (v > m) m = v;
    }
    return nan ? bits_f32(0x7FC00000u) : m;
}

static float clamp_nan(float x, float lo, float hi) {
    if (x != x) return x;
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
}

/*
 * Scaled store.  key/value: [T, H, D] with element strides; caches are flat
 * [num_slots, H, D] uint8 (E4M3FN bytes); scale caches flat [num_slots, H] fp32.
 */
void oracle_store_scaled(const void* key, const void* value, int in_dtype,
                         const int64_t* k_strides, const int64_t* v_strides,
                         uint8_t* k_cache, uint8_t* v_cache, float* k_scale, float* v_scale,
                         const int32_t* slot_mapping, int64_t num_tokens, int num_heads, int head_dim,
                         int64_t num_slots) {
    const float qmax = 448.0f;
    const float floor_ = (float)1.0e-6; /* the Python float 1e-6 rounded to fp32 */
    for (int64_t t = 0; t < num_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= num_slots) continue;
        for (int h = 0; h < num_heads; ++h) {
            for (int which = 0; which < 2; ++which) {
                const void* src = which ? value : key;
                const int64_t* st = which ? v_strides : k_strides;
                uint8_t* cache = which ? v_cache : k_cache;
                float* scales = which ? v_scale : k_scale;
                int64_t base = t * st[0] + (int64_t)h * st[1];
                float amax = amax_abs(src, in_dtype, base, st[2], head_dim);
                float s = amax / qmax;
                if (s == s && s < floor_) s = floor_;
                uint8_t* dst = cache + (slot * num_heads + h) * (int64_t)head_dim;
                for (int d = 0; d < head_dim; ++d) {
                    float x = load_elem(src, in_dtype, base + (int64_t)d * st[2]);
                    float q = clamp_nan(x / s, -qmax, qmax);
                    dst[d] = oracle_e4m3fn_from_f32(q);
                }
                scales[slot * num_heads + h] = s;
            }
        }
    }
}

/* Unit-scale store into an FP8 cache: a plain RNE cast of every element. */
void oracle_store_unit(const void* key, const void* value, int in_dtype,
                       const int64_t* k_strides, const int64_t* v_strides,
                       uint8_t* k_cache, uint8_t* v_cache,
                       const int32_t* slot_mapping, int64_t num_tokens, int num_heads, int head_dim,
                       int64_t num_slots) {
    for (int64_t t = 0; t < num_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= num_slots) continue;
        for (int h = 0; h < num_heads; ++h) {
            for (int d = 0; d < head_dim; ++d) {
                int64_t kb = t * k_strides[0] + (int64_t)h * k_strides[1] + (int64_t)d * k_strides[2];
                int64_t vb = t * v_strides[0] + (int64_t)h * v_strides[1] + (int64_t)d * v_strides[2];
                int64_t o = (slot * num_heads + h) * (int64_t)head_dim + d;
                k_cache[o] = oracle_e4m3fn_from_f32(load_elem(key, in_dtype, kb));
                v_cache[o] = oracle_e4m3fn_from_f32(load_elem(value, in_dtype, vb));
            }
        }
    }
}

/*
 * Compaction: cache is [rows, num_slots, vec_bytes] contiguous.  All reads
 * happen before any write (gather into a temporary, then scatter).
 * Returns 0 on success, -1 on allocation failure, -2 on an out-of-range slot.
 */
int oracle_compact_slots(uint8_t* cache, int64_t rows, int64_t num_slots, int64_t vec_bytes,
                         const int64_t* src, const int64_t* dst, int64_t retained) {
    for (int64_t i = 0; i < retained; ++i) {
        if (src[i] < 0 || src[i] >= num_slots || dst[i] < 0 || dst[i] >= num_slots) return -2;
    }
    uint8_t* tmp = (uint8_t*)malloc((size_t)(rows * retained * vec_bytes));
    if (!tmp) return -1;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < retained; ++i)
            memcpy(tmp + (r * retained + i) * vec_bytes, cache + (r * num_slots + src[i]) * vec_bytes,
                   (size_t)vec_bytes);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < retained; ++i)
            memcpy(cache + (r * num_slots + dst[i]) * vec_bytes, tmp + (r * retained + i) * vec_bytes,
                   (size_t)vec_bytes);
    free(tmp);
    return 0;
}
