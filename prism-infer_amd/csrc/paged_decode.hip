// Paged decode attention over scaled-FP8 (or unit-scale FP8 / 16-bit / fp32)
// KV pages, one query token per sequence, grouped-query attention.
//
// Semantics follow prism_infer/ops/paged_decode.py:83-180: query head hq reads
// kv head hq / G; a token t of sequence b is attended iff
// t < min(context_lens[b], *max_context_len, W * P) and its block id is valid;
// K and V are dequantised with their per-token, per-head fp32 scales; online
// softmax in fp32; a sequence with no attended token outputs zeros.
//
// Split-K path (FP8 cache, head_dim 128, <= 8 kv heads, G <= 16):
//   grid (batch, kv heads, chunks); one workgroup per (sequence, kv head,
//   chunk of SPLIT tokens), its eight waves on neighbouring 32-token tiles of
//   that head.  Per tile and wave:
//     QK: 2 x 4 MFMA f32_16x16x32_bf16, A = K rows (fp8 -> bf16 exact),
//         B = Q^T (G valid columns of 16).  Lane (g, c) receives the scores of
//         q head c for tokens 4g+i and 16+4g+i.
//     softmax: k_scale * sm_scale * log2(e) applied to the fp32 scores, exp2,
//         max/sum across the 4 lane groups with lane shuffles.
//     PV: 2 x 8 MFMA f32_16x16x32_bf16, A = P * v_scale as a bf16 hi/lo pair
//         (fp32-like accuracy), whose k slots are
//         exactly the 8 tokens the lane already holds scores for, B = V with
//         output column c of N-tile j mapped to dim 8c + j, so each lane loads
//         8 contiguous bytes per token and the byte transpose is one v_perm
//         plus two native fp8 -> bf16 conversions per 4 values.
//   The waves merge through LDS.  A sequence with one chunk writes its output
//   directly; otherwise each chunk writes an (m, l, acc) partial and the last
//   chunk of (sequence, kv head) to finish merges them in the same launch.
// Generic path (any other supported shape): one wave per (sequence, q head),
//   lane-per-token scores, lane-per-dim accumulation, no split-K.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "fp8_mfma.h"

namespace prism {
namespace {

// Measurement aids of the streaming kernel (bit 1: skip compute, 2: skip
// loads, 4: plan phase stamps, 8: per-workgroup start/end times, 16: default
// cache policy for private pages, 32: per-workgroup stamps of the kernel's
// phases and merge counts, 64: per-wave cycles spent waiting, issuing,
// computing and flushing, 128: trust the plan slot without comparing its
// key) exist only in a build that defines PRISM_DECODE_MEASURE (read from
// PRISM_STREAM_DEBUG there).  Bits 32 and 64 write into a stamp area after
// the plan slots.  The product library compiles them out: it always checks
// the plan and loads and computes every tile.
#ifdef PRISM_DECODE_MEASURE
#define PRISM_DBG(a) ((a).debug)
#else
#define PRISM_DBG(a) 0
#endif

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 32;          // tokens per tile
constexpr int kHeadDim = 128;      // fast-path head_dim

struct DecodeArgs {
  const void* q;
  int64_t q_sb, q_sh, q_sd;
  const uint8_t* k;
  const uint8_t* v;
  int64_t k_sblk, k_stok, k_sh;  // bytes
  int64_t v_sblk, v_stok, v_sh;  // bytes
  const float* ks;
  const float* vs;
  int64_t ks_sblk, ks_stok, ks_sh;  // elements
  int64_t vs_sblk, vs_stok, vs_sh;
  const int32_t* bt;
  int64_t bt_sb, bt_sn;
  const int32_t* ctx;
  const int32_t* max_ctx;
  void* out;
  int64_t o_sb, o_sh, o_sd;
  float* part_acc;  // [B][S][Hq][D]
  float* part_ml;   // [B][S][Hq][2]
  int* plan_region;  // streaming path: plan word, two plan slots, measurement stamps (workspace start)
  int64_t vrow0;    // streaming path: first partial row of the virtual sequences
  int share;        // streaming path: analyse prefix sharing
  int stream_nwg;   // streaming path: grid size
  int batch, num_heads, num_kv_heads, groups, page_size, width, head_dim;
  int64_t num_blocks;
  int q_vec;     // q rows are 16-byte aligned with unit dim stride
  int split;     // split-K path: tokens per chunk (multiple of 8 tiles)
  int max_splits;  // split-K path: chunks per (sequence, kv head)
  unsigned long long* split_cnt;  // split-K path: arrival counters, [batch][kv heads]
  unsigned int epoch;             // this call's tag (nonzero): split-K counters, streaming plan word
  float scale_log2;  // sm_scale * log2(e)
  int cache_dtype;
  int debug;         // measurement aid for the stream kernel (0 in normal use)
  // streaming path: tokens per 1 KB LDS row (8 / num_kv_heads) and per tile
  // (16 rows); the streaming and merge kernels take the former as a template
  // parameter, the plan code reads both
  int s_tpr, s_ttok;
  int plan_spin;  // streaming path: polls a workgroup waits for a plan build before it gives up
  int vcols;      // streaming path: query columns of a virtual sequence (16, or 32 = two MFMA column blocks)
};

// Read-only int32 metadata (block tables, context lengths) through the
// constant address space: uniform indices then become scalar loads, which
// neither wait on nor delay the vector-memory counter.
__device__ __forceinline__ int32_t ld_meta(const int32_t* p) {
  return *reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ int effective_len(const DecodeArgs& a, int b) {
  int ctx = ld_meta(a.ctx + b);
  int mx = ld_meta(a.max_ctx);
  int64_t cap = static_cast<int64_t>(a.width) * a.page_size;
  int64_t n = ctx < mx ? ctx : mx;
  if (n > cap) n = cap;
  return n > 0 ? static_cast<int>(n) : 0;
}

template <int QDT>
__device__ __forceinline__ float load_q(const void* q, int64_t idx) {
  if constexpr (QDT == PRISM_DTYPE_F32) return static_cast<const float*>(q)[idx];
  else if constexpr (QDT == PRISM_DTYPE_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(q)[idx]);
  else return f16_bits_to_f32(static_cast<const uint16_t*>(q)[idx]);
}

template <int QDT>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
  if constexpr (QDT == PRISM_DTYPE_F32) static_cast<float*>(out)[idx] = v;
  else if constexpr (QDT == PRISM_DTYPE_BF16) static_cast<uint16_t*>(out)[idx] = f32_to_bf16_bits(v);
  else static_cast<uint16_t*>(out)[idx] = f32_to_f16_bits(v);
}


// Eight consecutive dims of one output row, o[j] * inv at idx + j * o_sd.
// 16-bit outputs with unit dim stride and a 16-byte aligned address take one
// 16-byte store (the same conversion per element) instead of eight 2-byte
// stores with their 64-bit address arithmetic; anything else is stored
// element by element.
template <int QDT, typename Args>
__device__ __forceinline__ void store_out8(const Args& a, int64_t idx, const float (&o)[8], float inv) {
  if constexpr (QDT != PRISM_DTYPE_F32) {
    uint16_t* p = static_cast<uint16_t*>(a.out) + idx;
    if (a.o_sd == 1 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
      u32x4 w;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = o[2 * j] * inv, hi = o[2 * j + 1] * inv;
        const uint32_t blo = QDT == PRISM_DTYPE_BF16 ? f32_to_bf16_bits(lo) : f32_to_f16_bits(lo);
        const uint32_t bhi = QDT == PRISM_DTYPE_BF16 ? f32_to_bf16_bits(hi) : f32_to_f16_bits(hi);
        w[j] = blo | (bhi << 16);
      }
      *reinterpret_cast<u32x4*>(p) = w;
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) store_out<QDT>(a.out, idx + j * a.o_sd, o[j] * inv);
}

struct TileRegs {
  u32x4 k[2][2];   // [half][part]: 32 bytes of K row (c + 16 * half), dims 32g..32g+31
  u32x2 v[8];      // V rows of tokens {4g+i, 16+4g+i}, dims 8c..8c+7
  float ksc[8];    // k scale of the same 8 tokens
  float vsc[8];    // v scale
  uint32_t kvalid; // bit e: token of slot e is attended
};

// Token order of the 8 per-lane "slots": e < 4 -> 4g + e; e >= 4 -> 16 + 4g + (e - 4).
__device__ __forceinline__ int slot_token(int g, int e) { return (e < 4) ? (4 * g + e) : (16 + 4 * g + e - 4); }

template <bool SCALED, bool PAGE_ALIGNED>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, int b, int h, int g, int c, int t0, int t_end,
                                          TileRegs& r, int32_t blk_pre = -1, bool use_pre = false) {
  const int32_t* bt_row = a.bt + static_cast<int64_t>(b) * a.bt_sb;
  r.kvalid = 0;
  if constexpr (PAGE_ALIGNED) {
    // The whole tile lies in one page.  Branch-free: an absent block reads
    // page 0 (always allocated on this path) and the tile is masked, so the
    // compiler can keep this prefetch asynchronous.
    const int page = t0 / a.page_size;
    const int off0 = t0 - page * a.page_size;
    const int32_t blk_raw = use_pre ? blk_pre : bt_row[page * a.bt_sn];
    const bool blk_ok = blk_raw >= 0 && blk_raw < a.num_blocks;
    const int64_t blk = blk_ok ? blk_raw : 0;
    const uint8_t* kbase = a.k + blk * a.k_sblk + static_cast<int64_t>(off0) * a.k_stok + h * a.k_sh;
    const uint8_t* vbase = a.v + blk * a.v_sblk + static_cast<int64_t>(off0) * a.v_stok + h * a.v_sh;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const u32x4* p = reinterpret_cast<const u32x4*>(kbase + (c + 16 * hh) * a.k_stok + 32 * g);
      r.k[hh][0] = p[0];
      r.k[hh][1] = p[1];
    }
    const float* ksb = a.ks + blk * a.ks_sblk + static_cast<int64_t>(off0) * a.ks_stok + h * a.ks_sh;
    const float* vsb = a.vs + blk * a.vs_sblk + static_cast<int64_t>(off0) * a.vs_stok + h * a.vs_sh;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tk = slot_token(g, e);
      r.v[e] = *reinterpret_cast<const u32x2*>(vbase + tk * a.v_stok + 8 * c);
      if (SCALED) {
        r.ksc[e] = ksb[tk * a.ks_stok];
        r.vsc[e] = vsb[tk * a.vs_stok];
      } else {
        r.ksc[e] = r.vsc[e] = 1.f;
      }
      r.kvalid |= (blk_ok && t0 + tk < t_end) ? (1u << e) : 0u;
    }
  } else {
    // Tiles may straddle pages: resolve every row separately.
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int tok = t0 + c + 16 * hh;
      r.k[hh][0] = r.k[hh][1] = u32x4{0, 0, 0, 0};
      if (tok < t_end) {
        const int page = tok / a.page_size;
        const int32_t blk = bt_row[page * a.bt_sn];
        if (blk >= 0 && blk < a.num_blocks) {
          const u32x4* p = reinterpret_cast<const u32x4*>(
              a.k + blk * a.k_sblk + static_cast<int64_t>(tok - page * a.page_size) * a.k_stok + h * a.k_sh + 32 * g);
          r.k[hh][0] = p[0];
          r.k[hh][1] = p[1];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = t0 + slot_token(g, e);
      r.v[e] = u32x2{0, 0};
      r.ksc[e] = r.vsc[e] = 0.f;
      if (tok < t_end) {
        const int page = tok / a.page_size;
        const int off = tok - page * a.page_size;
        const int32_t blk = bt_row[page * a.bt_sn];
        if (blk >= 0 && blk < a.num_blocks) {
          r.v[e] = *reinterpret_cast<const u32x2*>(a.v + blk * a.v_sblk + static_cast<int64_t>(off) * a.v_stok +
                                                   h * a.v_sh + 8 * c);
          if (SCALED) {
            r.ksc[e] = a.ks[blk * a.ks_sblk + static_cast<int64_t>(off) * a.ks_stok + h * a.ks_sh];
            r.vsc[e] = a.vs[blk * a.vs_sblk + static_cast<int64_t>(off) * a.vs_stok + h * a.vs_sh];
          } else {
            r.ksc[e] = r.vsc[e] = 1.f;
          }
          r.kvalid |= 1u << e;
        }
      }
    }
  }
}

// The same tile of a 16-bit (bf16 or f16) cache: lane (g, c) holds 64 bytes of
// K rows c and c + 16 (dims 32g .. 32g + 31) and 16 bytes of the V rows of its
// 8 slot tokens (dims 8c .. 8c + 7).  No scales (16-bit caches are unscaled).
struct TileRegs16 {
  u32x4 k[2][4];   // [half][dims 8q .. 8q + 7 of the lane's 32]
  u32x4 v[8];      // V rows of tokens {4g+i, 16+4g+i}, dims 8c..8c+7
  uint32_t kvalid; // bit e: token of slot e is attended
};

template <bool PAGE_ALIGNED>
__device__ __forceinline__ void load_tile16(const DecodeArgs& a, int b, int h, int g, int c, int t0, int t_end,
                                            TileRegs16& r, int32_t blk_pre = -1, bool use_pre = false) {
  const int32_t* bt_row = a.bt + static_cast<int64_t>(b) * a.bt_sb;
  r.kvalid = 0;
  if constexpr (PAGE_ALIGNED) {
    // The whole tile lies in one page; an absent block reads page 0 and is masked.
    const int page = t0 / a.page_size;
    const int off0 = t0 - page * a.page_size;
    const int32_t blk_raw = use_pre ? blk_pre : bt_row[page * a.bt_sn];
    const bool blk_ok = blk_raw >= 0 && blk_raw < a.num_blocks;
    const int64_t blk = blk_ok ? blk_raw : 0;
    const uint8_t* kbase = a.k + blk * a.k_sblk + static_cast<int64_t>(off0) * a.k_stok + h * a.k_sh;
    const uint8_t* vbase = a.v + blk * a.v_sblk + static_cast<int64_t>(off0) * a.v_stok + h * a.v_sh;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const u32x4* p = reinterpret_cast<const u32x4*>(kbase + (c + 16 * hh) * a.k_stok + 64 * g);
#pragma unroll
      for (int q = 0; q < 4; ++q) r.k[hh][q] = p[q];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tk = slot_token(g, e);
      r.v[e] = *reinterpret_cast<const u32x4*>(vbase + tk * a.v_stok + 16 * c);
      r.kvalid |= (blk_ok && t0 + tk < t_end) ? (1u << e) : 0u;
    }
  } else {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int tok = t0 + c + 16 * hh;
#pragma unroll
      for (int q = 0; q < 4; ++q) r.k[hh][q] = u32x4{0, 0, 0, 0};
      if (tok < t_end) {
        const int page = tok / a.page_size;
        const int32_t blk = bt_row[page * a.bt_sn];
        if (blk >= 0 && blk < a.num_blocks) {
          const u32x4* p = reinterpret_cast<const u32x4*>(
              a.k + blk * a.k_sblk + static_cast<int64_t>(tok - page * a.page_size) * a.k_stok + h * a.k_sh + 64 * g);
#pragma unroll
          for (int q = 0; q < 4; ++q) r.k[hh][q] = p[q];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = t0 + slot_token(g, e);
      r.v[e] = u32x4{0, 0, 0, 0};
      if (tok < t_end) {
        const int page = tok / a.page_size;
        const int off = tok - page * a.page_size;
        const int32_t blk = bt_row[page * a.bt_sn];
        if (blk >= 0 && blk < a.num_blocks) {
          r.v[e] = *reinterpret_cast<const u32x4*>(a.v + blk * a.v_sblk + static_cast<int64_t>(off) * a.v_stok +
                                                   h * a.v_sh + 16 * c);
          r.kvalid |= 1u << e;
        }
      }
    }
  }
}

// Query operand type per q dtype: bf16 MFMA for bf16 (and the hi/lo split of
// fp32), f16 MFMA for fp16.
template <int QDT>
struct QOperand {
  bf16x8 hi[4];
  bf16x8 lo[4];  // used for fp32 queries only
};

template <>
struct QOperand<PRISM_DTYPE_F16> {
  f16x8 hi[4];
};

// Partials cross workgroups (and XCDs, whose L2 caches are not coherent with
// each other) inside one launch.  They are written with device-scope stores
// (sc1: written through to the device-coherent level) and read back with
// device-scope loads (sc1 buffer loads), so neither side needs a cache-wide
// writeback or invalidate.  A partial is counted only after its writer's
// stores have completed (s_waitcnt vmcnt(0)), and the merging workgroup
// loads the partials only after the counter told it every one is in.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kCoherentLoad = 16;  // buffer-load cache policy: sc1 (device scope)

__device__ __forceinline__ floatx4 load_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(byte_off), 0, kCoherentLoad);
  return floatx4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
}

__device__ __forceinline__ float2 load_coherent2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(byte_off), 0, kCoherentLoad);
  return float2{__uint_as_float(v[0]), __uint_as_float(v[1])};
}

constexpr int kSplitWaves = 8;       // waves per split-K workgroup (tile lanes of one kv head)
constexpr int kSplitMaxChunks = 64;  // chunks per (sequence, kv head) at most

// Chunk counters of the split-K path, one 64-bit word per (sequence, kv
// head): (epoch << 32) | arrivals.  Every call carries its own nonzero epoch,
// so a word holding anything of another call (or bytes of another use of the
// workspace) counts as zero arrivals and the workspace needs no clearing.
// Every chunk of the launch claims the word for its call: an exchange
// 0 -> (epoch, 0) issued first thing, whose answer only a live chunk reads,
// when it arrives (the round trip hides behind the chunk's tiles); if the
// word held neither 0 nor this call's tag, the arriving chunk repeats the
// exchange with the value seen until the word carries the tag.  The arrival
// is then a single add.  An exchange succeeds only on 0 or a foreign value,
// so no claim disturbs a word this call has tagged; every live chunk has
// claimed the word before its own add, so the count starts from this call's
// zero.  The completing chunk resets the word to 0 (a chunk without tokens
// that claims after that leaves (epoch, 0): a replay of the same launch
// counts from it, any other call sees a foreign tag).
__device__ __forceinline__ unsigned long long split_claim_issue(unsigned long long* cnt, unsigned int epoch) {
  unsigned long long seen = 0;
  __hip_atomic_compare_exchange_strong(cnt, &seen, static_cast<unsigned long long>(epoch) << 32, __ATOMIC_RELAXED,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return seen;  // 0 when the exchange succeeded, else the word's value
}

// Completes the claim (from the first exchange's answer) and arrives; true
// for the chunk that completes the word.
__device__ __forceinline__ bool split_arrive(unsigned long long* cnt, unsigned int epoch, unsigned long long seen,
                                             int n_live) {
  const unsigned long long tag = static_cast<unsigned long long>(epoch) << 32;
  // a failed exchange leaves the word's current value in `seen`
  while (seen != 0 && (seen >> 32) != epoch) {
    if (__hip_atomic_compare_exchange_strong(cnt, &seen, tag, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      break;
  }
  const unsigned long long now = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
  const bool last = static_cast<int>(now & 0xFFFFFFFFull) == n_live;
  if (last) __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// Split-K kernel: grid (batch, num_kv_heads, chunks), eight waves per
// workgroup, all on kv head h = blockIdx.y.  Chunk z covers tokens
// [z * split, (z + 1) * split) of its sequence; wave w takes the chunk's
// tiles w, w + 8, w + 16, ... (the eight waves read eight neighbouring
// 32-token tiles of the same head together).  The waves' (m, l, acc) are
// merged through LDS; a sequence with one live chunk writes its output there
// and then, otherwise the chunk writes a partial and the last chunk of
// (sequence, kv head) to arrive merges all of them: no second launch.
template <int QDT, bool SCALED, bool PAGE_ALIGNED, bool QVEC, int CB>
__global__ void __launch_bounds__(512)
paged_decode_split_kernel(const DecodeArgs a) {
  // CB: bytes per cache element, 1 (FP8, scaled or unit) or 2 (a bf16 / f16
  // cache of the query's dtype, unscaled)
  static_assert(CB == 1 || (CB == 2 && !SCALED && QDT != PRISM_DTYPE_F32), "16-bit caches: unscaled, 16-bit q");
  using Tile = typename std::conditional<CB == 1, TileRegs, TileRegs16>::type;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // tile lane of this wave (uniform)
  const int g = lane >> 4;
  const int c = lane & 15;
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int z = blockIdx.z;
  const int G = a.groups;
  const int nkv = a.num_kv_heads;

  unsigned long long* const cnt = a.split_cnt + static_cast<int64_t>(b) * nkv + h;
  unsigned long long claim_seen = 0;  // thread 0: the claim exchange's answer
  const int c_begin = z * a.split;
  int t0 = c_begin + wv * kTile;
  // The block id of this wave's first tile is requested together with the
  // context length (both scalar loads, one round trip), so the first K/V
  // loads do not wait for two dependent trips.
  int32_t blk0 = 0;
  if constexpr (PAGE_ALIGNED) {
    if (t0 < a.width * a.page_size) blk0 = ld_meta(a.bt + static_cast<int64_t>(b) * a.bt_sb + (t0 / a.page_size) * a.bt_sn);
  }
  const int n_eff = effective_len(a, b);
  if (c_begin >= n_eff) {
    if (z == 0) {
      // No attended token: zeros (the reference kernel's l == 0 branch).
      for (int idx = threadIdx.x; idx < G * kHeadDim; idx += blockDim.x) {
        const int qh = h * G + idx / kHeadDim;
        const int d = idx % kHeadDim;
        store_out<QDT>(a.out, b * a.o_sb + qh * a.o_sh + d * a.o_sd, 0.f);
      }
    }
    return;
  }
  const int c_end = min(c_begin + a.split, n_eff);
  const int n_live = (n_eff + a.split - 1) / a.split;  // chunks with attended tokens (>= 1)

  floatx4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max (log2 domain) of q head c
  float l_run = 0.f;        // this lane's share of the running sum

  if (t0 < c_end) {  // wave-uniform; a wave past the chunk's end keeps empty state
    // First tile's loads go out before the query is read and converted.
    Tile ta, tb;
    auto load = [&](int t, Tile& r, int32_t pre, bool use_pre) {
      if constexpr (CB == 1) load_tile<SCALED, PAGE_ALIGNED>(a, b, h, g, c, t, c_end, r, pre, use_pre);
      else load_tile16<PAGE_ALIGNED>(a, b, h, g, c, t, c_end, r, pre, use_pre);
    };
    load(t0, ta, blk0, true);
    // The claim goes out behind the first tile's loads (the load counter is
    // in order: ahead of them it would delay the first tile by its own
    // round trip) and is not waited for before the arrival.
    if (n_live > 1 && threadIdx.x == 0) claim_seen = split_claim_issue(cnt, a.epoch);

    // ---- query operand (B of QK): column c = q head h*G + c, k slot 8g+e of
    // chunk cc <-> dim 32g + 8cc + e.
    QOperand<QDT> qop;
    {
      // Lanes c >= G read q head h*G (a valid row) and zero their copy, so the
      // loads carry no branch.
      const bool qvalid = c < G;
      const int64_t qbase =
          static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(h * G + (qvalid ? c : 0)) * a.q_sh;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        float x[8];
        const int64_t d0 = 32 * g + 8 * cc;
        if constexpr (QVEC) {
          if constexpr (QDT == PRISM_DTYPE_F32) {
            const floatx4* p = reinterpret_cast<const floatx4*>(static_cast<const float*>(a.q) + qbase + d0);
            const floatx4 lo = p[0], hi = p[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = lo[e], x[4 + e] = hi[e];
          } else {
            const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) + qbase + d0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (QDT == PRISM_DTYPE_BF16) {
                x[2 * e] = bf16_bits_to_f32(w[e] & 0xFFFFu);
                x[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
              } else {
                x[2 * e] = f16_bits_to_f32(w[e] & 0xFFFFu);
                x[2 * e + 1] = f16_bits_to_f32(w[e] >> 16);
              }
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = load_q<QDT>(a.q, qbase + (d0 + e) * a.q_sd);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float xv = qvalid ? x[e] : 0.f;
          if constexpr (QDT == PRISM_DTYPE_F16) {
            qop.hi[cc][e] = static_cast<_Float16>(xv);
          } else {
            const __bf16 hi = static_cast<__bf16>(xv);
            qop.hi[cc][e] = hi;
            if constexpr (QDT == PRISM_DTYPE_F32) qop.lo[cc][e] = static_cast<__bf16>(xv - static_cast<float>(hi));
          }
        }
      }
    }


    // One 32-token tile of kv head h: QK, online softmax, PV.
    auto compute = [&](Tile& cur) {
      // ---- QK
      floatx4 sc[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        floatx4 accs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          if constexpr (CB == 2) {  // the cache rows are already MFMA operands
            if constexpr (QDT == PRISM_DTYPE_F16)
              accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur.k[hh][cc]), qop.hi[cc],
                                                            accs, 0, 0, 0);
            else
              accs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, cur.k[hh][cc]), qop.hi[cc],
                                                             accs, 0, 0, 0);
            continue;
          } else {
          const uint32_t w0 = cur.k[hh][cc >> 1][(cc & 1) * 2];
          const uint32_t w1 = cur.k[hh][cc >> 1][(cc & 1) * 2 + 1];
          if constexpr (QDT == PRISM_DTYPE_F16) {
            accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8(w0, w1), qop.hi[cc], accs, 0, 0, 0);
          } else {
            const bf16x8 kb = fp8x8_to_bf16x8(w0, w1);
            accs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qop.hi[cc], accs, 0, 0, 0);
            if constexpr (QDT == PRISM_DTYPE_F32)
              accs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qop.lo[cc], accs, 0, 0, 0);
          }
          }
        }
        sc[hh] = accs;
      }

      // ---- online softmax (log2 domain).  Value e of this lane: half e/4, row e%4.
      float x[8];
      float tmax = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool ok = ((cur.kvalid >> e) & 1u) && c < G;
        float ksc = 1.f;
        if constexpr (CB == 1) ksc = cur.ksc[e];
        const float v = sc[e >> 2][e & 3] * (ksc * a.scale_log2);
        x[e] = ok ? v : -INFINITY;
        tmax = fmaxf(tmax, x[e]);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      const float m_new = fmaxf(m_run, tmax);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);
      m_run = m_new;
      // P * v_scale as a hi/lo pair of the PV MFMA's 16-bit type (about 16
      // significant bits): the PV product then matches fp32 accumulation
      // closely (V itself is exact).  bf16 for FP8 and bf16 caches, f16 for
      // an f16 cache (P <= 1 there: no scale).
      using PvT = typename std::conditional<CB == 2 && QDT == PRISM_DTYPE_F16, f16x8, bf16x8>::type;
      float psum = 0.f;
      PvT pa, pa_lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = exp2f(x[e] - m_use);  // 0 for masked slots
        psum += p;
        float vsc = 1.f;
        if constexpr (CB == 1) vsc = cur.vsc[e];
        const float pv = ((cur.kvalid >> e) & 1u) ? p * vsc : 0.f;
        if constexpr (CB == 2 && QDT == PRISM_DTYPE_F16) {
          const _Float16 hi = static_cast<_Float16>(pv);
          pa[e] = hi;
          pa_lo[e] = static_cast<_Float16>(pv - static_cast<float>(hi));
        } else {
          const __bf16 hi = static_cast<__bf16>(pv);
          pa[e] = hi;
          pa_lo[e] = static_cast<__bf16>(pv - static_cast<float>(hi));
        }
      }
      l_run = l_run * alpha + psum;

      // Rescale accumulator rows (q heads 4g+i) by their alpha.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ai = __shfl(alpha, 4 * g + i);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j][i] *= ai;
      }

      // Rows past the end of the chunk may hold anything (NaN codes included);
      // their V bytes are zeroed because the PV MFMA would turn 0 * NaN into
      // NaN.  (Done here, at use, so the prefetch of this tile stays
      // asynchronous.)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (!((cur.kvalid >> e) & 1u)) {
          if constexpr (CB == 1) cur.v[e] = u32x2{0, 0};
          else cur.v[e] = u32x4{0, 0, 0, 0};
        }
      }

      // ---- PV: B operand of N-tile j = element j of the lane's 8 V rows.
#pragma unroll
      for (int jp = 0; jp < 4; ++jp) {  // column pairs (2jp, 2jp+1)
        const int j = 2 * jp;
        PvT b0, b1;
        if constexpr (CB == 2) {
          // dims 8c + 2jp and 8c + 2jp + 1 are the low and high halves of
          // dword jp of each token's row: pair them across slot pairs
#pragma unroll
          for (int ep = 0; ep < 4; ++ep) {  // slot pairs (2ep, 2ep+1)
            const uint32_t lo = cur.v[2 * ep][jp];
            const uint32_t hi = cur.v[2 * ep + 1][jp];
            const uint32_t w0 = __builtin_amdgcn_perm(hi, lo, 0x05040100u);  // low halves
            const uint32_t w1 = __builtin_amdgcn_perm(hi, lo, 0x07060302u);  // high halves
            using Pair = typename std::conditional<QDT == PRISM_DTYPE_F16, f16x2, bf16x2>::type;
            const Pair c0 = __builtin_bit_cast(Pair, w0);
            const Pair c1 = __builtin_bit_cast(Pair, w1);
            b0[2 * ep] = c0[0];
            b0[2 * ep + 1] = c0[1];
            b1[2 * ep] = c1[0];
            b1[2 * ep + 1] = c1[1];
          }
        } else {
          const int dw = j >> 2;
          const int jj = j & 3;
          const uint32_t sel = (jj) | ((4 + jj) << 8) | ((jj + 1) << 16) | ((5 + jj) << 24);
#pragma unroll
          for (int ep = 0; ep < 4; ++ep) {  // slot pairs (2ep, 2ep+1)
            const uint32_t lo = cur.v[2 * ep][dw];
            const uint32_t hi = cur.v[2 * ep + 1][dw];
            const uint32_t pr = __builtin_amdgcn_perm(hi, lo, sel);
            const bf16x2 cj = fp8x2_to_bf16x2<false>(pr);
            const bf16x2 cj1 = fp8x2_to_bf16x2<true>(pr);
            b0[2 * ep] = cj[0];
            b0[2 * ep + 1] = cj[1];
            b1[2 * ep] = cj1[0];
            b1[2 * ep + 1] = cj1[1];
          }
        }
        if constexpr (CB == 2 && QDT == PRISM_DTYPE_F16) {
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, b0, acc[j], 0, 0, 0);
          acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, b1, acc[j + 1], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_lo, b0, acc[j], 0, 0, 0);
          acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_lo, b1, acc[j + 1], 0, 0, 0);
        } else {
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, b0, acc[j], 0, 0, 0);
          acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, b1, acc[j + 1], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_lo, b0, acc[j], 0, 0, 0);
          acc[j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_lo, b1, acc[j + 1], 0, 0, 0);
        }
      }
    };

    // Ping-pong prefetch over this wave's tiles (stride 8 tiles): the next
    // tile's loads are in flight while the current one is computed.  The
    // loads are unconditional (past the end they re-read the current tile, a
    // cache hit) so the waitcnt pass can count them exactly.
    constexpr int kStep = kSplitWaves * kTile;
    while (true) {
      int tn = (t0 + kStep < c_end) ? t0 + kStep : t0;
      load(tn, tb, -1, false);
      compute(ta);
      t0 += kStep;
      if (t0 >= c_end) break;
      tn = (t0 + kStep < c_end) ? t0 + kStep : t0;
      load(tn, ta, -1, false);
      compute(tb);
      t0 += kStep;
      if (t0 >= c_end) break;
    }
  }

  // ---- merge the eight waves through LDS.  Wave w's row r (q head h*G + r)
  // goes to s_acc[(w * G + r) * 128 + d]; its (m, l) to s_ml[w][r].
  __shared__ float s_acc[kSplitWaves * 16 * kHeadDim];
  __shared__ float2 s_ml[kSplitWaves * 16];
  __shared__ int s_last;
  {
    float l_tot = l_run + __shfl_xor(l_run, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (g == 0) s_ml[wv * 16 + c] = float2{m_run, l_tot};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      if (r < G) {
        floatx4* dst = reinterpret_cast<floatx4*>(s_acc + (wv * G + r) * kHeadDim + 8 * c);
        dst[0] = floatx4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
        dst[1] = floatx4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]};
      }
    }
  }
  // LDS-only barrier: outstanding global operations (the claim) need not
  // complete here.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  const int64_t prow0 = ((static_cast<int64_t>(b) * nkv + h) * a.max_splits + z) * G;  // first partial row
  for (int e = threadIdx.x; e < G * kHeadDim; e += blockDim.x) {
    const int r = e / kHeadDim;
    const int d = e - r * kHeadDim;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) mx = fmaxf(mx, s_ml[w * 16 + r].x);
    const float m_use = mx == -INFINITY ? 0.f : mx;
    float l_sum = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) {
      const float2 ml = s_ml[w * 16 + r];
      const float wgt = exp2f(ml.x - m_use);  // 0 for a wave without attended tokens
      l_sum += wgt * ml.y;
      o += wgt * s_acc[(w * G + r) * kHeadDim + d];
    }
    if (n_live == 1) {
      const float inv = l_sum > 0.f ? 1.f / l_sum : 0.f;
      store_out<QDT>(a.out, b * a.o_sb + (h * G + r) * a.o_sh + d * a.o_sd, o * inv);
    } else {
      store_coherent(a.part_acc + (prow0 + r) * kHeadDim + d, o);
      if (d == 0) {
        store_coherent(a.part_ml + (prow0 + r) * 2, mx);
        store_coherent(a.part_ml + (prow0 + r) * 2 + 1, l_sum);
      }
    }
  }
  if (n_live == 1) return;

  // ---- arrival; the last chunk of (b, h) merges the n_live partials.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) s_last = split_arrive(cnt, a.epoch, claim_seen, n_live);
  __syncthreads();
  if (!s_last) return;

  // Thread (cg, u): unit u = float4 u of the G x 128 outputs, chunk group cg
  // takes chunks cg, cg + NG, ...; the NG groups then meet in LDS.
  const int units = G * (kHeadDim / 4);
  const int NG = blockDim.x / units;  // 1 (G = 16) .. 16 (G = 1)
  const int cg = threadIdx.x / units;
  const int u = threadIdx.x - cg * units;
  const int r = u / (kHeadDim / 4);
  const int d0 = 4 * (u - r * (kHeadDim / 4));
  const int64_t hrow0 = (static_cast<int64_t>(b) * nkv + h) * a.max_splits * G;  // chunk 0's first row
  const __amdgpu_buffer_rsrc_t acc_r = __builtin_amdgcn_make_buffer_rsrc(a.part_acc, 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t ml_r = __builtin_amdgcn_make_buffer_rsrc(a.part_ml, 0, 0x7FFFFFFF, 0x00020000);
  float m_acc = -INFINITY, l_acc = 0.f;
  floatx4 o = {0.f, 0.f, 0.f, 0.f};
  if (cg < NG) {
    constexpr int kU = 8;
    for (int k0 = cg; k0 < n_live; k0 += kU * NG) {
      float mv[kU], lv[kU];
      floatx4 xv[kU];
#pragma unroll
      for (int q = 0; q < kU; ++q) {
        const int k = k0 + q * NG;
        // only live chunks are loaded (device-scope loads bypass the caches)
        const int64_t row = hrow0 + static_cast<int64_t>(k) * G + r;
        float2 ml = {-INFINITY, 0.f};
        xv[q] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (k < n_live) {
          ml = load_coherent2(ml_r, static_cast<uint32_t>(row * 8));
          xv[q] = load_coherent4(acc_r, static_cast<uint32_t>((row * kHeadDim + d0) * 4));
        }
        mv[q] = ml.x;
        lv[q] = ml.y;
      }
      float mx = m_acc;
#pragma unroll
      for (int q = 0; q < kU; ++q) mx = fmaxf(mx, mv[q]);
      if (mx == -INFINITY) continue;  // nothing attended so far
      const float alpha = exp2f(m_acc - mx);  // 0 while m_acc = -inf
      l_acc *= alpha;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] *= alpha;
#pragma unroll
      for (int q = 0; q < kU; ++q) {
        const float wgt = mv[q] == -INFINITY ? 0.f : exp2f(mv[q] - mx);  // rows with m = -inf weigh 0
        l_acc += wgt * lv[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] += wgt * (wgt != 0.f ? xv[q][j] : 0.f);
      }
      m_acc = mx;
    }
  }
  // meet in LDS (s_acc is free again: every thread passed the barriers above)
  floatx4* red = reinterpret_cast<floatx4*>(s_acc);
  float2* red_ml = reinterpret_cast<float2*>(s_acc + 512 * 4);  // after up to 512 floatx4
  if (cg < NG) {
    red[cg * units + u] = o;
    red_ml[cg * units + u] = float2{m_acc, l_acc};
  }
  __syncthreads();
  if (cg == 0) {
    float mx = -INFINITY;
    for (int k = 0; k < NG; ++k) mx = fmaxf(mx, red_ml[k * units + u].x);
    const float m_use = mx == -INFINITY ? 0.f : mx;
    float l_sum = 0.f;
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < NG; ++k) {
      const float2 ml = red_ml[k * units + u];
      const float wgt = exp2f(ml.x - m_use);
      l_sum += wgt * ml.y;
      const floatx4 x = red[k * units + u];
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] += wgt * x[j];
    }
    const float inv = l_sum > 0.f ? 1.f / l_sum : 0.f;
    const int64_t obase = static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(h * G + r) * a.o_sh;
#pragma unroll
    for (int j = 0; j < 4; ++j) store_out<QDT>(a.out, obase + (d0 + j) * a.o_sd, s[j] * inv);
  }
}

// ---------------------------------------------------------------- streaming path
//
// Persistent, tile-balanced kernel for the canonical page layout
// ([num_blocks][P % 16 == 0][8 kv heads][128] FP8, scales [num_blocks][P][8]):
//
// * One launch.  Every workgroup first checks the plan (prefix-sharing
//   groups and the tile prefix sums, see "shared pages" below) left in the
//   workspace by an earlier call against this call's metadata; when it
//   differs, one workgroup rebuilds it into the other of two plan slots while
//   the rest wait (plan_select_slow).  The workgroups merge the partials of
//   the sequences they complete (stream_finish).
// * One workgroup (8 waves, wave = kv head) per CU.  The 16-token tiles
//   of the stream (virtual sequences over shared pages first, then every
//   sequence's own tiles) are split into gridDim.x equal contiguous ranges, so
//   every CU streams the same number of bytes whatever the context-length
//   mix.  A range spanning several stream entries emits one (m, l, acc)
//   partial per (workgroup, entry) pair; as ranges are contiguous and
//   monotone the pairs form a staircase and `wg + entry` indexes them
//   uniquely.  The last workgroup to finish a sequence combines them.
// * A tile is one contiguous slab per tensor (K [16 tok][8 h][128 B], V
//   likewise, and the fp32 scales).  The workgroup copies tiles straight into
//   LDS with global_load_lds (16 B per lane), four stages, so while the
//   workgroup computes a tile three more (about 100 KB) are in flight and no
//   VGPRs hold prefetched data.  (Measured: two workgroups per CU with two
//   stages each keep only two tiles in flight per CU and stream ~5% slower.)  16-byte chunks of a
//   head row are XOR-swizzled by token so row-parallel K reads and transposed
//   V reads spread over the banks.
//   Scales are stored [head][token] so a lane's four tokens are one 16-byte read.
// * QK: MFMA f32_16x16x128_f8f6f4 on the fp8 K rows as they are (B = Q^T
//   split into fp8 terms whose sum carries q's value, two for bf16
//   queries and three for f16/f32; 16 query
//   columns: the G heads of one sequence, or of up to 16/G sequences for a
//   virtual sequence).  Lane (g, c) gets the scores of query column c for
//   tokens 4g..4g+3.
// * PV: MFMA f32_16x16x16_bf16, whose four k slots per lane are exactly those
//   four tokens, so P needs no data movement; P * v_scale goes in as bf16
//   (2^-9 relative, fp32's exponent range; V bytes convert to bf16 exactly),
//   one MFMA per N-tile.  The V operand comes
//   from ds_read_b64_tr_b8, which hands lane i of each 16-lane group byte i of
//   eight 16-byte rows: rows 0-3 = tokens 4g..4g+3 at dims 16j.., rows 4-7 =
//   the same tokens at dims 16(j+1).., i.e. two N-tiles per read.
// * Softmax rescaling is lazy: the running max moves only when a score
//   exceeds it by more than 2^8, which after the first tiles is rare.

// The tile is 16 rows of 1 KB.  A row holds 8 head slots of 128 bytes: one
// token of an 8-kv-head cache, or 8 / Hkv consecutive tokens of an Hkv-head
// cache (Hkv = 1, 2, 4), whose token rows are 128 * Hkv bytes.  Wave h owns
// slot h: kv head h % Hkv, token h / Hkv of each row.  Everything below the
// row level (loads, LDS layout, swizzle, MFMAs) is the same for every Hkv;
// the scale of (row r, slot h) is element 8 r + h of the tile's scales in
// both layouts.
constexpr int kSKv = 8;                                 // head slots per row (waves per workgroup)
constexpr int kSTile = 16;                              // rows per tile (tokens: 16 * 8 / Hkv)
constexpr int kSStages = 4;                             // pipeline depth per workgroup
constexpr int kSWgPerCu = 1;                            // workgroups per CU
constexpr int kSRow = kSKv * kHeadDim;                  // 1024 bytes per token row
constexpr int kSKBytes = kSTile * kSRow;                // 16 KB of K per tile
constexpr int kSScaleBytes = kSTile * kSKv * 4;         // 512 B of k scales per tile
constexpr int kSStage = 2 * kSKBytes + 2 * kSScaleBytes;  // 33792 bytes
constexpr int kSMaxBatch = 1024;
constexpr int kSThreads = 64 * kSKv;
constexpr int kSWaves = kSKv;  // waves per streaming workgroup
constexpr int kSLoadsPerStage = 5;                      // per lane: 2 K, 2 V, 1 scale
constexpr float kSRescaleThreshold = 8.0f;              // log2 domain
// PV is one bf16 MFMA per N-tile with P * v_scale as one bf16 (8 significant
// bits, RNE: 2^-9 relative per weight, the precision of the bf16 output
// itself).  bf16 has fp32's exponent range, so P * v_scale needs no range
// handling for any v scale (a tile may mix rows at the 1e-6 scale floor with
// rows at 1e4), and V's E4M3FN bytes convert to bf16 exactly.

// 16-byte LDS reads at a byte address of the LDS aperture.
__device__ __forceinline__ u32x4 lds_load_b128(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(static_cast<uintptr_t>(addr));
}
__device__ __forceinline__ floatx4 lds_load_f4(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) floatx4*>(static_cast<uintptr_t>(addr));
}

// LDS layout of a tile row (16-byte chunks of 8 head slots of 128 bytes).
// gfx950 LDS (measured with SQ_LDS_BANK_CONFLICT): 64 banks of 4 bytes
// (address bits 2..7); ds_read_b64 (and _tr_b8) serves lanes 0-31 and 32-63
// in separate passes; ds_read_b128 serves 16 lanes per pass, the lanes whose
// bit 5 and parity of bits 2..4 agree.  A wave reads one head slot of every
// row, 128 bytes, i.e. one half of the banks; so that rows of opposite
// parity use opposite halves, LDS slot s of row t holds head slot
// s ^ (t & 1) (stream_slot), and inside a slot the chunks are swizzled by
// chunk ^= 4 t1 ^ 3 t2 (stream_swz, GF(2)-linear in the row index t).
// Together they make the K rows' b128 reads (lane (g, c): row c, chunks 2g,
// 2g + 1) and the V tiles' transposed b64 reads (lane (g, c): rows
// 4g + (c >> 1 & 3), chunk 2 jp + (c >> 3)) conflict-free under that model
// (the previous layout cost 4 and 2 extra cycles per read).
// Eight 16-bit transposed reads at the addresses ad[i] + off, one wait.
__device__ __forceinline__ void lds_read_tr16_x8(const uint32_t (&ad)[8], uint32_t off, uint64_t (&o)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n\t"
      "ds_read_b64_tr_b16 %1, %9\n\t"
      "ds_read_b64_tr_b16 %2, %10\n\t"
      "ds_read_b64_tr_b16 %3, %11\n\t"
      "ds_read_b64_tr_b16 %4, %12\n\t"
      "ds_read_b64_tr_b16 %5, %13\n\t"
      "ds_read_b64_tr_b16 %6, %14\n\t"
      "ds_read_b64_tr_b16 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7])
      : "v"(ad[0] + off), "v"(ad[1] + off), "v"(ad[2] + off), "v"(ad[3] + off), "v"(ad[4] + off), "v"(ad[5] + off),
        "v"(ad[6] + off), "v"(ad[7] + off)
      : "memory");
}

__device__ __forceinline__ int stream_swz(int t) { return (((t >> 1) & 1) * 4) ^ (((t >> 2) & 1) * 3); }
__device__ __forceinline__ int stream_slot(int h, int t) { return h ^ (t & 1); }




// Global tile index -> sequence, by walking the prefix sums.
__device__ __forceinline__ void advance_seq(const int* tstart, int batch, int64_t tile, int& b) {
  while (b + 1 < batch && tstart[b + 1] <= tile) ++b;
  b = __builtin_amdgcn_readfirstlane(b);  // uniform: lets the metadata reads use scalar loads
}

// Workgroup barrier without a memory fence.  __syncthreads() adds a
// workgroup-scope release that waits for every outstanding load-to-LDS,
// including the prefetch of later tiles; the stream kernel instead waits for
// exactly the current tile's loads (s_waitcnt vmcnt) before this barrier.
// The empty asm keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stream_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Per-lane, loop-invariant parts of a tile's load addresses.
struct StreamLanePlan {
  int32_t goff[2];   // byte offset of this lane's K/V chunks inside the tile slab
  int32_t soff;      // element offset of this lane's scale inside the tile's scales
  uint32_t lk[2];    // LDS offsets (from the stage base) of the K chunks' wave slice
  uint32_t ls;       // LDS offset of the scale slice
  int which;         // 0: k scales, 1: v scales
};

__device__ __forceinline__ StreamLanePlan stream_plan(int wave, int lane) {
  StreamLanePlan pl;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int p = r * (kSThreads * 16) + wave * 1024 + lane * 16;  // byte in the K slab
    const int t = p >> 10;
    const int hh = (p >> 7) & 7;
    const int chunk = ((p >> 4) & 7) ^ stream_swz(t);
    pl.goff[r] = t * kSRow + stream_slot(hh, t) * kHeadDim + chunk * 16;  // LDS slot hh holds this head slot
    pl.lk[r] = r * (kSThreads * 16) + wave * 1024;
  }
  // scales: waves 0/1 k, 2/3 v, 4-7 repeat 0-3 (same bytes, L2 hits) so
  // every wave issues the same number of loads.  LDS layout [head][token].
  const int w4 = wave & 3;
  pl.which = w4 >> 1;
  const int p = (w4 & 1) * 64 + lane;  // 0..127
  const int hh = p >> 4;
  const int t = p & 15;
  pl.soff = t * kSKv + hh;
  pl.ls = 2 * kSKBytes + pl.which * kSScaleBytes + (w4 & 1) * 256;
  return pl;
}

// Issue the loads of one tile into `stage` (5 per lane).  Written as asm so
// the compiler's waitcnt pass does not track these load-to-LDS operations (it
// cannot tell the stage buffers apart and would drain every outstanding load
// before each LDS read).  The kernel waits for them explicitly (s_waitcnt
// vmcnt + s_barrier); compiler-issued vector loads elsewhere can only
// over-wait because of them.
//
// NT selects the non-temporal cache policy.  Pages a sequence reads alone are
// touched once per call, and on MI355X streaming them with `nt` loads moves
// about 7.0 TB/s against 6.0 TB/s with the default policy (a 1 GiB
// load-to-LDS read at 256 workgroups).  Shared pages, which the virtual
// sequences of one group each walk, keep the default policy so their
// re-reads can hit in the caches.
// One tile's loads go out as scalar page base + 32-bit per-lane offset (the
// `saddr` form): the per-lane offsets are loop invariant, so a tile costs
// three 64-bit scalar adds and no vector address arithmetic.
#define PRISM_STREAM_ISSUE_ASM(POL)                                                       \
  "s_mov_b32 m0, %[lk0]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g0], %[kb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lv0]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g0], %[vb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lk1]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g1], %[kb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lv1]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g1], %[vb]" POL "\n\t"   \
  "s_mov_b32 m0, %[ls]\n\ts_nop 0\n\tglobal_load_lds_dword %[gs], %[sb]" POL

// kb / vb: the tile's first K / V byte; sb: its first scale of this lane's
// kind (k or v); stage_lds: the stage's LDS address.
// A pointer the compiler must keep in scalar registers (the asm's `saddr`).
template <typename T>
__device__ __forceinline__ T* scalar_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ void stream_issue(const StreamLanePlan& pl, const uint8_t* kb, const uint8_t* vb,
                                             const float* sb, uint32_t stage_lds, bool nt) {
  kb = scalar_ptr(kb);
  vb = scalar_ptr(vb);
  sb = scalar_ptr(sb);
  const uint32_t lk0 = stage_lds + pl.lk[0];
  const uint32_t lk1 = stage_lds + pl.lk[1];
  const uint32_t lv0 = lk0 + kSKBytes;
  const uint32_t lv1 = lk1 + kSKBytes;
  const uint32_t ls = stage_lds + pl.ls;
  const uint32_t g0 = static_cast<uint32_t>(pl.goff[0]);
  const uint32_t g1 = static_cast<uint32_t>(pl.goff[1]);
  const uint32_t gs = static_cast<uint32_t>(pl.soff) * 4u;
  if (nt) {  // wave-uniform
    asm volatile(PRISM_STREAM_ISSUE_ASM(" nt")
                 :
                 : [g0] "v"(g0), [g1] "v"(g1), [gs] "v"(gs), [kb] "s"(kb), [vb] "s"(vb), [sb] "s"(sb),
                   [lk0] "s"(lk0), [lk1] "s"(lk1), [lv0] "s"(lv0), [lv1] "s"(lv1), [ls] "s"(ls)
                 : "memory", "m0");
  } else {
    asm volatile(PRISM_STREAM_ISSUE_ASM("")
                 :
                 : [g0] "v"(g0), [g1] "v"(g1), [gs] "v"(gs), [kb] "s"(kb), [vb] "s"(vb), [sb] "s"(sb),
                   [lk0] "s"(lk0), [lk1] "s"(lk1), [lv0] "s"(lv0), [lv1] "s"(lv1), [ls] "s"(ls)
                 : "memory", "m0");
  }
}
#undef PRISM_STREAM_ISSUE_ASM

// ---- 16-bit caches (bf16 or f16 of the query's dtype, no scales; 8 kv
// heads).  A token row is 8 head slots of 256 bytes (2 KB) and a tile is
// still 16 tokens: 32 KB of K and 32 KB of V, so a stage is 64 KB and the
// workgroup keeps two stages (one tile in flight while one is computed).
// Inside a head slot the 16-byte chunks are swizzled by chunk ^= 8 t0 ^ 5 t1
// ^ 2 t2 (t the token in the tile): under the LDS model above this makes the
// K reads (lane (g, c): token c, chunks 4g .. 4g + 3, b128) and the
// transposed V reads (lane j of group g: token 4g + (j >> 2), 8 bytes at
// 32 nt + 8 (j & 3), b64_tr_b16) conflict-free; a 256-byte slot spans every
// bank, so no slot permutation is needed.
constexpr int kS16Row = kSKv * kHeadDim * 2;  // 2048 bytes per token row
constexpr int kS16KBytes = kSTile * kS16Row;  // 32 KB of K per tile
constexpr int kS16Stage = 2 * kS16KBytes;     // K then V
constexpr int kS16Stages = 2;
constexpr int kS16LoadsPerStage = 8;          // per lane: 4 K, 4 V
static_assert(kS16Stages * kS16Stage <= kSStages * kSStage, "the 16-bit stages fit the stage buffer");

__device__ __forceinline__ int stream_swz16(int t) {
  return ((t & 1) * 8) ^ (((t >> 1) & 1) * 5) ^ (((t >> 2) & 1) * 2);
}

// Per-lane offsets of a 16-bit tile's loads (the same for K and V): load r of
// wave w fills LDS bytes [8 KB r + 1 KB w, +1 KB) of the K (or V) slab.
struct StreamLanePlan16 {
  int32_t goff[4];  // byte offset of this lane's chunk inside the tile slab
  uint32_t lk[4];   // LDS offset (from the stage base) of the wave's kilobyte
};

__device__ __forceinline__ StreamLanePlan16 stream_plan16(int wave, int lane) {
  StreamLanePlan16 pl;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int p = r * (kSThreads * 16) + wave * 1024 + lane * 16;  // byte in the LDS slab
    const int t = p >> 11;
    const int hh = (p >> 8) & 7;
    const int chunk = ((p >> 4) & 15) ^ stream_swz16(t);
    pl.goff[r] = t * kS16Row + hh * (2 * kHeadDim) + chunk * 16;
    pl.lk[r] = r * (kSThreads * 16) + wave * 1024;
  }
  return pl;
}

#define PRISM_STREAM16_ISSUE_ASM(POL)                                                     \
  "s_mov_b32 m0, %[lk0]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g0], %[kb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lk1]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g1], %[kb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lk2]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g2], %[kb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lk3]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g3], %[kb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lv0]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g0], %[vb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lv1]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g1], %[vb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lv2]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g2], %[vb]" POL "\n\t"   \
  "s_mov_b32 m0, %[lv3]\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[g3], %[vb]" POL

__device__ __forceinline__ void stream_issue16(const StreamLanePlan16& pl, const uint8_t* kb, const uint8_t* vb,
                                               uint32_t stage_lds, bool nt) {
  kb = scalar_ptr(kb);
  vb = scalar_ptr(vb);
  const uint32_t lk0 = stage_lds + pl.lk[0], lk1 = stage_lds + pl.lk[1];
  const uint32_t lk2 = stage_lds + pl.lk[2], lk3 = stage_lds + pl.lk[3];
  const uint32_t lv0 = lk0 + kS16KBytes, lv1 = lk1 + kS16KBytes, lv2 = lk2 + kS16KBytes, lv3 = lk3 + kS16KBytes;
  const uint32_t g0 = static_cast<uint32_t>(pl.goff[0]), g1 = static_cast<uint32_t>(pl.goff[1]);
  const uint32_t g2 = static_cast<uint32_t>(pl.goff[2]), g3 = static_cast<uint32_t>(pl.goff[3]);
  if (nt) {  // wave-uniform
    asm volatile(PRISM_STREAM16_ISSUE_ASM(" nt")
                 :
                 : [g0] "v"(g0), [g1] "v"(g1), [g2] "v"(g2), [g3] "v"(g3), [kb] "s"(kb), [vb] "s"(vb),
                   [lk0] "s"(lk0), [lk1] "s"(lk1), [lk2] "s"(lk2), [lk3] "s"(lk3), [lv0] "s"(lv0), [lv1] "s"(lv1),
                   [lv2] "s"(lv2), [lv3] "s"(lv3)
                 : "memory", "m0");
  } else {
    asm volatile(PRISM_STREAM16_ISSUE_ASM("")
                 :
                 : [g0] "v"(g0), [g1] "v"(g1), [g2] "v"(g2), [g3] "v"(g3), [kb] "s"(kb), [vb] "s"(vb),
                   [lk0] "s"(lk0), [lk1] "s"(lk1), [lk2] "s"(lk2), [lk3] "s"(lk3), [lv0] "s"(lv0), [lv1] "s"(lv1),
                   [lv2] "s"(lv2), [lv3] "s"(lv3)
                 : "memory", "m0");
  }
}
#undef PRISM_STREAM16_ISSUE_ASM

// Query operand of one wave: column c (0..15) holds one query vector.
template <int QDT, bool QVEC>
__device__ __forceinline__ void stream_load_q(const DecodeArgs& a, int qrow, int qhead, bool qvalid, int g,
                                              QOperand<QDT>& qop) {
  const int64_t qbase = static_cast<int64_t>(qrow) * a.q_sb + static_cast<int64_t>(qhead) * a.q_sh;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    float x[8];
    const int64_t d0 = 32 * g + 8 * cc;
    if constexpr (QVEC) {
      if constexpr (QDT == PRISM_DTYPE_F32) {
        const floatx4* p = reinterpret_cast<const floatx4*>(static_cast<const float*>(a.q) + qbase + d0);
        const floatx4 lo = p[0], hi = p[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = lo[e], x[4 + e] = hi[e];
      } else {
        const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) + qbase + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (QDT == PRISM_DTYPE_BF16) {
            x[2 * e] = bf16_bits_to_f32(w[e] & 0xFFFFu);
            x[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
          } else {
            x[2 * e] = f16_bits_to_f32(w[e] & 0xFFFFu);
            x[2 * e + 1] = f16_bits_to_f32(w[e] >> 16);
          }
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = load_q<QDT>(a.q, qbase + (d0 + e) * a.q_sd);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xv = qvalid ? x[e] : 0.f;
      if constexpr (QDT == PRISM_DTYPE_F16) {
        qop.hi[cc][e] = static_cast<_Float16>(xv);
      } else {
        const __bf16 hi = static_cast<__bf16>(xv);
        qop.hi[cc][e] = hi;
        if constexpr (QDT == PRISM_DTYPE_F32) qop.lo[cc][e] = static_cast<__bf16>(xv - static_cast<float>(hi));
      }
    }
  }
}



// Query operand of the streaming kernel for the fp8 MFMA (16x16x128): lane
// (g, c) holds column c's dims 32g..32g+31 as fp8 bytes, the same bytes of
// the K rows it multiplies.  Each column is scaled by 2^e so that its
// largest |q| lies in [128, 256), then split into three E4M3FN terms,
// hi + mid + lo, each the round-to-nearest of what the previous terms left
// (four significant bits per term).  A bf16 query (eight bits) is held
// exactly by hi + mid for elements of 2^-2 and up after scaling (2^-10 of
// the column's largest) and within 2^-10 below (2^-18 of the largest); its
// lo term is then zero, so the kernel skips that MFMA for bf16 queries.  An
// f16 query is held exactly from 2 up and within 2^-10 below, an f32 query
// to about 2^-12 relative.  The score is then (K . (hi + mid + lo)) * 2^-e,
// and 2^-e is folded into the per-column score multiplier.
struct QOperandF8 {
  i32x8 t[3];      // hi, mid, lo
  float colscale;  // scale_log2 * 2^-e of this lane's column
};

// B operand of S^T = K Q^T for 16-bit caches (bf16 / f16 MFMA 16x16x32):
// lane (g, c) holds query column c's dims 32g + 8kb .. 32g + 8kb + 7 for MFMA
// kb, the dims of the K chunk 4g + kb it meets.
struct QOperand16 {
  u32x4 t[4];
  float colscale;  // scale_log2
};

template <int QDT, bool QVEC>
__device__ __forceinline__ void stream_load_q16(const DecodeArgs& a, int qrow, int qhead, bool qvalid, int g,
                                                QOperand16& qop) {
  const int64_t qbase = static_cast<int64_t>(qrow) * a.q_sb + static_cast<int64_t>(qhead) * a.q_sh;
  const uint16_t* q = static_cast<const uint16_t*>(a.q);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int64_t d0 = 32 * g + 8 * kb;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (qvalid) {
      if constexpr (QVEC) {
        w = *reinterpret_cast<const u32x4*>(q + qbase + d0);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = static_cast<uint32_t>(q[qbase + (d0 + 2 * e) * a.q_sd]) |
                 (static_cast<uint32_t>(q[qbase + (d0 + 2 * e + 1) * a.q_sd]) << 16);
      }
    }
    qop.t[kb] = w;
  }
  qop.colscale = a.scale_log2;
}

template <int QDT, bool QVEC>
__device__ __forceinline__ void stream_load_q8(const DecodeArgs& a, int qrow, int qhead, bool qvalid, int g,
                                               QOperandF8& qop) {
  const int64_t qbase = static_cast<int64_t>(qrow) * a.q_sb + static_cast<int64_t>(qhead) * a.q_sh;
  float x[32];
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    const int64_t d0 = 32 * g + 8 * cc;
    float* xc = x + 8 * cc;
    if constexpr (QVEC) {
      if constexpr (QDT == PRISM_DTYPE_F32) {
        const floatx4* p = reinterpret_cast<const floatx4*>(static_cast<const float*>(a.q) + qbase + d0);
        const floatx4 lo = p[0], hi = p[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) xc[e] = lo[e], xc[4 + e] = hi[e];
      } else {
        const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) + qbase + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (QDT == PRISM_DTYPE_BF16) {
            xc[2 * e] = bf16_bits_to_f32(w[e] & 0xFFFFu);
            xc[2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
          } else {
            xc[2 * e] = f16_bits_to_f32(w[e] & 0xFFFFu);
            xc[2 * e + 1] = f16_bits_to_f32(w[e] >> 16);
          }
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xc[e] = load_q<QDT>(a.q, qbase + (d0 + e) * a.q_sd);
    }
  }
  float mx = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    x[e] = qvalid ? x[e] : 0.f;
    mx = fmaxf(mx, fabsf(x[e]));
  }
  mx = wave_max_across_groups(mx);
  // 2^e puts the column's largest |q| in [128, 256); clamped so that 2^-e
  // stays a normal fp32 number (columns of zeros keep e = 0).
  // ilogb(mx) = frexp exponent - 1 (exact for subnormals too, no library call)
  const int e = (mx > 0.f && mx <= 3.0e38f) ? min(max(8 - __builtin_amdgcn_frexp_expf(mx), -120), 120) : 0;
  qop.colscale = ldexpf(a.scale_log2, -e);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const float y[4] = {ldexpf(x[4 * w], e), ldexpf(x[4 * w + 1], e), ldexpf(x[4 * w + 2], e),
                        ldexpf(x[4 * w + 3], e)};
    uint32_t parts[3];
    fp8_split3(y, parts);
#pragma unroll
    for (int t = 0; t < 3; ++t) qop.t[t][w] = static_cast<int>(parts[t]);
  }
}

// ------------------------------------------------------------ shared pages
//
// Prefix sharing: sequences whose block tables start with the same physical
// pages (a shared read-only prefix) would each stream those pages.  The plan
// build finds, on the device, groups of sequences with the same first page
// and, per member, how many leading whole pages it shares with the group's
// leader (the lowest-numbered member).  Members are packed M = vcols / G at
// a time into "virtual sequences": a virtual sequence walks the leader's
// shared pages once with a query operand whose vcols columns are the G query
// heads of each of its M members, so every shared page is read once per M
// members instead of once per member.  vcols is 32 (two MFMA column blocks
// computed from one LDS tile) on FP8 tiles of 8 kv heads and 16 (one block)
// otherwise.  A member then
// streams only its private tail (the tokens after the shared pages), and the
// merge combines the partials of its tail with those of its virtual sequence.
//
// Plan slot layout (int32; two slots follow the plan word at the start of
// the workspace):
//   [0] V (virtual sequences), [1] total tiles
//   tstart[NS + 1]      tile prefix sums over the stream order, NS = V + batch:
//                       virtual sequences first, then the real ones
//   skip[batch]         tokens a real sequence leaves to its virtual sequence
//   vslot[batch]        v * kVMax + member slot, or -1
//   vsrc[kSMaxVirt]     block-table row (the leader) of virtual sequence v
//   vmem[kSMaxVirt][kVMax] members of v (-1 = unused slot)
//   vrot[kSMaxVirt]     tile at which virtual sequence v starts its walk (it
//                       wraps around): the virtual sequences of one group
//                       start at different pages, so the workgroups reading
//                       them at the same time do not all hit the same pages
//
// Work split: workgroup w streams the tiles whose cost positions fall in
// [w * total / nwg, (w+1) * total / nwg) of the stream (cost model below);
// ranges are contiguous and in stream order, so the pair
// (workgroup, stream entry) indexes a partial uniquely as w + entry.

constexpr int kSCols = 16;                 // query columns of the MFMA operand
constexpr int kVMax = 32;                  // query columns of a virtual sequence at most (two column blocks)
constexpr int kSMinKv = 1;                 // fewest kv heads on the streaming path (8 token slots)
constexpr int kSMaxWg = 1024;              // grid size bound of the streaming kernel
constexpr int kSMaxVirt = 128;             // virtual sequences (>= 2 members each)
constexpr int kSShareMaxBatch = 256;       // batches above this are not analysed
constexpr int kPlanMaxPages = 64;          // leading pages compared per sequence
constexpr int kPlanTstart = 16;
constexpr int kPlanSkip = kPlanTstart + kSMaxBatch + kSMaxVirt + 16;
constexpr int kPlanVslot = kPlanSkip + kSMaxBatch;
constexpr int kPlanVsrc = kPlanVslot + kSMaxBatch;
constexpr int kPlanVmem = kPlanVsrc + kSMaxVirt;
constexpr int kPlanVrot = kPlanVmem + kSMaxVirt * kVMax;  // first tile of each virtual walk
constexpr int kPlanWgTime = kPlanVrot + kSMaxVirt;         // measurement aid: per-workgroup times
// Key of the plan: everything the plan is computed from.  A call whose
// inputs equal the key left by the previous call on the same workspace keeps
// that plan (every layer of a decode step has the same metadata).
// Per real sequence b, 8 ints at kPlanRec + 8 b: first and end tile of its
// own stream entry, its virtual slot (or -1), first and end tile of its
// virtual sequence, and the number of partial flushes its output waits for
// (workgroups meeting its own tiles plus those meeting its virtual
// sequence's): what the merge needs, at an offset independent of V.
constexpr int kPlanRec = kPlanWgTime + 2 * kSMaxWg;
// Per streaming workgroup w, 8 ints at kPlanWgRec + 8 w: where its range
// starts (stream entry, tile within it, the entry's tile count, block-table
// row, first token, end token, rotation) and the raw block id of its first
// tile's page (kNoBlock when that page is outside the compared block-table
// prefix: only pages the plan's key covers may be cached here).  Empty
// ranges hold entry -1.  The streaming kernel starts from this record
// instead of searching the prefix sums and reading the entry's metadata.
constexpr int kPlanWgRec = kPlanRec + 8 * kSMaxBatch;
constexpr int kNoBlock = INT_MIN;
constexpr int kPlanKey = kPlanWgRec + 8 * kSMaxWg;
constexpr int kPlanKeyParams = 12;
constexpr int kPlanKeyEff = kPlanKey + kPlanKeyParams;       // attended lengths
constexpr int kPlanKeyBt = kPlanKeyEff + kSMaxBatch;         // compared block-table prefix
// Per real sequence b, one int at kPlanCnt + b: how many workgroups have
// flushed a partial that sequence's output depends on in the running call.
// A plan build zeroes them in the slot it writes; the workgroup whose
// flush completes a sequence merges it and sets the counter back to 0, so a
// call that reuses the plan finds them at zero.
constexpr int kPlanCnt = kPlanKeyBt + kSShareMaxBatch * kPlanMaxPages;
constexpr int kPlanInts = kPlanCnt + kSMaxBatch + kSMaxWg;  // + measurement aid: finish times
// The plan region of the workspace: the plan word (below), then two plan
// slots of kPlanInts each (4 KB multiples, so no cache line holds parts of
// both), then the measurement build's stamps.
constexpr int kPlanHdrInts = 1024;
constexpr int kPlanSlotInts = (kPlanInts + 1023) / 1024 * 1024;
constexpr int kPlanMeasure = kPlanHdrInts + 2 * kPlanSlotInts;
constexpr int kPlanBuildStamps = kPlanMeasure + 8 * kSMaxWg + 4 * kSMaxWg * kSKv;  // measurement aid: 16 ints
constexpr int kPlanMergeStamps = kPlanBuildStamps + 16;  // measurement aid: 4 ints per workgroup
constexpr int kPlanPrologueStamps = kPlanMergeStamps + 4 * kSMaxWg;  // measurement aid: 4 ints per workgroup
constexpr int kPlanRegionInts = kPlanPrologueStamps + 4 * kSMaxWg;
constexpr int kPlanMagic = 0x504C414E;
static_assert(kPlanKeyBt % 4 == 0 && kPlanHdrInts % 4 == 0 && kPlanSlotInts % 4 == 0, "16-byte key reads");
constexpr int kPlanThreads = 1024;
constexpr int kPlanHashBits = 10;
constexpr int kPlanHash = 1 << kPlanHashBits;  // >= 2 * kSShareMaxBatch slots
static_assert(2 * kSShareMaxBatch <= kPlanHash, "hash table load factor");
static_assert(kSShareMaxBatch / 2 <= kSMaxVirt, "virtual sequences of a full batch fit");
static_assert(kSShareMaxBatch <= kSThreads, "one thread per sequence in the sharing analysis");

// Work split: workgroup w streams tiles [floor(w * total / nwg),
// floor((w + 1) * total / nwg)).  (Measured on MI355X: per-workgroup times
// vary with stream position and with the order in which workgroups reach a
// CU, but the kernel is bandwidth-bound in aggregate, so neither weighting the
// split nor handing out the last tiles dynamically shortened it.)
struct StreamSplit {
  int64_t total, nwg;
};

__device__ __forceinline__ StreamSplit stream_split(const DecodeArgs& a, int64_t total) {
  return StreamSplit{total, a.stream_nwg};
}

// floor(x / d) for 0 <= x < 2^53, 0 < d < 2^53, through one fp64 division
// and an exact correction (64-bit integer division is a long emulated
// sequence; these run on the merge's critical path).  The operands convert to
// fp64 exactly, so the correctly rounded quotient is at least floor(x / d)
// and exceeds it by at most one.
__device__ __forceinline__ int64_t div_floor_small(int64_t x, int64_t d) {
  int64_t q = static_cast<int64_t>(static_cast<double>(x) / static_cast<double>(d));
  q -= q * d > x ? 1 : 0;
  q += (q + 1) * d <= x ? 1 : 0;
  return q;
}

// (w * total < 2^41: total < 2^31 tiles, w <= nwg <= 1024)
__device__ __forceinline__ int64_t split_begin(const StreamSplit& sp, int64_t w) {
  return div_floor_small(w * sp.total, sp.nwg);
}

// The workgroup whose range holds tile t (0 <= t < total): the last w with
// split_begin(w) <= t, i.e. ceil((t + 1) * nwg / total) - 1.
__device__ __forceinline__ int64_t split_owner(const StreamSplit& sp, int64_t t) {
  return div_floor_small((t + 1) * sp.nwg + sp.total - 1, sp.total) - 1;
}

// Number of streaming workgroups whose ranges meet tiles [first, end) of a
// stream of `total` tiles split over nwg workgroups: each such workgroup
// flushes one partial for that tile range.  With total >= nwg every range is
// non-empty and the owners of first and end - 1 bound them; with fewer tiles
// than workgroups every range holds at most one tile.
__device__ __forceinline__ int stream_owner_count(int first, int end, int total, int nwg) {
  if (end <= first) return 0;
  if (total < nwg) return end - first;
  const StreamSplit sp{total, nwg};
  return static_cast<int>(split_owner(sp, end - 1) - split_owner(sp, first)) + 1;
}

// Cost-weighted split.  Workgroup ranges are equal in cost units rather than
// tiles: a tile of a sequence's own pages costs kCostTile, a tile of a
// virtual walk (shared pages, which the other walks of its group have pulled
// into the caches) kCostVirt, and every stream entry kCostEntry more (a range
// that starts an entry reloads the query and its first pages' metadata, and
// one that ends an entry flushes a partial).  Entry i occupies cost positions
// [cs(i), cs(i + 1)), its first kCostEntry positions charged to whichever
// range holds them, then its tiles; a tile belongs to the range holding its
// first position.  The weights apply when the stream has at least
// kCostMinTilesPerWg tiles per workgroup, so that every range still holds
// tiles; otherwise every weight is the unit one and the split is the plain
// tile split.  Measured on the batch-64 mixed step (8 kv heads, 256
// workgroups, about 124 tiles each): entry costs of 0 / 1 / 2 / 3 / 4 / 6 / 8
// / 12 tiles gave 176.0 / 174.9 / 174.5 / 173.6 / 173.6 / 172.2 / 171.9 /
// 172.6 us, and virtual tiles at 22/16 of a tile 171.1 us (at 13/16: 188 us;
// a walk of shared pages is followed by merges over its members' outputs).
// Before the weights, a workgroup meeting two entries ended its loop 2.6 us
// after one meeting one, and the last loops ended 7 us after the mean.
// With two column blocks per virtual walk (a wide walk computes both blocks
// from one LDS tile, about 1.6 us per tile against 1.25 us for a private
// tile) the measured step was, over three runs each: virtual 22 / 26 / 30 /
// 34 with entry 128: 171.0 / 169.8 / 171.6 / 170.6 us; virtual 26 with
// entry 96 / 160: 169.0 / 170.3 us.  A walk's workgroup must end its loop
// well before the others, or it completes its members' sequences and
// merges them one after another (virtual 16: 215 us, eight merges).
#ifndef PRISM_COST_ENTRY
#define PRISM_COST_ENTRY 96
#endif
#ifndef PRISM_COST_VIRT
#define PRISM_COST_VIRT 26
#endif
constexpr int kCostTile = 16;
constexpr int kCostEntry = PRISM_COST_ENTRY;
constexpr int kCostVirt = PRISM_COST_VIRT;
constexpr int kCostMinTilesPerWg = 4;
// (An entry's first kCostEntry positions may fill a whole range, which then
// holds no tile and flushes nothing; the merges only visit the ranges that
// meet an entry's tile positions, and each of those holds a tile start, as a
// weighted range spans at least kCostTile * kCostMinTilesPerWg positions.)
static_assert(kCostVirt >= 1 && kCostVirt <= kCostTile * kCostMinTilesPerWg, "a tile fits a range");

struct CostModel {
  int ce, cv, cr;  // per entry, per virtual tile, per real tile
  int V;           // virtual entries come first
  int tv;          // tiles of all virtual entries (tile prefix at entry V)
};

__device__ __forceinline__ CostModel cost_model(int tiles, int nwg, int V, int tv) {
  const bool weighted = static_cast<int64_t>(tiles) >= static_cast<int64_t>(kCostMinTilesPerWg) * nwg;
  return weighted ? CostModel{kCostEntry, kCostVirt, kCostTile, V, tv} : CostModel{0, 1, 1, V, tv};
}

// Cost position where entry i starts, from its tile prefix ti (entries before
// V are virtual).
__device__ __forceinline__ int64_t cost_start(const CostModel& m, int i, int ti) {
  const int64_t c = static_cast<int64_t>(m.ce) * i;
  return i <= m.V ? c + static_cast<int64_t>(m.cv) * ti
                  : c + static_cast<int64_t>(m.cv) * m.tv + static_cast<int64_t>(m.cr) * (ti - m.tv);
}

// Cost position of tile k of entry i.
__device__ __forceinline__ int64_t cost_of_tile(const CostModel& m, int i, int ti, int k) {
  return cost_start(m, i, ti) + m.ce + static_cast<int64_t>(i < m.V ? m.cv : m.cr) * k;
}

// Inclusive prefix sum over the workgroup of NT threads (every thread calls
// it): shuffles within each wave, one pass over the wave totals.
template <int NT>
__device__ __forceinline__ int plan_scan(int v, int* wsum_s, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum_s[wave] = x;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    const int ws = wsum_s[i];
    before += i < wave ? ws : 0;
    tot += ws;
  }
  __syncthreads();
  total = tot;
  return x + before;
}

// LDS of the plan computation (the streaming kernel lays it over its stage
// buffers, which are idle until the plan is known).
struct PlanLds {
  int eff_s[kSMaxBatch];
  int cap_s[kSMaxBatch];    // whole pages covered by the attended length (<= kPlanMaxPages)
  int full_s[kSMaxBatch];   // leading whole pages with valid block ids
  int lead_s[kSMaxBatch];   // group leader
  int sh_s[kSMaxBatch];     // leading pages equal to the leader's
  int cnt_s[kSMaxBatch];    // at a leader: members besides itself
  int smax_s[kSMaxBatch];   // at a leader: longest member share
  int vb_s[kSMaxBatch];     // at a leader: first virtual sequence
  int skip_s[kSMaxBatch];
  int vslot_s[kSMaxBatch];
  int vlen_s[kSMaxVirt];    // pages of virtual sequence v
  int vk_s[kSMaxVirt];      // chunk index of v in its group
  int vn_s[kSMaxVirt];      // virtual sequences of v's group
  int vsrc_s[kSMaxVirt];
  int vmem_s[kSMaxVirt * kVMax];
  int hkey[kPlanHash];
  int hmin[kPlanHash];
  __attribute__((aligned(16))) int bt_s[kSShareMaxBatch * kPlanMaxPages];  // compared part of the block tables
  int wsum_s[kPlanThreads / 64];
  unsigned long long w_s;  // plan word as read by thread 0
  int won_s;               // this workgroup builds the plan
  __attribute__((aligned(16))) int cnt_rank_s[kSShareMaxBatch];  // group of each member or -1
};

// Whether prefix sharing is analysed for this call.
__device__ __forceinline__ bool plan_share(const DecodeArgs& a) {
  const int Wc = min(a.width, kPlanMaxPages);
  return a.share && a.batch <= kSShareMaxBatch && (a.vcols / a.groups) >= 2 && Wc >= 1;
}

__device__ __forceinline__ void plan_key_params(const DecodeArgs& a, bool share, int (&kp)[kPlanKeyParams]) {
  const int vals[kPlanKeyParams] = {kPlanMagic, a.batch, a.width, a.page_size, a.groups,
                                    static_cast<int>(a.num_blocks & 0x7FFFFFFF),
                                    static_cast<int>(a.num_blocks >> 31), share ? a.vcols : 0, a.stream_nwg,
                                    a.num_kv_heads, 0, 0};
#pragma unroll
  for (int i = 0; i < kPlanKeyParams; ++i) kp[i] = vals[i];
}

// Compares the inputs of this call with the key stored next to the plan
// (geometry, attended lengths, compared block-table prefix, plan header)
// and stages the lengths and the compared block-table prefix into L for a
// rebuild.  Returns this thread's verdict; the workgroup ANDs them.  All
// loads of the check go out before anything is compared (one round).  The
// slot compared is one the plan word names, which no workgroup writes while
// the word names it, so ordinary loads read it whole (they are served by each
// XCD's L2: device-scope loads, which bypass it, send every workgroup of the
// launch to the same few memory channels and cost about 5 us).
template <int NT>
__device__ __forceinline__ bool plan_key_check(const DecodeArgs& a, const int* plan, PlanLds& L) {
  const int tid = threadIdx.x;
  const int B = a.batch;
  const int P = a.page_size;
  const int Wc = min(a.width, kPlanMaxPages);
  const bool share = plan_share(a);
  const int* key = plan + kPlanKey;
  auto kld = [](const int* p) { return *p; };
  int kp[kPlanKeyParams];
  plan_key_params(a, share, kp);
  // Every load of the check goes out before the first comparison: lanes
  // 0..11 read one key word each (a branch per word with a uniform address
  // would be a chain of dependent scalar loads; words 10 and 11 are copies
  // of the plan header), each thread the lengths of up to kE sequences and kU
  // entries of the compared block-table prefix, each with its key word.
  constexpr int kE = (kSMaxBatch + NT - 1) / NT;
  constexpr int kU = 8;
  const int items = share ? B * Wc : 0;
  int kword = 0, kwant = 0;  // lanes without a key word compare 0 with 0
  if (tid < kPlanKeyParams) {
    kwant = kp[0];
#pragma unroll
    for (int i = 1; i < kPlanKeyParams - 2; ++i) kwant = tid == i ? kp[i] : kwant;
    kword = kld(key + tid);
    if (tid >= kPlanKeyParams - 2) kwant = kld(plan + (tid - (kPlanKeyParams - 2)));
  }
  const int mx = ld_meta(a.max_ctx);
  int ctxv[kE], keff[kE];
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const int b = tid + e * NT;
    ctxv[e] = b < B ? a.ctx[b] : 0;
    keff[e] = b < B ? kld(key + kPlanKeyEff - kPlanKey + b) : 0;
  }
  // block-table prefix entries base + u * NT + tid with their key words
  bool same = true;
  int val[kU], old[kU];
  auto load_bt = [&](int base) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int idx = base + u * NT + tid;
      const int b = idx / Wc;
      const int j = idx - b * Wc;
      val[u] = idx < items ? a.bt[static_cast<int64_t>(b) * a.bt_sb + static_cast<int64_t>(j) * a.bt_sn] : -1;
      old[u] = idx < items ? kld(key + kPlanKeyBt - kPlanKey + idx) : -1;
    }
  };
  auto check_bt = [&](int base) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int idx = base + u * NT + tid;
      if (idx < items) L.bt_s[idx] = val[u];
      same &= old[u] == val[u];
    }
  };
  // block tables with contiguous, 16-byte aligned rows of a multiple of 4
  // compared pages: 16-byte loads, 4 entries per lane (a quarter of the
  // requests: every workgroup of the launch reads the same 2 x 16 KB)
  const bool vec = a.bt_sn == 1 && (a.bt_sb & 3) == 0 && (reinterpret_cast<uintptr_t>(a.bt) & 15) == 0 &&
                   (Wc & 3) == 0;
  constexpr int kU4 = 2;
  int4 val4[kU4], old4[kU4];
  auto load_bt4 = [&](int base) {  // entries base + 4 (u * NT + tid) .. + 3
#pragma unroll
    for (int u = 0; u < kU4; ++u) {
      const int idx = base + 4 * (u * NT + tid);
      const int b = idx / Wc;
      const int j = idx - b * Wc;
      const bool in = idx < items;
      val4[u] = in ? *reinterpret_cast<const int4*>(a.bt + static_cast<int64_t>(b) * a.bt_sb + j) : int4{-1, -1, -1, -1};
      old4[u] = in ? *reinterpret_cast<const int4*>(key + kPlanKeyBt - kPlanKey + idx) : int4{-1, -1, -1, -1};
    }
  };
  auto check_bt4 = [&](int base) {
#pragma unroll
    for (int u = 0; u < kU4; ++u) {
      const int idx = base + 4 * (u * NT + tid);
      if (idx < items) *reinterpret_cast<int4*>(&L.bt_s[idx]) = val4[u];
      same &= old4[u].x == val4[u].x && old4[u].y == val4[u].y && old4[u].z == val4[u].z &&
              old4[u].w == val4[u].w;
    }
  };
  if (vec) load_bt4(0);
  else load_bt(0);  // the first (usually only) batch leaves with the loads above
  same = kword == kwant;
  const int64_t cap_tok = static_cast<int64_t>(a.width) * P;
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const int b = tid + e * NT;
    if (b >= B) continue;
    int64_t n = ctxv[e] < mx ? ctxv[e] : mx;  // effective_len() from the loaded values
    if (n > cap_tok) n = cap_tok;
    const int ni = n > 0 ? static_cast<int>(n) : 0;
    same &= keff[e] == ni;
    L.eff_s[b] = ni;
    L.cap_s[b] = min(ni / P, Wc);
  }
  if (vec) {
    check_bt4(0);
    for (int base = 4 * kU4 * NT; base < items; base += 4 * kU4 * NT) {
      load_bt4(base);
      check_bt4(base);
    }
  } else {
    check_bt(0);
    for (int base = kU * NT; base < items; base += kU * NT) {
      load_bt(base);
      check_bt(base);
    }
  }
  return same;
}

// Builds the plan from L (filled by plan_key_check) with NT threads and
// writes it, its key and zeroed merge counters to the workspace.  tst_s
// receives the tile prefix sums (NS + 1 entries).
template <int NT>
__device__ void plan_build(const DecodeArgs& a, int* plan, PlanLds& L, int* tst_s) {
  const int tid = threadIdx.x;
  const int B = a.batch;
  const int P = a.page_size;
  const int Wc = min(a.width, kPlanMaxPages);
  const int M = a.vcols / a.groups;  // members per virtual sequence
  const bool share = plan_share(a);
  const int items = share ? B * Wc : 0;
  for (int b = tid; b < B; b += NT) {
    const int cap = L.cap_s[b];
    L.full_s[b] = cap;
    L.sh_s[b] = cap;
    L.lead_s[b] = b;
    L.cnt_s[b] = 0;
    L.smax_s[b] = 0;
    L.skip_s[b] = 0;
    L.vslot_s[b] = -1;
  }
  int V = 0;
  __syncthreads();
  if (share) {  // B <= kSShareMaxBatch <= NT here: one thread per sequence
    for (int i = tid; i < kPlanHash; i += NT) {
      L.hkey[i] = -1;
      L.hmin[i] = INT_MAX;
    }
    for (int i = tid; i < kSMaxVirt * kVMax; i += NT) L.vmem_s[i] = -1;
    __syncthreads();
    // group by first page: open addressing, the lowest index wins the slot
    int slot = -1;
    if (tid < B && L.cap_s[tid] >= 1) {
      const int raw = L.bt_s[tid * Wc];
      if (raw >= 0 && raw < a.num_blocks) {
        uint32_t hsh = (static_cast<uint32_t>(raw) * 2654435761u) >> (32 - kPlanHashBits);
        for (;;) {
          const int prev = atomicCAS(&L.hkey[hsh], -1, raw);
          if (prev == -1 || prev == raw) {
            atomicMin(&L.hmin[hsh], tid);
            slot = static_cast<int>(hsh);
            break;
          }
          hsh = (hsh + 1) & (kPlanHash - 1);
        }
      }
    }
    __syncthreads();
    if (slot >= 0) L.lead_s[tid] = L.hmin[slot];
    __syncthreads();
    // page by page: validity of each whole page, equality with the leader's
    for (int idx = tid; idx < items; idx += NT) {
      const int b = idx / Wc;
      const int j = idx - b * Wc;
      if (j >= L.cap_s[b]) continue;
      const int raw = L.bt_s[idx];
      const bool valid = raw >= 0 && raw < a.num_blocks;
      if (!valid) atomicMin(&L.full_s[b], j);
      const int ld = L.lead_s[b];
      if (ld != b) {
        const int lraw = j < L.cap_s[ld] ? L.bt_s[ld * Wc + j] : -1;
        if (!valid || lraw != raw) atomicMin(&L.sh_s[b], j);
      }
    }
    __syncthreads();
    if (tid < B && L.lead_s[tid] != tid) {
      const int sv = min(L.sh_s[tid], L.full_s[tid]);
      L.sh_s[tid] = sv;
      if (sv >= 1) {
        atomicAdd(&L.cnt_s[L.lead_s[tid]], 1);
        atomicMax(&L.smax_s[L.lead_s[tid]], sv);
      }
    }
    __syncthreads();
    // virtual sequences per group: chunks of M members in index order, kept
    // only when a chunk has at least two members
    int nv = 0;
    if (tid < B && L.lead_s[tid] == tid && L.cnt_s[tid] >= 1) {
      const int n = L.cnt_s[tid] + 1;
      nv = n / M + ((n % M) >= 2 ? 1 : 0);
    }
    const int incl = plan_scan<NT>(nv, L.wsum_s, V);
    if (tid < B) L.vb_s[tid] = incl - nv;
    for (int i = tid; i < V; i += NT) L.vlen_s[i] = INT_MAX;
    // group of each member (-1 for non-members), for the rank count below
    if (tid < kSShareMaxBatch) {
      int ml = -1;
      if (tid < B) {
        const int ld = L.lead_s[tid];
        ml = ((ld == tid) ? L.cnt_s[tid] >= 1 : L.sh_s[tid] >= 1) ? ld : -1;
      }
      L.cnt_rank_s[tid] = ml;
    }
    __syncthreads();
    if (tid < B) {
      const int ld = L.lead_s[tid];
      const bool member = L.cnt_rank_s[tid] >= 0;
      if (member) {
        // rank = members of the group with a lower index (the leader is rank 0);
        // independent 16-byte LDS reads so the latencies overlap
        int rank = 0;
        const int4* ml4 = reinterpret_cast<const int4*>(L.cnt_rank_s);
#pragma unroll 8
        for (int q = 0; q < (tid + 3) / 4; ++q) {
          const int4 x = ml4[q];
          const int b0 = 4 * q;
          rank += (b0 + 0 < tid && x.x == ld) + (b0 + 1 < tid && x.y == ld) + (b0 + 2 < tid && x.z == ld) +
                  (b0 + 3 < tid && x.w == ld);
        }
        const int n = L.cnt_s[ld] + 1;
        const int k = rank / M;
        const int chunk = min(M, n - k * M);
        if (chunk >= 2) {
          const int v = L.vb_s[ld] + k;
          const int m = rank - k * M;
          L.vmem_s[v * kVMax + m] = tid;
          L.vslot_s[tid] = v * kVMax + m;
          atomicMin(&L.vlen_s[v], ld == tid ? L.smax_s[tid] : L.sh_s[tid]);
          if (m == 0) {
            L.vsrc_s[v] = ld;
            L.vk_s[v] = k;
            L.vn_s[v] = n / M + ((n % M) >= 2 ? 1 : 0);
          }
        }
      }
    }
    __syncthreads();
    if (tid < B && L.vslot_s[tid] >= 0) L.skip_s[tid] = L.vlen_s[L.vslot_s[tid] / kVMax] * P;
    __syncthreads();
  }
  // tile prefix sums in stream order: virtual sequences, then real ones
  const int NS = B + V;
  int carry = 0;
  if (tid == 0) tst_s[0] = 0;
  for (int base = 0; base < NS; base += NT) {
    const int i = base + tid;
    int n = 0;
    if (i < V) n = L.vlen_s[i] * (P / a.s_ttok);
    else if (i < NS) n = (L.eff_s[i - V] - L.skip_s[i - V] + a.s_ttok - 1) / a.s_ttok;
    int chunk_total;
    const int incl = plan_scan<NT>(n, L.wsum_s, chunk_total);
    if (i < NS) tst_s[i + 1] = carry + incl;
    carry += chunk_total;
  }
  __syncthreads();
  const CostModel cm = cost_model(carry, a.stream_nwg, V, tst_s[V]);
  const int64_t ctotal = cost_start(cm, NS, carry);  // cost positions of the whole stream
  // ---- write-out
  for (int i = tid; i <= NS; i += NT) plan[kPlanTstart + i] = tst_s[i];
  for (int b = tid; b < B; b += NT) {
    plan[kPlanSkip + b] = L.skip_s[b];
    plan[kPlanVslot + b] = L.vslot_s[b];
    const int vs = L.vslot_s[b];
    const int v = vs >= 0 ? vs / kVMax : 0;
    // each tile range as [cost position of its first tile, that of its last + 1)
    int first = 0, end = 0, vfirst = 0, vend = 0;
    if (tst_s[V + b + 1] > tst_s[V + b]) {
      first = static_cast<int>(cost_of_tile(cm, V + b, tst_s[V + b], 0));
      end = static_cast<int>(cost_of_tile(cm, V + b, tst_s[V + b], tst_s[V + b + 1] - tst_s[V + b] - 1)) + 1;
    }
    if (vs >= 0 && tst_s[v + 1] > tst_s[v]) {
      vfirst = static_cast<int>(cost_of_tile(cm, v, tst_s[v], 0));
      vend = static_cast<int>(cost_of_tile(cm, v, tst_s[v], tst_s[v + 1] - tst_s[v] - 1)) + 1;
    }
    const int expect = stream_owner_count(first, end, static_cast<int>(ctotal), a.stream_nwg) +
                       stream_owner_count(vfirst, vend, static_cast<int>(ctotal), a.stream_nwg);
    int4* rec = reinterpret_cast<int4*>(plan + kPlanRec + 8 * b);
    rec[0] = int4{first, end, vs, vfirst};
    rec[1] = int4{vend, expect, 0, 0};
    plan[kPlanCnt + b] = 0;
  }
  for (int i = tid; i < V * kVMax; i += NT) plan[kPlanVmem + i] = L.vmem_s[i];
  for (int v = tid; v < V; v += NT) {
    plan[kPlanVsrc + v] = L.vsrc_s[v];
    plan[kPlanVrot + v] = (L.vk_s[v] * L.vlen_s[v] / L.vn_s[v]) * (P / a.s_ttok);
  }
  int kp[kPlanKeyParams];
  plan_key_params(a, share, kp);
  if (tid < kPlanKeyParams - 2) {
#pragma unroll
    for (int i = 0; i < kPlanKeyParams - 2; ++i)
      if (i == tid) plan[kPlanKey + i] = kp[i];
  }
  if (tid == 0) {  // copies of the plan header, checked before the plan is reused
    plan[kPlanKey + kPlanKeyParams - 2] = V;
    plan[kPlanKey + kPlanKeyParams - 1] = static_cast<int>(ctotal);
  }
  for (int b = tid; b < B; b += NT) plan[kPlanKeyEff + b] = L.eff_s[b];
  for (int i = tid; i < items; i += NT) plan[kPlanKeyBt + i] = L.bt_s[i];
  // the first tile at or after cost position c (carry past the end)
  auto tile_at = [&](int64_t c) -> int {
    int lo = 0, hi = NS - 1;  // the last entry starting at or before c
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cost_start(cm, mid, tst_s[mid]) <= c) lo = mid;
      else hi = mid - 1;
    }
    const int64_t rel = c - cost_start(cm, lo, tst_s[lo]) - cm.ce;
    const int step = lo < V ? cm.cv : cm.cr;
    const int64_t k = rel <= 0 ? 0 : (rel + step - 1) / step;
    return tst_s[lo] + static_cast<int>(min(k, static_cast<int64_t>(tst_s[lo + 1] - tst_s[lo])));
  };
  for (int w = tid; w < a.stream_nwg; w += NT) {
    const int s0 = NS > 0 ? tile_at(static_cast<int64_t>(w) * ctotal / a.stream_nwg) : 0;
    const int s1 = NS > 0 ? tile_at(static_cast<int64_t>(w + 1) * ctotal / a.stream_nwg) : 0;
    int4 r0 = {-1, 0, 0, 0}, r1 = {0, 0, 0, kNoBlock};
    if (s0 < s1) {
      // the entry holding tile s0: the last i with tst_s[i] <= s0
      int lo = 0, hi = NS - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tst_s[mid] <= s0) lo = mid;
        else hi = mid - 1;
      }
      const int i = lo;
      const int ilt = static_cast<int>(s0 - tst_s[i]);
      const int intl = tst_s[i + 1] - tst_s[i];
      int bt_row, tok0, n_end, rot;
      if (i >= V) {
        bt_row = i - V;
        tok0 = L.skip_s[bt_row];
        n_end = L.eff_s[bt_row];
        rot = 0;
      } else {
        bt_row = L.vsrc_s[i];
        tok0 = 0;
        n_end = intl * a.s_ttok;
        rot = (L.vk_s[i] * L.vlen_s[i] / L.vn_s[i]) * (P / a.s_ttok);
      }
      const int lr = ilt + rot;
      const int t0 = tok0 + (lr >= intl ? lr - intl : lr) * a.s_ttok;
      const int page = t0 / P;
      r0 = int4{i, ilt, s1 - s0, bt_row};  // entry, tile within it, tiles of the range, block-table row
      r1 = int4{tok0, n_end, rot, (share && page < Wc) ? L.bt_s[bt_row * Wc + page] : kNoBlock};
    }
    int4* rec = reinterpret_cast<int4*>(plan + kPlanWgRec + 8 * w);
    rec[0] = r0;
    rec[1] = r1;
  }
  if (tid == 0) {
    plan[0] = V;
    plan[1] = static_cast<int>(ctotal);
  }
}

// The plan word, 64 bits at the start of the plan region:
//   (epoch << 32) | (building << 1) | slot.
// `slot` names the plan slot holding the current plan.  A launch whose inputs
// differ from that slot's key builds the other slot and publishes it by
// rewriting the word with its own epoch; while it builds, the word carries
// the building bit and that epoch.  The slot a word names is never written
// while the word names it, so a reader that compares the key of the slot the
// word names with its inputs reads a plan that is whole: within a launch only
// the other slot is written, and a launch starts with the previous launches'
// writes visible on every XCD.
constexpr unsigned long long kPlanBuilding = 2;
constexpr int kPlanSpinLimit = 1 << 22;  // polls of a waiting workgroup (far beyond any build)
// Give-up count, one int of the plan header (kPlanGiveUps): how many
// workgroups abandoned a launch because a plan build they waited for did not
// appear within the poll limit.  Such a launch leaves the completion counters
// of the slot it used part-way (its flushes are missing), so while the count
// is nonzero every launch treats the plan as stale: it rebuilds (which zeroes
// the counters) and the builder resets the count to the value it read at the
// start of its launch, with a compare-exchange, so that a give-up of the same
// launch keeps the count nonzero for the next one.
constexpr int kPlanGiveUps = 2;

__device__ __forceinline__ unsigned long long* plan_word(const DecodeArgs& a) {
  return reinterpret_cast<unsigned long long*>(a.plan_region);
}

__device__ __forceinline__ int* plan_slot(const DecodeArgs& a, int slot) {
  return a.plan_region + kPlanHdrInts + slot * kPlanSlotInts;
}

__device__ __forceinline__ bool plan_building_here(unsigned long long w, unsigned int epoch) {
  return (w & kPlanBuilding) != 0 && static_cast<unsigned int>(w >> 32) == epoch;
}

// Plan selection after the fast check failed (the inputs differ from the key
// of the slot that word w names, or a workgroup of this launch is building):
// the first workgroup to swap the plan word from the value it read builds the
// other slot, writes it back to the device-coherent level (release fence) and
// publishes it; every other workgroup waits for the publication.  The builder
// waits for nobody, so the wait ends; it is bounded all the same (after
// kPlanSpinLimit polls the workgroup gives up with -1).  Returns the slot to
// use.  Every thread of the workgroup calls it.  `staged`: L already holds
// this call's inputs from a failed check of the slot w names (the first
// attempt goes straight to the election).
template <int NT>
__device__ int plan_select_slow(const DecodeArgs& a, PlanLds& L, int* tst_s, unsigned long long w,
                                bool staged = false, unsigned int give_ups = 0) {
  unsigned long long* word = plan_word(a);
  const unsigned int epoch = a.epoch;
  for (int attempt = 0; attempt < 4; ++attempt) {
    if (plan_building_here(w, epoch)) {
      if (threadIdx.x == 0) {
        unsigned long long x = w;
        for (int n = 0; n < a.plan_spin && plan_building_here(x, epoch); ++n) {
          __builtin_amdgcn_s_sleep(4);
          x = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        L.w_s = x;
      }
      __syncthreads();
      w = L.w_s;
      __syncthreads();
      if (plan_building_here(w, epoch)) return -1;
      if ((PRISM_DBG(a) & 32) && blockIdx.x == 1 && threadIdx.x == 0)  // measurement aid
        a.plan_region[kPlanBuildStamps + 4] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
      // Published by this launch's builder, from this call's inputs: use it
      // without another check.  No acquire fence (an L2 invalidate, which
      // 255 workgroups issuing at once made take 12 us): this workgroup has
      // not read the new slot in this launch, so no cache level here holds a
      // line of it from before the publication (a launch starts with its
      // caches coherent).
      if (static_cast<unsigned int>(w >> 32) == epoch) return static_cast<int>(w & 1);
    }
    const int slot = static_cast<int>(w & 1);
    // a nonzero give-up count makes the slot the word names stale whatever its key
    if (!(staged && attempt == 0) && !(give_ups != 0 && attempt == 0)) {
      const bool same = plan_key_check<NT>(a, plan_slot(a, slot), L);
      if (__syncthreads_and(same ? 1 : 0)) return slot;
    }
    if (threadIdx.x == 0) {
      // Test, then swap.  Compare-exchanges on one word serialise at the
      // memory (about 0.1 us each), so 256 of them would hold the losers for
      // tens of microseconds: workgroup 0 tries at once, every other one
      // first watches the word for up to 3 us and tries only if it is still
      // unclaimed (any running workgroup may win; none is waited for).
      unsigned long long expect = w;
      if (blockIdx.x != 0) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();  // 100 MHz
        while (expect == w && __builtin_amdgcn_s_memrealtime() - t0 < 300) {
          __builtin_amdgcn_s_sleep(8);
          expect = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      const unsigned long long mine =
          (static_cast<unsigned long long>(epoch) << 32) | kPlanBuilding | static_cast<unsigned long long>(slot);
      const bool won = expect == w && __hip_atomic_compare_exchange_strong(word, &expect, mine, __ATOMIC_RELAXED,
                                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      L.won_s = won ? 1 : 0;
      L.w_s = won ? mine : expect;
      if ((PRISM_DBG(a) & 32) && blockIdx.x == 1) {  // measurement aid: when workgroup 1 left the election
        a.plan_region[kPlanBuildStamps + 6] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
        a.plan_region[kPlanBuildStamps + 7] = won ? 2 : (expect == w ? 1 : 0);
      }
    }
    __syncthreads();
    const bool won = L.won_s != 0;
    const unsigned long long seen = L.w_s;
    __syncthreads();
    if (won) {
      int* bs = a.plan_region + kPlanBuildStamps;  // measurement aid (bit 32): the builder's phases
      auto stamp = [&](int k) {
        if ((PRISM_DBG(a) & 32) && threadIdx.x == 0)
          bs[k] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
      };
      stamp(0);
      plan_build<NT>(a, plan_slot(a, 1 - slot), L, tst_s);
      stamp(1);
      if (threadIdx.x == 0 && give_ups != 0) {
        unsigned int seen_gu = give_ups;
        __hip_atomic_compare_exchange_strong(reinterpret_cast<unsigned int*>(a.plan_region) + kPlanGiveUps, &seen_gu,
                                             0u, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // the slot reaches the device-coherent level
      __syncthreads();
      stamp(2);
      if (threadIdx.x == 0)
        __hip_atomic_store(word, (static_cast<unsigned long long>(epoch) << 32) | static_cast<unsigned long long>(1 - slot),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((PRISM_DBG(a) & 32) && threadIdx.x == 0) bs[3] = static_cast<int>(blockIdx.x);
      return 1 - slot;
    }
    w = seen;  // another workgroup builds (or the word changed): wait for it, then check again
  }
  return -1;
}

// The plan on its own (stage 3): check the key of the current slot, build
// and publish the other one when it differs.
__global__ void __launch_bounds__(kPlanThreads) paged_decode_stream_plan_kernel(const DecodeArgs a) {
  __shared__ PlanLds L;
  __shared__ int tst_s[kSMaxBatch + kSMaxVirt + 1];
  if (threadIdx.x == 0) {
    L.w_s = __hip_atomic_load(plan_word(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    L.won_s = static_cast<int>(__hip_atomic_load(reinterpret_cast<unsigned int*>(a.plan_region) + kPlanGiveUps,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  }
  __syncthreads();
  const unsigned long long w = L.w_s;
  const unsigned int give_ups = static_cast<unsigned int>(L.won_s);
  __syncthreads();
  plan_select_slow<kPlanThreads>(a, L, tst_s, w, false, give_ups);
}

// Walk parameters of stream entry i (i < V: virtual sequence i, else real
// sequence i - V): block-table row, first token, end token, and the tile at
// which a virtual sequence starts its walk (it wraps around).
template <int TPR>
__device__ __forceinline__ void stream_seq(const DecodeArgs& a, const int* plan, const int* tstart, int V, int i,
                                           int& bt_row,
                                           int& tok0, int& n_end, int& rot) {
  if (i >= V) {
    const int b = i - V;
    bt_row = b;
    tok0 = ld_meta(plan + kPlanSkip + b);
    n_end = effective_len(a, b);
    rot = 0;
  } else {
    bt_row = ld_meta(plan + kPlanVsrc + i);
    tok0 = 0;
    n_end = (tstart[i + 1] - tstart[i]) * (kSTile * TPR);
    rot = ld_meta(plan + kPlanVrot + i);
  }
}

// Query column c of wave h (kv head hk = h % Hkv) for stream entry i: real
// sequence b -> q head hk*G + c (c < G); virtual sequence -> q head hk*G + qh
// of member m, c = m*G + qh (c < vcols: the second column block passes
// c + 16).
template <int TPR>
__device__ __forceinline__ void stream_column(const DecodeArgs& a, const int* plan, int V, int i, int h_slot, int c,
                                              int& qrow,
                                              int& qhead, bool& valid) {
  const int G = a.groups;
  const int h = h_slot % (kSKv / TPR);  // kv head of the slot
  if (i >= V) {
    valid = c < G;
    qrow = i - V;
    qhead = h * G + (valid ? c : 0);
    return;
  }
  const int m = c / G;
  const int qh = c - m * G;
  const int member = (m < a.vcols / G) ? plan[kPlanVmem + i * kVMax + m] : -1;
  valid = member >= 0;
  qrow = valid ? member : 0;
  qhead = h * G + (valid ? qh : 0);
}

// Outputs of a batch of nb merged sequences from the streaming partials, by
// the whole workgroup.  A unit is (q head, 8 dims): 16 units per head.  When
// the heads fill fewer units than threads (fewer q heads than 32, as on a
// tensor-parallel rank), the threads form ng = threads / units slots of
// `units` threads and each of the batch's nb <= ng sequences takes one slot,
// so the batch's loads are in flight together.  Otherwise (nb = 1) one slot
// covers the heads in passes of 32.  A sequence's candidates are always
// summed by one slot in candidate order, so its output does not depend on
// how many sequences the completing workgroup happens to merge at once
// (splitting a sequence's candidates over the free slots made the rounding,
// and so the output bits, depend on that count, which timing decides).  The
// candidates are the (workgroup, token slot) pairs whose workgroups met b's
// own tiles or its virtual sequence's tiles (one per workgroup: with fewer kv
// heads the workgroup merged its token slots before writing); their rows
// follow the layout the streaming kernel writes (real entry e of workgroup w
// at (w + e) * 8G + slot * G + column; virtual entry v at
// vrow0 + ((w + v) * 8 + slot) * vcols + column).  A
// partial with m = -inf attended nothing and weighs 0.  Eight candidates are
// loaded per round and slot, (m, l) and 32 accumulator bytes each, with a
// running maximum across rounds; the usual sequence needs one round.  This
// code runs once per workgroup, from a cold instruction cache, so it is kept
// small: row arithmetic in 32 bits (the partial region is addressed with
// 32-bit byte offsets anyway).  `recs` holds per sequence b and its plan
// record (first, end, virtual slot, virtual first, virtual end), stride 8.
template <int QDT, int TPR>
__device__ __forceinline__ void stream_merge_batch(const DecodeArgs& a, int V, const int* recs, int nb,
                                                   const StreamSplit& sp, bool stamp = false) {
  constexpr int tl = 0;  // one partial per kv head and workgroup entry: the token slots met at the flush
  constexpr int hkv = kSKv / TPR;
  constexpr int kU = 8;
  const int units = a.num_heads * 16;
  const int ng = units >= kSThreads ? 1 : kSThreads / units;  // slots (nb <= ng)
  const int slot = ng > 1 ? static_cast<int>(threadIdx.x) / units : 0;
  const int u0 = ng > 1 ? static_cast<int>(threadIdx.x) - slot * units : static_cast<int>(threadIdx.x);
  const int kseq = min(slot, nb - 1);  // this slot's sequence in the batch
  const bool active = slot < nb;
  const int* rec = recs + 8 * kseq;
  const int b = rec[0];
  const int first = rec[1], end = rec[2], vslot = rec[3], vfirst = rec[4], vend = rec[5];
  int lo0 = 0, cnt0 = 0, lo1 = 0, cnt1 = 0;
  if (end > first) {
    lo0 = static_cast<int>(split_owner(sp, first));
    cnt0 = static_cast<int>(split_owner(sp, end - 1)) - lo0 + 1;
  }
  if (vslot >= 0) {
    lo1 = static_cast<int>(split_owner(sp, vfirst));
    cnt1 = static_cast<int>(split_owner(sp, vend - 1)) - lo1 + 1;
  }
  const int cnt = (cnt0 + cnt1) << tl;
  const int d0 = 8 * (u0 & 15);
  // with at least one tile per workgroup every range is non-empty; otherwise
  // a workgroup with an empty range wrote nothing (64-bit divisions to tell)
  const bool all_ranges = sp.total >= sp.nwg;
  // per candidate: row = base + w * stride + slot * slot_stride, where the
  // real candidates' (w from lo0) and the virtual ones' (w from lo1) differ
  const int stride0 = kSKv * a.groups, stride1 = kSKv * a.vcols;
  const int sstride0 = a.num_heads, sstride1 = hkv * kSCols;
  // whole-region resources (the partial region is far below 4 GiB)
  const __amdgpu_buffer_rsrc_t acc_r = __builtin_amdgcn_make_buffer_rsrc(a.part_acc, 0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t ml_r = __builtin_amdgcn_make_buffer_rsrc(a.part_ml, 0, 0x7FFFFFFF, 0x00020000);
  for (int u = u0; u < units; u += (ng > 1 ? units : kSThreads)) {  // one pass when ng > 1
    const int hq = u >> 4;
    const int rbase0 = (V + b) * stride0 + hq + lo0 * stride0;
    int rbase1 = 0;
    if (vslot >= 0) {
      const int v = vslot / kVMax;
      const int m = vslot - v * kVMax;
      const int hk = hq / a.groups;
      rbase1 = static_cast<int>(a.vrow0) + (v * kSKv + hk) * a.vcols + m * a.groups + (hq - hk * a.groups) +
               lo1 * stride1;
    }
    float m_run = -INFINITY, l_sum = 0.f;
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = 0.f;
    const int mine = active ? cnt : 0;
    for (int base = 0; base < mine; base += kU) {
      float mv[kU], lv[kU];
      floatx4 x0[kU], x1[kU];
#pragma unroll
      for (int k = 0; k < kU; ++k) {
        const int i = min(base + k, mine - 1);
        const int wi = i >> tl;
        const int sl = i & ((1 << tl) - 1);
        const bool second = wi >= cnt0;
        const int wk = second ? wi - cnt0 : wi;  // workgroup offset from lo0 or lo1
        const int row = (second ? rbase1 : rbase0) + wk * (second ? stride1 : stride0) +
                        sl * (second ? sstride1 : sstride0);
        bool ok = base + k < mine;
        if (!all_ranges) {
          const int64_t w = (second ? lo1 : lo0) + wk;
          ok = ok && split_begin(sp, w) < split_begin(sp, w + 1);
        }
        // only live candidates are loaded: these device-scope loads bypass
        // the caches, and re-reading a live row for every unused candidate
        // slot made a 2-candidate merge move 4x its bytes through one CU
        float2 ml = {-INFINITY, 0.f};
        x0[k] = floatx4{0.f, 0.f, 0.f, 0.f};
        x1[k] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (base + k < mine) {
          ml = load_coherent2(ml_r, static_cast<uint32_t>(row) * 8u);
          const uint32_t off = (static_cast<uint32_t>(row) * kHeadDim + d0) * 4u;
          x0[k] = load_coherent4(acc_r, off);
          x1[k] = load_coherent4(acc_r, off + 16);
        }
        mv[k] = ok ? ml.x : -INFINITY;
        lv[k] = ok ? ml.y : 0.f;
      }
      float mx = m_run;
#pragma unroll
      for (int k = 0; k < kU; ++k) mx = fmaxf(mx, mv[k]);
      if ((PRISM_DBG(a) & 32) && stamp && threadIdx.x == 0 && base == 0 && mx != 12345.f)  // measurement aid: loads back
        a.plan_region[kPlanMergeStamps + 4 * blockIdx.x + 1] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
      if (mx == -INFINITY) continue;  // nothing attended so far
      const float alpha = exp2f(m_run - mx);  // 0 while m_run = -inf
      l_sum *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] *= alpha;
#pragma unroll
      for (int k = 0; k < kU; ++k) {
        const float wgt = mv[k] == -INFINITY ? 0.f : exp2f(mv[k] - mx);  // rows with m = -inf weigh 0
        l_sum += wgt * lv[k];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[j] += wgt * (wgt != 0.f ? x0[k][j] : 0.f);
          o[4 + j] += wgt * (wgt != 0.f ? x1[k][j] : 0.f);
        }
      }
      m_run = mx;
      if ((PRISM_DBG(a) & 32) && stamp && threadIdx.x == 0 && base == 0 && o[7] != 12345.f)  // measurement aid: accumulated
        a.plan_region[kPlanMergeStamps + 4 * blockIdx.x + 2] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
    }
    if (!active) continue;
    const float inv = l_sum > 0.f ? 1.f / l_sum : 0.f;
    const int64_t obase = static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(hq) * a.o_sh;
    store_out8<QDT>(a, obase + d0 * a.o_sd, o, inv);
  }
}

// End of a streaming workgroup's range.  Every wave has written the partials
// of the stream entries [e_first, e_first + nent) it met (nent = 0: an empty
// range).  Each flush is counted on the sequences it serves (a virtual entry
// serves each of its members); the workgroup whose count completes a
// sequence merges that sequence's output and resets its counter.  Sequences
// that attend no token at all (no tiles, no flushes) get zeros from
// workgroup b % nwg.  `scratch` is LDS no longer in use (the drained stages).
template <int QDT, int TPR>
__device__ __forceinline__ void stream_finish(const DecodeArgs& a, int* plan, int V, int64_t total, const int* tstart,
                                              int e_first, int nent, int* scratch) {
  constexpr int kRec = 5;
  int* n_merge = scratch;
  int* merge_rec = scratch + 4;  // per merged sequence: b, then its 5-int plan record (stride 8)
  // this wave's partial stores have completed (device scope): the flushes may be counted
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (threadIdx.x == 0) *n_merge = 0;
  __syncthreads();
  int* cnt = plan + kPlanCnt;
  const int members = a.vcols / a.groups;
  for (int t = threadIdx.x; t < nent * kVMax; t += kSThreads) {
    const int i = e_first + t / kVMax;
    const int slot = t - (t / kVMax) * kVMax;
    if (tstart[i + 1] == tstart[i]) continue;  // no tiles: never flushed
    int seq = -1;
    if (i >= V) seq = slot == 0 ? i - V : -1;
    else if (slot < members) seq = plan[kPlanVmem + i * kVMax + slot];
    if (seq < 0) continue;
    const int4 r0 = *reinterpret_cast<const int4*>(plan + kPlanRec + 8 * seq);
    const int2 r1 = *reinterpret_cast<const int2*>(plan + kPlanRec + 8 * seq + 4);  // virtual end, expected
    const int prev = __hip_atomic_fetch_add(cnt + seq, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev + 1 == r1.y) {
      __hip_atomic_store(cnt + seq, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int* e = merge_rec + 8 * atomicAdd(n_merge, 1);
      e[0] = seq;
      e[1] = r0.x;
      e[2] = r0.y;
      e[3] = r0.z;
      e[4] = r0.w;
      e[5] = r1.x;
    }
  }
  // zeros for sequences without a single partial
  for (int b = blockIdx.x; b < a.batch; b += a.stream_nwg) {
    if (plan[kPlanRec + 8 * b + 5] != 0) continue;  // uniform
    for (int e = threadIdx.x; e < a.num_heads * kHeadDim; e += kSThreads) {
      const int hq = e / kHeadDim;
      const int d = e - hq * kHeadDim;
      store_out<QDT>(a.out, static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(hq) * a.o_sh + d * a.o_sd, 0.f);
    }
  }
  __syncthreads();
  const int nm = *n_merge;
  if ((PRISM_DBG(a) & 32) && threadIdx.x == 0) {  // measurement aid: merges, counted
    int* d = a.plan_region + kPlanMeasure + 8 * blockIdx.x;
    d[3] = nm;
    d[4] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
  }
  if (nm == 0) return;
  const StreamSplit sp = stream_split(a, total);  // (not re-read: a round trip on the kernel's tail)
  // merges in batches: as many at once as the workgroup has slots (one at a
  // time when the q heads fill the workgroup)
  const int units = a.num_heads * 16;
  const int slots = units >= kSThreads ? 1 : kSThreads / units;
  for (int k = 0; k < nm; k += slots) {
    if ((PRISM_DBG(a) & 32) && k == 0 && threadIdx.x == 0)  // measurement aid: first batch starts
      a.plan_region[kPlanMergeStamps + 4 * blockIdx.x] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
    stream_merge_batch<QDT, TPR>(a, V, merge_rec + 8 * k, min(slots, nm - k), sp, k == 0);
    if ((PRISM_DBG(a) & 32) && k == 0 && threadIdx.x == 0) {  // measurement aid: first batch done
      int* d = a.plan_region + kPlanMeasure + 8 * blockIdx.x;
      d[6] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
    }
  }
  static_assert(kRec + 1 <= 8, "merge record stride");
}

// A workgroup that waited for a plan build past the poll limit (the builder
// never published: not expected, since the builder waits for nobody) leaves
// the launch without its tiles.  The sequences it served never complete, so
// their output rows would keep stale values: it writes NaN to every output
// row instead (rows that other workgroups complete may overwrite it with
// their result), and counts the give-up in the plan header, which makes the
// next launch rebuild the plan and zero the completion counters this launch
// left part-way.
template <int QDT>
__device__ __forceinline__ void stream_give_up(const DecodeArgs& a) {
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(reinterpret_cast<unsigned int*>(a.plan_region) + kPlanGiveUps, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  const int64_t per_row = static_cast<int64_t>(a.num_heads) * kHeadDim;
  const int64_t n = static_cast<int64_t>(a.batch) * per_row;
  for (int64_t base = 0; base < n; base += kSThreads) {  // uniform trip count
    const int64_t e = base + threadIdx.x;
    const int64_t b = e / per_row;
    const int64_t r = e - b * per_row;
    const int64_t hq = r / kHeadDim;
    const int64_t d = r - hq * kHeadDim;
    if (e < n) store_out<QDT>(a.out, b * a.o_sb + hq * a.o_sh + d * a.o_sd, __builtin_nanf(""));
  }
}

// kSWgPerCu 8-wave workgroups per CU need 2 * kSWgPerCu waves per SIMD.
template <int QDT, bool QVEC, int TPR, bool C16>
__global__ void __launch_bounds__(kSThreads) __attribute__((amdgpu_waves_per_eu(2 * kSWgPerCu)))
paged_decode_stream_kernel(const DecodeArgs a) {
  static_assert(!C16 || (TPR == 1 && QDT != PRISM_DTYPE_F32), "16-bit tiles: 8 kv heads, 16-bit queries");
  constexpr int kTTok = kSTile * TPR;  // tokens per tile
  // stage geometry: FP8 tiles (K, V, scales; four stages) or 16-bit tiles (K, V; two stages)
  constexpr int kStg = C16 ? kS16Stages : kSStages;
  constexpr int kStgBytes = C16 ? kS16Stage : kSStage;
  constexpr int kRowB = C16 ? kS16Row : kSRow;
  constexpr int kTileKB = C16 ? kS16KBytes : kSKBytes;
  __shared__ __attribute__((aligned(256))) uint8_t stages[kSStages * kSStage];
  __shared__ int tstart[kSMaxBatch + kSMaxVirt + 1];
  static_assert(sizeof(PlanLds) <= sizeof(stages), "the plan's LDS lies over the idle stages");
  const int lane = threadIdx.x & 63;
  const int h = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // head slot of this wave (uniform)
  const int g = lane >> 4;
  const int c = lane & 15;
  const int B = a.batch;
  const uint64_t r_entry = (PRISM_DBG(a) & 32) ? __builtin_amdgcn_s_memrealtime() : 0;

  // ---- the plan.  First load: the plan word.  Then, together: from the slot it names,
  // this workgroup's start record, the plan header, the tile prefix sums
  // (virtual sequences, then real ones; copied up to the largest possible
  // entry count, so that these loads need not wait for V) and the key, which
  // is compared with this call's inputs.  When they differ, the plan is
  // (re)built by one workgroup of the launch while the others wait, and the
  // same loads are repeated on the new slot.
  PlanLds& L = *reinterpret_cast<PlanLds*>(stages);
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t hdr = *reinterpret_cast<const __attribute__((address_space(4))) u32x4_t*>(
      reinterpret_cast<uintptr_t>(a.plan_region));
  const unsigned long long w0 = static_cast<unsigned long long>(hdr.x) | (static_cast<unsigned long long>(hdr.y) << 32);
  const unsigned int give_ups = hdr.z;  // plan header int kPlanGiveUps
  int* plan = plan_slot(a, __builtin_amdgcn_readfirstlane(static_cast<int>(w0 & 1)));
  auto prologue_stamp = [&](int k, unsigned long long dep) {  // measurement aid (bit 32)
    if ((PRISM_DBG(a) & 32) && threadIdx.x == 0)
      a.plan_region[kPlanPrologueStamps + 4 * blockIdx.x + k] =
          static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF) + (dep == 0x1234567ull ? 1 : 0);
  };
  prologue_stamp(0, w0);
  // prefix sums go to registers first and to LDS after the key check, so the
  // check's loads leave in the same round
  constexpr int kTs = (kSMaxBatch + kSMaxVirt + 1 + kSThreads - 1) / kSThreads;
  int4 wr0, wr1;
  int tsv[kTs];
  int V;
  int64_t total;
  auto load_plan = [&]() {
    wr0 = *reinterpret_cast<const int4*>(plan + kPlanWgRec + 8 * blockIdx.x);
    wr1 = *reinterpret_cast<const int4*>(plan + kPlanWgRec + 8 * blockIdx.x + 4);
#pragma unroll
    for (int t = 0; t < kTs; ++t) {
      const int i = threadIdx.x + t * kSThreads;
      tsv[t] = i <= B + kSMaxVirt ? plan[kPlanTstart + i] : 0;
    }
    V = ld_meta(plan);
    total = ld_meta(plan + 1);
  };
  auto store_tstart = [&]() {
#pragma unroll
    for (int t = 0; t < kTs; ++t) {
      const int i = threadIdx.x + t * kSThreads;
      if (i <= B + kSMaxVirt) tstart[i] = tsv[t];
    }
  };
  load_plan();
  const bool same =
      (PRISM_DBG(a) & 128) ? true
                           : (!plan_building_here(w0, a.epoch) && plan_key_check<kSThreads>(a, plan, L) && give_ups == 0);
  prologue_stamp(1, same ? 1 : 0);
  store_tstart();
  const bool all_same = __syncthreads_and(same ? 1 : 0);
  prologue_stamp(2, all_same ? 1 : 0);
  if (__builtin_expect(!all_same, 0)) {
    const bool staged = !(PRISM_DBG(a) & 128) && !plan_building_here(w0, a.epoch);  // the check above staged L
    const int slot =
        __builtin_amdgcn_readfirstlane(plan_select_slow<kSThreads>(a, L, tstart, w0, staged, give_ups));
    if (slot < 0) {
      stream_give_up<QDT>(a);
      return;
    }
    plan = plan_slot(a, slot);
    __syncthreads();  // every thread is done with the build's tstart before it is reloaded
    load_plan();
    store_tstart();
    __syncthreads();
  }
  const int NS = B + V;
  const int count = __builtin_amdgcn_readfirstlane(wr0.x) < 0 ? 0 : __builtin_amdgcn_readfirstlane(wr0.z);
  __syncthreads();
  if (count == 0) {  // uniform: an empty range flushes nothing
    stream_finish<QDT, TPR>(a, plan, V, total, tstart, 0, 0, reinterpret_cast<int*>(stages));
    return;
  }
  const uint64_t t_begin = __builtin_amdgcn_s_memrealtime();

  const StreamLanePlan pl = stream_plan(h, lane);
  const StreamLanePlan16 pl16 = stream_plan16(h, lane);
  const uint32_t stage0 = lds_addr(stages);
  const int P = a.page_size;
  const int tpp = P / kTTok;  // tiles per page (the streaming shape has P % kTTok == 0)
  // unit-scale FP8 caches (no scale tensors): every stage still issues its
  // fifth load per lane -- the loop's waits count five -- from the tile's own
  // K bytes (valid memory, a cache hit), and the scales read as 1
  const bool unscaled = a.ks == nullptr;
  const float* sbase = pl.which ? a.vs : a.ks;  // wave-uniform: the scales this wave's lanes load

  // ---- issue side: walks this workgroup's tiles kSStages - 1 ahead of the
  // compute side.  Per stream entry: physical tile pt of ntl (virtual walks
  // start at a rotation and wrap), tile-in-page tip, and the scalar addresses
  // of the tile's K, V and scale rows, advanced by constants; the block id
  // is read only when the page changes.  Per stage it records for the
  // compute side how many of the tile's tokens are attended (0: the block id
  // is invalid, skip the tile).
  int ie = __builtin_amdgcn_readfirstlane(wr0.x);
  int ileft, intl, ipt, itip, ipage, ipage0, irow, it0, itok0, iend;
  const uint8_t* ikb;
  const uint8_t* ivb;
  const float* isb;
  bool ivalid;
  bool iprivate;          // the entry is a real sequence: its pages stream past the caches
  uint32_t stage_nv = 0;  // byte s: attended tokens of the tile in stage s
  auto ipage_set = [&](int raw_or_load) {
    // raw_or_load: a block id already known, or kNoBlock to read it
    int raw = raw_or_load;
    if (raw == kNoBlock)
      raw = ld_meta(a.bt + static_cast<int64_t>(irow) * a.bt_sb + static_cast<int64_t>(ipage) * a.bt_sn);
    ivalid = raw >= 0 && raw < a.num_blocks;
    const int64_t blk = ivalid ? raw : 0;  // loads of an invalid block read page 0 and are skipped
    const int64_t tip_rows = static_cast<int64_t>(itip) * kSTile;
    ikb = a.k + blk * a.k_sblk + tip_rows * kRowB;
    ivb = a.v + blk * a.v_sblk + tip_rows * kRowB;
    isb = unscaled ? reinterpret_cast<const float*>(ikb) : sbase + blk * a.ks_sblk + tip_rows * kSKv;
  };
  auto ientry = [&](int lt, int first_raw) {
    intl = __builtin_amdgcn_readfirstlane(tstart[ie + 1] - tstart[ie]);
    int rot;
    stream_seq<TPR>(a, plan, tstart, V, ie, irow, itok0, iend, rot);
    irow = __builtin_amdgcn_readfirstlane(irow);
    itok0 = __builtin_amdgcn_readfirstlane(itok0);
    iend = __builtin_amdgcn_readfirstlane(iend);
    rot = __builtin_amdgcn_readfirstlane(rot);
    ileft = intl - lt;
    ipt = lt + rot;
    if (ipt >= intl) ipt -= intl;
    it0 = itok0 + ipt * kTTok;
    ipage = it0 / P;
    itip = (it0 - ipage * P) / kTTok;
    ipage0 = itok0 / P;
    iprivate = ie >= V && !(PRISM_DBG(a) & 16);
    ipage_set(first_raw);
  };
  ientry(__builtin_amdgcn_readfirstlane(wr0.y), __builtin_amdgcn_readfirstlane(wr1.w));
  int issued = 0;
  int istage = 0;
  auto issue_next = [&]() {
    const int nv = ivalid ? min(iend - it0, kTTok) : 0;
    stage_nv = (stage_nv & ~(0xFFu << (8 * istage))) | (static_cast<uint32_t>(nv) << (8 * istage));
    if (!(PRISM_DBG(a) & 2)) {
      if constexpr (C16) stream_issue16(pl16, ikb, ivb, stage0 + static_cast<uint32_t>(istage) * kStgBytes, iprivate);
      else stream_issue(pl, ikb, ivb, isb, stage0 + static_cast<uint32_t>(istage) * kStgBytes, iprivate);
    }
    ++issued;
    istage = istage == kStg - 1 ? 0 : istage + 1;
    if (issued == count) return;  // the range is done (no page past it is read)
    if (--ileft == 0) {  // the entry is done: the next one with tiles
      do {
        ++ie;
      } while (tstart[ie + 1] == tstart[ie] && ie + 1 < NS);
      ie = __builtin_amdgcn_readfirstlane(ie);
      ientry(0, kNoBlock);
      return;
    }
    ++ipt;
    it0 += kTTok;
    ++itip;
    ikb += kTileKB;
    ivb += kTileKB;
    isb += kSTile * kSKv;
    if (ipt == intl) {  // a rotated walk wraps to the entry's first tile
      ipt = 0;
      it0 = itok0;
      ipage = ipage0;
      itip = 0;
      ipage_set(kNoBlock);
    } else if (itip == tpp) {
      ++ipage;
      itip = 0;
      ipage_set(kNoBlock);
    }
  };
#pragma unroll
  for (int i = 0; i < kStg - 1; ++i)
    if (issued < count) issue_next();

  // ---- compute side: entry b, tiles left in it for this workgroup
  int b = __builtin_amdgcn_readfirstlane(wr0.x);
  int cleft = min(__builtin_amdgcn_readfirstlane(tstart[b + 1] - tstart[b]) - __builtin_amdgcn_readfirstlane(wr0.y),
                  count);
  using QOp = typename std::conditional<C16, QOperand16, QOperandF8>::type;
  // Wide virtual sequences (8 kv heads: FP8 or 16-bit tiles): a virtual
  // entry has two blocks of 16 query columns (twice the members per walk of
  // the shared pages); both read the same K and V of each tile from LDS.
  constexpr bool kWide = TPR == 1;
  const bool wide_call = kWide && a.vcols > kSCols;
  QOp qop;
  QOp qop2;  // second column block (wide virtual entries)
  bool colv, colv2;
  bool wide = false;  // the compute side's entry is a wide virtual one (wave-uniform)
  auto load_query = [&]() {
    int qrow, qhead;
    stream_column<TPR>(a, plan, V, b, h, c, qrow, qhead, colv);
    if constexpr (C16) stream_load_q16<QDT, QVEC>(a, qrow, qhead, colv, g, qop);
    else stream_load_q8<QDT, QVEC>(a, qrow, qhead, colv, g, qop);
    wide = wide_call && b < V;
    if constexpr (kWide) {
      if (wide) {
        stream_column<TPR>(a, plan, V, b, h, c + kSCols, qrow, qhead, colv2);
        if constexpr (C16) stream_load_q16<QDT, QVEC>(a, qrow, qhead, colv2, g, qop2);
        else stream_load_q8<QDT, QVEC>(a, qrow, qhead, colv2, g, qop2);
      }
    }
  };
  load_query();

  floatx4 acc[8], acc2[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, m_run2 = -INFINITY;  // running max (log2 domain) of query column c (16 + c)
  float l_run = 0.f, l_run2 = 0.f;              // this lane's share of the running sum

  // Per-lane LDS addresses inside stage 0 (loop invariant).
  const uint32_t k_off0 = stage0 + c * kSRow + stream_slot(h, c) * kHeadDim + (((2 * g) ^ stream_swz(c)) << 4);
  const uint32_t k_off1 = stage0 + c * kSRow + stream_slot(h, c) * kHeadDim + (((2 * g + 1) ^ stream_swz(c)) << 4);
  const uint32_t s_off = stage0 + 2 * kSKBytes + (h * kSTile + 4 * g) * 4;
  uint32_t v_off[4];
  {
    const int r = c >> 1;              // row of the 8x16 byte matrix this lane addresses
    const int t = 4 * g + (r & 3);     // token
    const int half = c & 1;
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const int chunk = 2 * jp + (r >> 2);
      v_off[jp] = stage0 + kSKBytes + t * kSRow + stream_slot(h, t) * kHeadDim + ((chunk ^ stream_swz(t)) << 4) +
                  half * 8;
    }
  }
  // first token this lane's score rows refer to, relative to the tile:
  // row 4g + i of this wave's slot is token TPR * (4g + i) + h / Hkv
  const int tok_lane = TPR * 4 * g + h / (kSKv / TPR);
  // 16-bit tiles: K chunks 4g + kb of token c; V for N-tile nt: token
  // 4g + (c >> 2), 8 bytes at 32 nt + 8 (c & 3) of the head slot (the b64_tr_b16
  // read then hands lane (g, n) dims 16 nt + n of tokens 4g .. 4g + 3)
  uint32_t k16_off[4], v16_off[8];
  if constexpr (C16) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      k16_off[kb] = stage0 + c * kS16Row + h * (2 * kHeadDim) + (((4 * g + kb) ^ stream_swz16(c)) << 4);
    const int t = 4 * g + (c >> 2);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      const int byte = 32 * nt + 8 * (c & 3);
      v16_off[nt] = stage0 + kS16KBytes + t * kS16Row + h * (2 * kHeadDim) + (((byte >> 4) ^ stream_swz16(t)) << 4) +
                    (byte & 15);
    }
  }

  int cstage = 0;
  // measurement aid (bit 64): cycles per section of the loop, per wave
  uint64_t xs[4] = {0, 0, 0, 0};
  uint64_t xs_t = (PRISM_DBG(a) & 64) ? __builtin_amdgcn_s_memtime() : 0;
  auto xs_mark = [&](int k) {
    if (PRISM_DBG(a) & 64) {
      const uint64_t n = __builtin_amdgcn_s_memtime();
      xs[k] += n - xs_t;
      xs_t = n;
    }
  };
  for (int done = 0; done < count; ++done) {
    // Wait for this tile's loads (the younger tiles' loads may stay in flight),
    // then one barrier: every wave's loads have landed and every wave has
    // finished the previous tile, whose stage the refill below reuses.  At
    // this wait the tiles issued are those before done + kStg - 1 (the
    // prologue issued kStg - 1, each earlier iteration one more after its
    // barrier), so min(kStg - 2, count - done - 1) younger tiles may be in
    // flight: two for FP8 tiles, none for 16-bit tiles.  Vector-memory
    // operations the compiler issued after this tile's loads (partial
    // stores, query loads) are younger still, so the count can only
    // over-wait for them.
    static_assert(kSStages == 4 && kS16Stages == 2, "wait counts below assume four (16-bit: two) stages");
    if constexpr (C16) {
      __builtin_amdgcn_s_waitcnt(0xF70);
    } else if (done + 2 < count) {  // steady state: two younger tiles in flight
      __builtin_amdgcn_s_waitcnt(0xF70 | (2 * kSLoadsPerStage));
    } else if (done + 1 < count) {
      __builtin_amdgcn_s_waitcnt(0xF70 | (1 * kSLoadsPerStage));
    } else {
      __builtin_amdgcn_s_waitcnt(0xF70);
    }
    stream_barrier();
    xs_mark(0);
    const int nv = __builtin_amdgcn_readfirstlane((stage_nv >> (8 * cstage)) & 0xFF);
    if (issued < count) issue_next();
    xs_mark(1);

    if constexpr (C16) {
      if (nv != 0 && !(PRISM_DBG(a) & 1)) {
        const uint32_t slot = static_cast<uint32_t>(cstage) * kS16Stage;
        // ---- all LDS reads of the tile first
        u32x4 kw[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) kw[kb] = lds_load_b128(k16_off[kb] + slot);
        uint64_t vt[8];
        lds_read_tr16_x8(v16_off, slot, vt);
        // ---- QK over 16 tokens: the K rows are the MFMA's A operand as they
        // are (row = token c, k = dims 32g + 8kb ..), the query the B operand.
        // Only a sequence's last tile can reach past its end: masked tokens
        // get score -inf and zero V elements (rows past the end may hold NaN).
        const bool partial = nv < kTTok;
        bool tv[4] = {true, true, true, true};
        if (partial) {
          uint64_t keep = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            tv[i] = tok_lane + i < nv;
            keep |= tv[i] ? (uint64_t{0xFFFF} << (16 * i)) : 0;
          }
#pragma unroll
          for (int nt = 0; nt < 8; ++nt) vt[nt] &= keep;
        }
        // one block of 16 query columns: scores, online softmax, PV
        auto column_block16 = [&](const QOperand16& qo, floatx4 (&ac)[8], float& mr, float& lr) {
          floatx4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            if constexpr (QDT == PRISM_DTYPE_BF16)
              sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kw[kb]),
                                                           __builtin_bit_cast(bf16x8, qo.t[kb]), sc, 0, 0, 0);
            else
              sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, kw[kb]),
                                                          __builtin_bit_cast(f16x8, qo.t[kb]), sc, 0, 0, 0);
          }
          float x[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x[i] = sc[i] * qo.colscale;
            if (partial) x[i] = tv[i] ? x[i] : -INFINITY;
          }
          float tmax = nan_max(nan_max(x[0], x[1]), nan_max(x[2], x[3]));
          tmax = wave_maximum_across_groups(tmax);
          const bool raise = tmax > mr + kSRescaleThreshold;
          if (__builtin_amdgcn_ballot_w64(raise) != 0) {  // wave-uniform branch
            const float m_new = raise ? tmax : mr;
            const float alpha = raise ? __builtin_amdgcn_exp2f(mr - m_new) : 1.f;
            mr = m_new;
            lr *= alpha;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float ai = __shfl(alpha, 4 * g + i);
#pragma unroll
              for (int j = 0; j < 8; ++j) ac[j][i] *= ai;
            }
          }
          const float m_use = (mr == -INFINITY) ? 0.f : mr;
          float pv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pv[i] = __builtin_amdgcn_exp2f(x[i] - m_use);  // 0 for masked tokens
            lr += pv[i];
          }
          // ---- PV: P (A operand, k = tokens 4g .. 4g + 3) in the cache's
          // 16-bit type, V N-tile nt from the transposed read (B operand)
          if constexpr (QDT == PRISM_DTYPE_BF16) {
            const shortx4 pa = {__builtin_bit_cast(short, static_cast<__bf16>(pv[0])),
                                __builtin_bit_cast(short, static_cast<__bf16>(pv[1])),
                                __builtin_bit_cast(short, static_cast<__bf16>(pv[2])),
                                __builtin_bit_cast(short, static_cast<__bf16>(pv[3]))};
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
              ac[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, __builtin_bit_cast(shortx4, vt[nt]), ac[nt], 0,
                                                                 0, 0);
          } else {
            const f16x4 pa = {static_cast<_Float16>(pv[0]), static_cast<_Float16>(pv[1]),
                              static_cast<_Float16>(pv[2]), static_cast<_Float16>(pv[3])};
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
              ac[nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(f16x4, vt[nt]), ac[nt], 0, 0, 0);
          }
        };
        column_block16(qop, acc, m_run, l_run);
        if (wide) column_block16(qop2, acc2, m_run2, l_run2);
      }
    } else if (nv != 0 && !(PRISM_DBG(a) & 1)) {
      const uint32_t slot = static_cast<uint32_t>(cstage) * kSStage;
      // ---- all LDS reads of the tile first, so their latencies overlap
      const u32x4 k0 = lds_load_b128(k_off0 + slot);
      const u32x4 k1 = lds_load_b128(k_off1 + slot);
      floatx4 ks = lds_load_f4(s_off + slot);
      floatx4 vs = lds_load_f4(s_off + slot + kSScaleBytes);
      if (unscaled) {  // uniform
        ks = floatx4{1.f, 1.f, 1.f, 1.f};
        vs = floatx4{1.f, 1.f, 1.f, 1.f};
      }
      uint32_t ad[4];
#pragma unroll
      for (int jp = 0; jp < 4; ++jp) ad[jp] = v_off[jp] + slot;
      uint64_t vt[4];
      lds_read_tr8_x4(ad, vt);
      // ---- QK over 16 tokens: the K bytes are the fp8 MFMA's A operand as
      // they are (row = token c, k = dims 32g..32g+31); smallest term first.
      const i32x8 ka = {static_cast<int>(k0[0]), static_cast<int>(k0[1]), static_cast<int>(k0[2]),
                        static_cast<int>(k0[3]), static_cast<int>(k1[0]), static_cast<int>(k1[1]),
                        static_cast<int>(k1[2]), static_cast<int>(k1[3])};
      // Only a sequence's last tile can reach past its end (uniform branch).
      // Masked slots get score -inf (weight 0) and v scale 0, and their V
      // bytes are zeroed: rows past the end may hold anything, and the MFMA
      // would turn 0 * NaN into NaN.
      float vsm[4];
      bool tv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        tv[i] = true;
        vsm[i] = vs[i];
      }
      const bool partial = nv < kTTok;
      if (partial) {
        uint32_t keep = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          tv[i] = tok_lane + TPR * i < nv;
          vsm[i] = tv[i] ? vsm[i] : 0.f;
          keep |= tv[i] ? (0xFFu << (8 * i)) : 0u;
        }
        const uint64_t keep2 = static_cast<uint64_t>(keep) | (static_cast<uint64_t>(keep) << 32);
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) vt[jp] &= keep2;
      }
      // V's E4M3FN bytes as bf16 (exact): one transposed read feeds N-tiles
      // 2jp and 2jp+1 of every column block
      shortx4 vb[8];
#pragma unroll
      for (int jp = 0; jp < 4; ++jp) {
        vb[2 * jp] = fp8x4_to_bf16x4_bits(static_cast<uint32_t>(vt[jp]));
        vb[2 * jp + 1] = fp8x4_to_bf16x4_bits(static_cast<uint32_t>(vt[jp] >> 32));
      }
      // One block of 16 query columns: scores, online softmax with lazy
      // rescaling, PV.
      auto column_block = [&](const QOperandF8& qo, floatx4 (&ac)[8], float& mr, float& lr) {
        floatx4 sc = {0.f, 0.f, 0.f, 0.f};
        // (a bf16 query's third term is zero: two terms hold every bf16 value
        // the fp8 grid can, and the third only refines f16/f32 queries)
        if constexpr (QDT != PRISM_DTYPE_BF16)
          sc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qo.t[2], sc, 0, 0, 0, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qo.t[1], sc, 0, 0, 0, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qo.t[0], sc, 0, 0, 0, 0, 0, 0);
        // ---- scores in the log2 domain.  Query columns without a query hold
        // q = 0, so their scores are finite and their rows are never written.
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[i] = sc[i] * (ks[i] * qo.colscale);
          if (partial) x[i] = tv[i] ? x[i] : -INFINITY;
        }
        // (IEEE maximum: no canonicalising of masked or swapped values)
        float tmax = nan_max(nan_max(x[0], x[1]), nan_max(x[2], x[3]));
        tmax = wave_maximum_across_groups(tmax);
        const bool raise = tmax > mr + kSRescaleThreshold;
        if (__builtin_amdgcn_ballot_w64(raise) != 0) {  // wave-uniform branch
          const float m_new = raise ? tmax : mr;
          const float alpha = raise ? __builtin_amdgcn_exp2f(mr - m_new) : 1.f;
          mr = m_new;
          lr *= alpha;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int j = 0; j < 8; ++j) ac[j][i] *= ai;
          }
        }
        const float m_use = (mr == -INFINITY) ? 0.f : mr;
        // v_exp_f32 directly: arguments are at most 2^3 above the running max,
        // and results below 2^-126 (flushed to 0) weigh nothing next to it.
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(x[i] - m_use);  // 0 for masked slots
          lr += p;
          pv[i] = p * vsm[i];
        }
        const shortx4 pa = {__builtin_bit_cast(short, static_cast<__bf16>(pv[0])),
                            __builtin_bit_cast(short, static_cast<__bf16>(pv[1])),
                            __builtin_bit_cast(short, static_cast<__bf16>(pv[2])),
                            __builtin_bit_cast(short, static_cast<__bf16>(pv[3]))};
#pragma unroll
        for (int n = 0; n < 8; ++n) ac[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb[n], ac[n], 0, 0, 0);
      };
      column_block(qop, acc, m_run, l_run);
      if constexpr (kWide) {
        if (wide) column_block(qop2, acc2, m_run2, l_run2);
      }
    }
    const int cdone = cstage;  // the stage just consumed (refilled only after the next barrier)
    cstage = cstage == kStg - 1 ? 0 : cstage + 1;
    xs_mark(2);

    // ---- flush at the end of a stream entry (or of this workgroup's range)
    if (--cleft == 0 || done + 1 == count) {
      const bool more = done + 1 < count;
      float l_tot = l_run + __shfl_xor(l_run, 16);
      l_tot += __shfl_xor(l_tot, 32);
      if constexpr (TPR > 1) {
        // With fewer kv heads a row holds TPR tokens per head and the waves
        // h, h + Hkv, ... hold token slots of the same kv head: their states
        // meet in LDS and one partial per kv head and entry is written.
        // * The range's last flush: no load is in flight, so every stage is
        //   free and all eight states fit at once; after one barrier wave
        //   (sub, hk) combines the TPR slots of kv head hk for its 8 / TPR of
        //   the accumulator chunks and writes them.
        // * Earlier flushes (the younger tiles' loads stay in flight): a tree
        //   of log2 TPR levels in the stage just consumed, which no load
        //   refills before the next barrier; LDS-only barriers; the head
        //   slots below Hkv then write the merged state.
        constexpr int kHk = kSKv / TPR;
        // One wave's state: its 64 lanes' accumulators as rows of eight
        // 16-byte chunks (chunk j = acc[j], XOR-swizzled by lane so that eight
        // consecutive lanes hit distinct banks), then the 16 columns' running
        // max and sum.  Writer and reader lanes of the same (g, c) meet, so
        // each side moves its 32 values with eight b128 accesses.
        constexpr int kAccFloats = 64 * 8 * 4;
        constexpr int kState = kAccFloats + 2 * kSCols;  // floats of one wave's state
        static_assert(kSKv / 2 * kState * 4 <= kSStage, "half the waves' states fit one stage");
        static_assert(kSKv * kState * 4 <= kSStages * kSStage, "all the waves' states fit the stages");
        float* buf = reinterpret_cast<float*>(stages + cdone * kSStage);
        const int sub = h / kHk;
        const int hk = h - sub * kHk;
        const int swz = lane & 7;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        stream_barrier();  // every wave is done reading the stage
        if (!more) {
          float* mine = reinterpret_cast<float*>(stages) + h * kState;
          floatx4* rowp = reinterpret_cast<floatx4*>(mine) + lane * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j) rowp[j ^ swz] = acc[j];
          if (g == 0) {
            mine[kAccFloats + c] = m_run;
            mine[kAccFloats + kSCols + c] = l_tot;
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          stream_barrier();
          // slot s of kv head hk is wave s * kHk + hk; this lane's columns
          // are 4g .. 4g + 3, its dims c + 16 j for the chunks j it combines
          constexpr int kJ = 8 / TPR;
          floatx4 ms[TPR], ls[TPR];
#pragma unroll
          for (int sl = 0; sl < TPR; ++sl) {
            const float* st = reinterpret_cast<const float*>(stages) + (sl * kHk + hk) * kState;
            ms[sl] = *reinterpret_cast<const floatx4*>(st + kAccFloats + 4 * g);
            ls[sl] = *reinterpret_cast<const floatx4*>(st + kAccFloats + kSCols + 4 * g);
          }
          floatx4 mx = ms[0];
#pragma unroll
          for (int sl = 1; sl < TPR; ++sl)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx[i] = fmaxf(mx[i], ms[sl][i]);
          floatx4 wt[TPR];
          floatx4 lsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float mu = mx[i] == -INFINITY ? 0.f : mx[i];
#pragma unroll
            for (int sl = 0; sl < TPR; ++sl) {
              // (v_exp_f32: the largest slot weighs exp2(0) = 1, and a weight
              // flushed below 2^-126 is nothing next to it)
              wt[sl][i] = __builtin_amdgcn_exp2f(ms[sl][i] - mu);
              lsum[i] += wt[sl][i] * ls[sl][i];
            }
          }
          const bool virt = b < V;
          const int ncols = virt ? kSCols : a.groups;
          const int64_t row0 = virt ? a.vrow0 + ((static_cast<int64_t>(blockIdx.x) + b) * kSKv + hk) * a.vcols
                                    : (static_cast<int64_t>(blockIdx.x) + b) * (kSKv * a.groups) + hk * a.groups;
#pragma unroll
          for (int jj = 0; jj < kJ; ++jj) {
            const int j = sub * kJ + jj;
            floatx4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sl = 0; sl < TPR; ++sl) {
              const floatx4 x = reinterpret_cast<const floatx4*>(stages)[((sl * kHk + hk) * kState) / 4 + lane * 8 +
                                                                         (j ^ swz)];
#pragma unroll
              for (int i = 0; i < 4; ++i) o[i] += wt[sl][i] * x[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int qr = 4 * g + i;
              if (qr < ncols) store_coherent(a.part_acc + (row0 + qr) * kHeadDim + c + 16 * j, o[i]);
            }
          }
          if (sub == 0 && c == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int qr = 4 * g + i;
              if (qr < ncols) {
                store_coherent(a.part_ml + (row0 + qr) * 2 + 0, mx[i]);
                store_coherent(a.part_ml + (row0 + qr) * 2 + 1, lsum[i]);
              }
            }
          }
        } else {
#pragma unroll
          for (int span = TPR / 2; span >= 1; span /= 2) {
            if (sub >= span && sub < 2 * span) {
              float* st = buf + ((sub - span) * kHk + hk) * kState;
              floatx4* rowp = reinterpret_cast<floatx4*>(st) + lane * 8;
#pragma unroll
              for (int j = 0; j < 8; ++j) rowp[j ^ swz] = acc[j];
              if (g == 0) {
                st[kAccFloats + c] = m_run;
                st[kAccFloats + kSCols + c] = l_tot;
              }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            stream_barrier();
            if (sub < span) {
              const float* st = buf + (sub * kHk + hk) * kState;
              const floatx4* rowp = reinterpret_cast<const floatx4*>(st) + lane * 8;
              floatx4 other[8];
#pragma unroll
              for (int j = 0; j < 8; ++j) other[j] = rowp[j ^ swz];
              const float pm = st[kAccFloats + c];
              const float pl = st[kAccFloats + kSCols + c];
              // (v_exp_f32: one weight of each pair is exp2(0) = 1, and a
              // weight flushed below 2^-126 is nothing next to it)
              const float mx = fmaxf(m_run, pm);
              const float mu = mx == -INFINITY ? 0.f : mx;
              l_tot = l_tot * __builtin_amdgcn_exp2f(m_run - mu) + pl * __builtin_amdgcn_exp2f(pm - mu);
              float ao[4], ap[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int qr = 4 * g + i;
                const float mo = __shfl(m_run, qr);
                const float mp = st[kAccFloats + qr];
                const float mxi = fmaxf(mo, mp);
                const float mui = mxi == -INFINITY ? 0.f : mxi;
                ao[i] = __builtin_amdgcn_exp2f(mo - mui);
                ap[i] = __builtin_amdgcn_exp2f(mp - mui);
              }
#pragma unroll
              for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] = acc[j][i] * ao[i] + other[j][i] * ap[i];
              m_run = mx;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            stream_barrier();  // the next level reuses the buffer
          }
        }
      }
      // partial rows: real entry b at (wg + b) * 8G + slot * G + column; virtual entry v
      // at vrow0 + ((wg + v) * 8 + h) * 16 + column (head slots below Hkv only)
      const bool virt = b < V;
      const int ncols = virt ? kSCols : a.groups;
      const int64_t row0 = virt ? a.vrow0 + ((static_cast<int64_t>(blockIdx.x) + b) * kSKv + h) * a.vcols
                                : (static_cast<int64_t>(blockIdx.x) + b) * (kSKv * a.groups) + h * a.groups;
      // one column block's rows: column qr at row rb + qr
      auto flush_block = [&](const floatx4 (&ac)[8], float mr, float lt, int64_t rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int qr = 4 * g + i;
          const float li = __shfl(lt, qr);
          const float mi = __shfl(mr, qr);
          if (qr < ncols && h < kSKv / TPR) {
            const int64_t row = rb + qr;
            float* dst = a.part_acc + row * kHeadDim + c;
#pragma unroll
            for (int j = 0; j < 8; ++j) store_coherent(dst + 16 * j, ac[j][i]);
            if (c == 0) {
              store_coherent(a.part_ml + row * 2 + 0, mi);
              store_coherent(a.part_ml + row * 2 + 1, li);
            }
          }
        }
      };
      if (TPR == 1 || more) flush_block(acc, m_run, l_tot, row0);
      if constexpr (kWide) {
        if (wide) {
          float l_tot2 = l_run2 + __shfl_xor(l_run2, 16);
          l_tot2 += __shfl_xor(l_tot2, 32);
          flush_block(acc2, m_run2, l_tot2, row0 + kSCols);
        }
      }
      if (more) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = acc2[j] = floatx4{0.f, 0.f, 0.f, 0.f};
        m_run = m_run2 = -INFINITY;
        l_run = l_run2 = 0.f;
        do {
          ++b;
        } while (tstart[b + 1] == tstart[b] && b + 1 < NS);
        b = __builtin_amdgcn_readfirstlane(b);
        cleft = min(__builtin_amdgcn_readfirstlane(tstart[b + 1] - tstart[b]), count - done - 1);
        load_query();
      }
    }
    xs_mark(3);
  }
  if ((PRISM_DBG(a) & 64) && lane == 0) {
    int* d = a.plan_region + kPlanMeasure + 8 * kSMaxWg + 4 * (blockIdx.x * kSKv + h);
    for (int k = 0; k < 4; ++k) d[k] = static_cast<int>(xs[k] & 0x7FFFFFFF);
  }

  // ---- completion: count this range's flushes, merge completed sequences
  __syncthreads();  // every wave is done with the stages (reused as scratch)
  const uint64_t t_loop = (PRISM_DBG(a) & (8 | 32)) ? __builtin_amdgcn_s_memrealtime() : 0;
  stream_finish<QDT, TPR>(a, plan, V, total, tstart, __builtin_amdgcn_readfirstlane(wr0.x), b - wr0.x + 1,
                          reinterpret_cast<int*>(stages));
  if ((PRISM_DBG(a) & 32) && threadIdx.x == 0) {  // measurement aid: phase stamps (100 MHz clock)
    int* d = a.plan_region + kPlanMeasure + 8 * blockIdx.x;
    d[0] = static_cast<int>(r_entry & 0x7FFFFFFF);
    d[1] = static_cast<int>(t_begin & 0x7FFFFFFF);
    d[2] = static_cast<int>(t_loop & 0x7FFFFFFF);
    d[5] = static_cast<int>(__builtin_amdgcn_s_memrealtime() & 0x7FFFFFFF);
    d[7] = (b - wr0.x + 1) | ((wr0.x < V) ? 0x10000 : 0) | (count << 17);  // entries, virtual first, tiles
    // where the workgroup ran: XCC id (high half), HW_ID's CU/SH/SE fields (low half)
    const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
    const unsigned xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);
    a.plan_region[kPlanMergeStamps + 4 * blockIdx.x + 3] = static_cast<int>(((xcc & 0xF) << 16) | ((hw >> 8) & 0xFF));
  }
  if ((PRISM_DBG(a) & 8) && threadIdx.x == 0) {  // measurement aid: start, loop end, end (100 MHz clock)
    const uint64_t t_end = __builtin_amdgcn_s_memrealtime();
    plan[kPlanWgTime + 2 * blockIdx.x] = static_cast<int>(t_begin & 0x7FFFFFFF);
    plan[kPlanWgTime + 2 * blockIdx.x + 1] = static_cast<int>(t_end & 0x7FFFFFFF);
    plan[kPlanCnt + kSMaxBatch + blockIdx.x] = static_cast<int>((t_end - t_loop) & 0x7FFFFFFF);
  }
}

// ---------------------------------------------------------------- generic path

constexpr int kGenericMaxDim = 256;

__device__ __forceinline__ float load_cache(const uint8_t* base, int dtype, int64_t elem) {
  switch (dtype) {
    case PRISM_DTYPE_FP8_E4M3FN: {
      uint32_t bytev = base[elem];
      return __builtin_amdgcn_cvt_f32_fp8(bytev, 0);
    }
    case PRISM_DTYPE_BF16: return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[elem]);
    case PRISM_DTYPE_F16: return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[elem]);
    default: return reinterpret_cast<const float*>(base)[elem];
  }
}

// Strides of k/v here are in ELEMENTS of the cache dtype.
template <int QDT>
__global__ void __launch_bounds__(64) paged_decode_generic_kernel(const DecodeArgs a) {
  __shared__ float q_s[kGenericMaxDim];
  __shared__ float p_s[64];
  __shared__ int valid_s[64];
  __shared__ int64_t vrow_s[64];
  const int b = blockIdx.x;
  const int hq = blockIdx.y;
  const int lane = threadIdx.x;
  const int D = a.head_dim;
  const int hk = hq / a.groups;
  const bool scaled = a.ks != nullptr;
  for (int d = lane; d < D; d += 64)
    q_s[d] = load_q<QDT>(a.q, static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(hq) * a.q_sh + d * a.q_sd);
  __syncthreads();
  const int n_eff = effective_len(a, b);
  const int32_t* bt_row = a.bt + static_cast<int64_t>(b) * a.bt_sb;
  float m_run = -INFINITY, l_run = 0.f;
  float acc[kGenericMaxDim / 64];
#pragma unroll
  for (int k = 0; k < kGenericMaxDim / 64; ++k) acc[k] = 0.f;
  for (int t0 = 0; t0 < n_eff; t0 += 64) {
    const int tok = t0 + lane;
    bool valid = tok < n_eff;
    int64_t krow = 0, vrow = 0;
    float ksc = 1.f, vsc = 1.f;
    if (valid) {
      const int page = tok / a.page_size;
      const int off = tok - page * a.page_size;
      const int32_t blk = bt_row[page * a.bt_sn];
      valid = blk >= 0 && blk < a.num_blocks;
      if (valid) {
        krow = blk * a.k_sblk + static_cast<int64_t>(off) * a.k_stok + hk * a.k_sh;
        vrow = blk * a.v_sblk + static_cast<int64_t>(off) * a.v_stok + hk * a.v_sh;
        if (scaled) {
          ksc = a.ks[blk * a.ks_sblk + static_cast<int64_t>(off) * a.ks_stok + hk * a.ks_sh];
          vsc = a.vs[blk * a.vs_sblk + static_cast<int64_t>(off) * a.vs_stok + hk * a.vs_sh];
        }
      }
    }
    float xs = -INFINITY;
    if (valid) {
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += q_s[d] * load_cache(a.k, a.cache_dtype, krow + d);
      xs = dot * ksc * a.scale_log2;
    }
    float tmax = xs;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, off));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    m_run = m_new;
    const float p = valid ? exp2f(xs - m_use) : 0.f;
    float psum = p;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) psum += __shfl_xor(psum, off);
    l_run = l_run * alpha + psum;
    p_s[lane] = valid ? p * vsc : 0.f;
    vrow_s[lane] = vrow;
    valid_s[lane] = valid;
    __syncthreads();
    const int chunk = min(64, n_eff - t0);
#pragma unroll
    for (int k = 0; k < kGenericMaxDim / 64; ++k) {
      const int d = lane + 64 * k;
      if (d < D) {
        float sum = acc[k] * alpha;
        for (int t = 0; t < chunk; ++t)
          if (valid_s[t]) sum += p_s[t] * load_cache(a.v, a.cache_dtype, vrow_s[t] + d);
        acc[k] = sum;
      }
    }
    __syncthreads();
  }
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  const int64_t base = static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(hq) * a.o_sh;
#pragma unroll
  for (int k = 0; k < kGenericMaxDim / 64; ++k) {
    const int d = lane + 64 * k;
    if (d < D) store_out<QDT>(a.out, base + d * a.o_sd, acc[k] * inv);
  }
}

// ---------------------------------------------------------------- host side

struct Geometry {
  bool fast;
  int split;
  int max_splits;
  int64_t ws_bytes;
  int64_t acc_off, ml_off, cnt_off;
  // streaming path (canonical layout only; chosen per call from the strides)
  bool stream_shape;
  int stream_nwg;
  int stream_vcols;  // query columns of a virtual sequence
  int64_t stream_acc_off, stream_ml_off, stream_vrow0;
};

// PRISM_DECODE_PATH=split|stream forces a kernel family (tests, A/B runs);
// unset, the streaming kernel is used when the table's capacity gives enough
// tiles for the batch size (geometry()) and the per-split kernel otherwise
// (lower latency for a few sequences, whose streaming partials one workgroup
// per sequence would merge).
// Kernel-family overrides: PRISM_DECODE_PATH (split|stream), PRISM_DECODE_SPLIT
// (tokens per split) and PRISM_DECODE_SHARE=0 (no shared-page analysis) are
// read from the environment once, on the first decode call of the process;
// prism_paged_decode_set_overrides changes them afterwards (tests run every
// family on the same inputs).  None of them skips work.
struct EnvOverrides {
  std::atomic<int> path{0};   // 0 automatic, 1 split, 2 stream
  std::atomic<int> split{0};  // 0 automatic, else tokens per split
  std::atomic<int> share{1};
  std::atomic<int> plan_spin{kPlanSpinLimit};
};

EnvOverrides& env_overrides() {
  static EnvOverrides* o = [] {
    auto* x = new EnvOverrides;
    const char* p = getenv("PRISM_DECODE_PATH");
    if (p && p[0] == 's') x->path = p[1] == 'p' ? 1 : (p[1] == 't' ? 2 : 0);
    const char* sp = getenv("PRISM_DECODE_SPLIT");
    if (sp) x->split = atoi(sp);
    const char* sh = getenv("PRISM_DECODE_SHARE");
    x->share = (sh && sh[0] == '0') ? 0 : 1;
    return x;
  }();  // thread-safe one-time initialisation
  return *o;
}

int forced_path() { return env_overrides().path.load(); }

// Tag of one split-K call's chunk counters: process-wide, nonzero, and
// different from the previous 2^32 - 2 calls'.
unsigned int next_split_epoch() {
  static std::atomic<unsigned int> counter{0};
  unsigned int e = counter.fetch_add(1, std::memory_order_relaxed) + 1;
  if (e == 0) e = counter.fetch_add(1, std::memory_order_relaxed) + 1;
  return e;
}

bool stream_disabled() { return forced_path() == 1; }

// FP8 caches (scaled or unit scale) and 16-bit caches (bf16, f16; the split-K
// kernel takes them when the query has the cache's dtype).
bool fast_geometry(int num_heads, int num_kv_heads, int head_dim, int cache_dtype) {
  const bool dtype_ok = cache_dtype == PRISM_DTYPE_FP8_E4M3FN || cache_dtype == PRISM_DTYPE_BF16 ||
                        cache_dtype == PRISM_DTYPE_F16;
  if (!dtype_ok || head_dim != kHeadDim) return false;
  if (num_kv_heads <= 0 || num_kv_heads > 8 || num_heads % num_kv_heads) return false;
  return num_heads / num_kv_heads <= 16;
}

// Tokens per chunk of the split-K path (a multiple of 8 tiles, one per
// wave): aim for about one workgroup per CU over batch x kv heads x chunks,
// with at least one tile per wave and at most kSplitMaxChunks chunks.  Fewer,
// longer chunks than two per CU: each wave keeps its tiles' loads in flight
// back to back and the merge reads half the partials.  Measured (8 kv heads,
// cold, 8 layers back to back, scaled FP8 / bf16 us, two per CU -> one): B = 1
// x 32k 37.8 -> 32.3 / 44.9 -> 40.6, B = 2 x 16k 35.5 -> 31.3, B = 4 x 16k
// 52.0 -> 46.3, B = 8 x 2k 24.6 -> 23.7 / 31.2 -> 27.1; shapes whose chunk
// count was already bound by one tile per wave (B = 1 x 1800, B = 4 x 1k)
// are unchanged.
int choose_split(int batch, int num_kv_heads, int page_size, int width) {
  constexpr int64_t kChunkTok = static_cast<int64_t>(kSplitWaves) * kTile;
  {
    const int v = env_overrides().split.load();
    if (v >= kTile) return static_cast<int>(align_up(v, kChunkTok));
  }
  const int64_t cap = static_cast<int64_t>(width) * page_size;
  const int64_t slots = std::max<int64_t>(1, static_cast<int64_t>(batch) * num_kv_heads);
  const int64_t target = static_cast<int64_t>(device_cu_count());
  int64_t chunks = ceil_div(target, slots);
  chunks = std::min<int64_t>(chunks, std::min<int64_t>(kSplitMaxChunks, std::max<int64_t>(1, ceil_div(cap, kChunkTok))));
  if (chunks < 1) chunks = 1;
  const int64_t per_wave = std::max<int64_t>(1, ceil_div(cap, chunks * kChunkTok));  // tiles per wave
  return static_cast<int>(per_wave * kChunkTok);
}

Geometry geometry(int batch, int num_heads, int num_kv_heads, int head_dim, int page_size, int width,
                  int cache_dtype) {
  Geometry geo{};
  geo.fast = fast_geometry(num_heads, num_kv_heads, head_dim, cache_dtype);
  if (!geo.fast) return geo;
  geo.split = choose_split(batch, num_kv_heads, page_size, width);
  const int64_t cap = static_cast<int64_t>(width) * page_size;
  // the in-kernel merge addresses the partials with 32-bit byte offsets
  while (cap > geo.split &&
         static_cast<int64_t>(batch) * ceil_div(cap, geo.split) * num_heads * head_dim * 4 >= (1LL << 31))
    geo.split *= 2;
  geo.max_splits = static_cast<int>(cap > 0 ? ceil_div(cap, geo.split) : 1);
  // Every fast-path workspace starts with the streaming kernel's plan region,
  // which only the plan code writes (a workspace shared by calls of
  // different geometries never has its plan overwritten by split partials).
  const int64_t plan_bytes = align_up(static_cast<int64_t>(kPlanRegionInts) * 4, 256);
  if (geo.max_splits <= 1) {
    geo.ws_bytes = 0;
  } else {
    const int64_t rows = static_cast<int64_t>(batch) * geo.max_splits * num_heads;
    geo.acc_off = plan_bytes;
    geo.ml_off = geo.acc_off + align_up(rows * head_dim * 4, 256);
    geo.cnt_off = geo.ml_off + align_up(rows * 2 * 4, 256);
    geo.ws_bytes = geo.cnt_off + align_up(static_cast<int64_t>(batch) * num_kv_heads * 8, 256);
  }
  const int ttok = (num_kv_heads > 0 && num_kv_heads <= kSKv && (kSKv % num_kv_heads) == 0 &&
                    (num_kv_heads & (num_kv_heads - 1)) == 0)
                       ? kSTile * (kSKv / num_kv_heads)
                       : 0;  // 8, 4, 2 or 1 kv heads
  // FP8 caches with 8, 4, 2 or 1 kv heads; 16-bit caches with 8 (a 2 KB token
  // row of 16-bit elements makes 16-token tiles of 8 heads)
  const bool stream_dtype = cache_dtype == PRISM_DTYPE_FP8_E4M3FN ||
                            ((cache_dtype == PRISM_DTYPE_BF16 || cache_dtype == PRISM_DTYPE_F16) &&
                             num_kv_heads == kSKv);
  geo.stream_shape = stream_dtype && ttok > 0 && page_size % ttok == 0 &&
                     batch <= kSMaxBatch && !stream_disabled() &&
                     device_cu_count() * kSWgPerCu <= kSMaxWg;
  if (geo.stream_shape && forced_path() != 2) {
    // Automatic choice, from the table's capacity in tiles (the lengths live
    // on the device).  The streaming kernel spreads each sequence over about
    // nwg / batch workgroups, whose partials one workgroup then merges, so
    // few sequences favour the per-split kernel even with many tiles.
    // Measured (8 kv heads, scaled FP8, cold, 8 layers back to back; stream
    // against split, us): B = 2 x 32k 71 / 46; B = 4 x 8k / 16k / 32k / 64k
    // 44 / 31, 52 / 46, 74 / 75, 111 / 133; B = 8 x 2k / 4k / 8k / 16k 29 /
    // 24, 33 / 31, 44 / 46, 62 / 76; B = 16 x 1k / 2k 23 / 23, 29 / 31; B =
    // 32 x 512 22 / 20, B = 64 x 256 20 / 21, B = 128 x 256 26 / 35.
    const int64_t cap_tiles = static_cast<int64_t>(batch) * ceil_div(static_cast<int64_t>(width) * page_size, ttok);
    const int64_t nwg = static_cast<int64_t>(device_cu_count()) * kSWgPerCu;
    const bool enough = (batch >= 16 && cap_tiles >= 4 * nwg) || (batch >= 8 && cap_tiles >= 16 * nwg) ||
                        (batch >= 4 && cap_tiles >= 32 * nwg);
    if (!enough) geo.stream_shape = false;
  }
  if (geo.stream_shape) {
    // workspace: shared-page plan, then partial rows of the real sequences
    // and of the virtual ones
    geo.stream_nwg = device_cu_count() * kSWgPerCu;
    // tiles of 8 kv heads (FP8 or 16-bit) walk shared pages for two column blocks at once
    geo.stream_vcols = num_kv_heads == kSKv ? kVMax : kSCols;
    const int members = geo.stream_vcols / (num_heads / num_kv_heads);
    const int64_t vmax = (batch <= kSShareMaxBatch && members >= 2) ? std::min(kSMaxVirt, batch / 2) : 0;
    // real rows: (wg + V + b) * 8G (one set of G per head slot); virtual
    // rows: (wg + v) * 8 * vcols
    const int64_t slot_rows = static_cast<int64_t>(kSKv) * (num_heads / num_kv_heads);
    geo.stream_vrow0 = (static_cast<int64_t>(geo.stream_nwg) + vmax + batch) * slot_rows;
    const int64_t rows =
        geo.stream_vrow0 + (vmax > 0 ? (static_cast<int64_t>(geo.stream_nwg) + vmax) * kSKv * geo.stream_vcols : 0);
    geo.stream_acc_off = plan_bytes;
    geo.stream_ml_off = geo.stream_acc_off + align_up(rows * head_dim * 4, 256);
    const int64_t need = geo.stream_ml_off + align_up(rows * 2 * 4, 256);
    if (need > geo.ws_bytes) geo.ws_bytes = need;
  }
  return geo;
}

template <int QDT>
int launch_stream(int stage, const DecodeArgs& args, const Geometry& geo, hipStream_t stream) {
  if (stage == 3) {  // the plan alone (the streaming kernel checks and, when needed, builds it itself)
    hipLaunchKernelGGL(paged_decode_stream_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, args);
    return check_launch("paged_decode_stream_plan_kernel launch");
  }
  // token slots per row: 1 (8 kv heads), 2 (4), 4 (2) or 8 (1)
  if (stage == 0 || stage == 1) {
    const dim3 grid(geo.stream_nwg), block(kSThreads);
#define PRISM_LAUNCH_STREAM(V, T) \
  hipLaunchKernelGGL((paged_decode_stream_kernel<QDT, V, T, false>), grid, block, 0, stream, args)
    if (args.cache_dtype != PRISM_DTYPE_FP8_E4M3FN) {  // 16-bit cache of the query's dtype, 8 kv heads
      if constexpr (QDT != PRISM_DTYPE_F32) {
        if (args.q_vec) hipLaunchKernelGGL((paged_decode_stream_kernel<QDT, true, 1, true>), grid, block, 0, stream, args);
        else hipLaunchKernelGGL((paged_decode_stream_kernel<QDT, false, 1, true>), grid, block, 0, stream, args);
      }
    } else if (args.q_vec) {
      if (args.s_tpr == 8) PRISM_LAUNCH_STREAM(true, 8);
      else if (args.s_tpr == 4) PRISM_LAUNCH_STREAM(true, 4);
      else if (args.s_tpr == 2) PRISM_LAUNCH_STREAM(true, 2);
      else PRISM_LAUNCH_STREAM(true, 1);
    } else {
      if (args.s_tpr == 8) PRISM_LAUNCH_STREAM(false, 8);
      else if (args.s_tpr == 4) PRISM_LAUNCH_STREAM(false, 4);
      else if (args.s_tpr == 2) PRISM_LAUNCH_STREAM(false, 2);
      else PRISM_LAUNCH_STREAM(false, 1);
    }
#undef PRISM_LAUNCH_STREAM
    return check_launch("paged_decode_stream_kernel launch");
  }
  return PRISM_OK;  // stage 2: the streaming kernel merges its own partials
}

template <int QDT>
int launch_all(int stage, const DecodeArgs& args, const Geometry& geo, bool page_aligned, bool use_stream,
               hipStream_t stream) {
  if (use_stream) return launch_stream<QDT>(stage, args, geo, stream);
  if (stage == 3) return PRISM_OK;  // no plan outside the streaming kernel
  const bool scaled = args.ks != nullptr;
  if (!geo.fast) {
    if (stage == 2) return PRISM_OK;
    hipLaunchKernelGGL(paged_decode_generic_kernel<QDT>, dim3(args.batch, args.num_heads), dim3(64), 0, stream,
                       args);
    return check_launch("paged_decode_generic_kernel launch");
  }
  if (stage == 2) return PRISM_OK;  // the split-K kernel merges its own chunks
  {
    const dim3 grid(args.batch, args.num_kv_heads, geo.max_splits);
    const dim3 block(64 * kSplitWaves);
#define PRISM_LAUNCH_SPLIT(S, A, CB)                                                                   \
  do {                                                                                                 \
    if (args.q_vec)                                                                                    \
      hipLaunchKernelGGL((paged_decode_split_kernel<QDT, S, A, true, CB>), grid, block, 0, stream, args);  \
    else                                                                                               \
      hipLaunchKernelGGL((paged_decode_split_kernel<QDT, S, A, false, CB>), grid, block, 0, stream, args); \
  } while (0)
    if (args.cache_dtype != PRISM_DTYPE_FP8_E4M3FN) {  // 16-bit cache of the query's dtype, unscaled
      if constexpr (QDT != PRISM_DTYPE_F32) {
        if (page_aligned) PRISM_LAUNCH_SPLIT(false, true, 2);
        else PRISM_LAUNCH_SPLIT(false, false, 2);
      }
    } else if (scaled && page_aligned) PRISM_LAUNCH_SPLIT(true, true, 1);
    else if (scaled) PRISM_LAUNCH_SPLIT(true, false, 1);
    else if (page_aligned) PRISM_LAUNCH_SPLIT(false, true, 1);
    else PRISM_LAUNCH_SPLIT(false, false, 1);
#undef PRISM_LAUNCH_SPLIT
    return check_launch("paged_decode_split_kernel launch");
  }
}

}  // namespace

// Loads this file's code object now rather than at its first kernel launch.
int preload_paged_decode() {
  hipFuncAttributes attr;
  return check_hip(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&paged_decode_stream_plan_kernel)),
                   "preload_paged_decode");
}

}  // namespace prism

extern "C" int prism_paged_decode_set_overrides(int path, int split_tokens, int share) {
  prism::clear_error();
  if (path < 0 || path > 2 || split_tokens < 0 || share < 0 || share > 1) {
    prism::set_error("prism_paged_decode_set_overrides: path must be 0-2, split_tokens >= 0, share 0 or 1");
    return PRISM_ERR_INVALID;
  }
  auto& o = prism::env_overrides();
  o.path = path;
  o.split = split_tokens;
  o.share = share;
  return PRISM_OK;
}

extern "C" int prism_paged_decode_set_plan_wait_limit(int polls) {
  prism::clear_error();
  if (polls < 0) {
    prism::set_error("prism_paged_decode_set_plan_wait_limit: polls must be >= 0, got %d", polls);
    return -1;
  }
  return prism::env_overrides().plan_spin.exchange(polls > 0 ? polls : 0);
}

extern "C" int prism_paged_decode_default_plan_wait_limit(void) { return prism::kPlanSpinLimit; }

extern "C" void prism_paged_decode_get_overrides(int out[3]) {
  auto& o = prism::env_overrides();
  out[0] = o.path.load();
  out[1] = o.split.load();
  out[2] = o.share.load();
}

extern "C" int64_t prism_paged_decode_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim,
                                                      int page_size, int max_blocks_per_seq, int cache_dtype) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || max_blocks_per_seq < 0)
    return -1;
  return prism::geometry(batch, num_heads, num_kv_heads, head_dim, page_size, max_blocks_per_seq, cache_dtype)
      .ws_bytes;
}

extern "C" int prism_paged_decode_split_tokens(int batch, int num_heads, int num_kv_heads, int head_dim,
                                               int page_size, int max_blocks_per_seq, int cache_dtype) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || max_blocks_per_seq < 0)
    return -1;
  prism::Geometry geo =
      prism::geometry(batch, num_heads, num_kv_heads, head_dim, page_size, max_blocks_per_seq, cache_dtype);
  return geo.fast ? geo.split : 0;
}

extern "C" int prism_paged_decode_kernel_family(int batch, int num_heads, int num_kv_heads, int head_dim,
                                                int page_size, int max_blocks_per_seq, int cache_dtype) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || max_blocks_per_seq < 0)
    return -1;
  prism::Geometry geo =
      prism::geometry(batch, num_heads, num_kv_heads, head_dim, page_size, max_blocks_per_seq, cache_dtype);
  if (!geo.fast) return 0;
  return geo.stream_shape ? 2 : 1;
}

extern "C" int prism_paged_decode_stage(
    int stage, const void* q, int q_dtype, const int64_t q_strides[3], const void* k_cache, const void* v_cache,
    int cache_dtype, const int64_t k_strides[4], const int64_t v_strides[4], const float* k_scale,
    const float* v_scale, const int64_t ks_strides[3], const int64_t vs_strides[3], const int32_t* block_tables,
    const int64_t bt_strides[2], const int32_t* context_lens, const int32_t* max_context_len, void* out,
    const int64_t out_strides[3], int batch, int num_heads, int num_kv_heads, int head_dim, int page_size,
    int64_t num_blocks, int max_blocks_per_seq, float scale, void* workspace, int64_t workspace_bytes,
    void* stream_ptr) {
  using namespace prism;
  clear_error();
  if (stage < 0 || stage > 3) {
    set_error("prism_paged_decode: stage must be 0, 1, 2 or 3");
    return PRISM_ERR_INVALID;
  }
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 ||
      max_blocks_per_seq < 0 || num_blocks < 0) {
    set_error("prism_paged_decode: invalid geometry");
    return PRISM_ERR_INVALID;
  }
  if (num_heads % num_kv_heads) {
    set_error("prism_paged_decode: num_heads must be divisible by num_kv_heads, got %d and %d", num_heads,
              num_kv_heads);
    return PRISM_ERR_INVALID;
  }
  if (q_dtype != PRISM_DTYPE_F32 && q_dtype != PRISM_DTYPE_BF16 && q_dtype != PRISM_DTYPE_F16) {
    set_error("prism_paged_decode: unsupported query dtype code %d", q_dtype);
    return PRISM_ERR_INVALID;
  }
  if (dtype_size(cache_dtype) == 0) {
    set_error("prism_paged_decode: unsupported cache dtype code %d", cache_dtype);
    return PRISM_ERR_INVALID;
  }
  if ((k_scale == nullptr) != (v_scale == nullptr)) {
    set_error("prism_paged_decode: K/V scale caches must be provided together");
    return PRISM_ERR_INVALID;
  }
  if (k_scale && cache_dtype != PRISM_DTYPE_FP8_E4M3FN) {
    set_error("prism_paged_decode: token-head scales require FP8 E4M3FN K/V payload caches");
    return PRISM_ERR_INVALID;
  }
  if (head_dim > kGenericMaxDim) {
    set_error("prism_paged_decode: supports head_dim <= %d, got %d", kGenericMaxDim, head_dim);
    return PRISM_ERR_INVALID;
  }
  if (k_strides[3] != 1 || v_strides[3] != 1) {
    set_error("prism_paged_decode: K/V caches need a unit head_dim stride");
    return PRISM_ERR_LAYOUT;
  }
  if (batch == 0) return PRISM_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !max_context_len || !out) {
    set_error("prism_paged_decode: null pointer argument");
    return PRISM_ERR_INVALID;
  }
  const int esz = dtype_size(cache_dtype);
  Geometry geo = geometry(batch, num_heads, num_kv_heads, head_dim, page_size, max_blocks_per_seq, cache_dtype);
  if (geo.fast) {
    // 16-byte row loads need 16-byte aligned rows.
    const bool ok = aligned(k_cache, 16) && aligned(v_cache, 16) && k_strides[0] % 16 == 0 && k_strides[1] % 16 == 0 &&
                    k_strides[2] % 16 == 0 && v_strides[0] % 16 == 0 && v_strides[1] % 16 == 0 &&
                    v_strides[2] % 16 == 0;
    // The branch-free tile loader reads page 0 for absent blocks: needs >= 1 page.
    // A 16-bit cache feeds the MFMAs as it is, so the query must have its dtype.
    const bool dtype_ok = cache_dtype == PRISM_DTYPE_FP8_E4M3FN || q_dtype == cache_dtype;
    if (!ok || num_blocks < 1 || !dtype_ok) geo.fast = false, geo.ws_bytes = 0, geo.max_splits = 1;
  }
  if (geo.fast && geo.ws_bytes > 0) {
    if (!workspace || workspace_bytes < geo.ws_bytes) {
      set_error("prism_paged_decode: workspace too small (%lld < %lld bytes)", static_cast<long long>(workspace_bytes),
                static_cast<long long>(geo.ws_bytes));
      return PRISM_ERR_INVALID;
    }
    if (!aligned(workspace, 256)) {
      set_error("prism_paged_decode: workspace must be 256-byte aligned");
      return PRISM_ERR_LAYOUT;
    }
  }
  DecodeArgs args{};
  args.q = q;
  args.q_sb = q_strides[0];
  args.q_sh = q_strides[1];
  args.q_sd = q_strides[2];
  args.k = static_cast<const uint8_t*>(k_cache);
  args.v = static_cast<const uint8_t*>(v_cache);
  // The fast path addresses K/V in bytes; the generic path in elements.
  const int64_t mul = geo.fast ? esz : 1;
  args.k_sblk = k_strides[0] * mul;
  args.k_stok = k_strides[1] * mul;
  args.k_sh = k_strides[2] * mul;
  args.v_sblk = v_strides[0] * mul;
  args.v_stok = v_strides[1] * mul;
  args.v_sh = v_strides[2] * mul;
  args.ks = k_scale;
  args.vs = v_scale;
  if (k_scale) {
    args.ks_sblk = ks_strides[0];
    args.ks_stok = ks_strides[1];
    args.ks_sh = ks_strides[2];
    args.vs_sblk = vs_strides[0];
    args.vs_stok = vs_strides[1];
    args.vs_sh = vs_strides[2];
  }
  args.bt = block_tables;
  args.bt_sb = bt_strides[0];
  args.bt_sn = bt_strides[1];
  args.ctx = context_lens;
  args.max_ctx = max_context_len;
  args.out = out;
  args.o_sb = out_strides[0];
  args.o_sh = out_strides[1];
  args.o_sd = out_strides[2];
  if (geo.fast && geo.ws_bytes > 0) {
    args.part_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + geo.acc_off);
    args.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + geo.ml_off);
    args.split_cnt = reinterpret_cast<unsigned long long*>(static_cast<uint8_t*>(workspace) + geo.cnt_off);
    args.epoch = next_split_epoch();
  }
  args.batch = batch;
  args.num_heads = num_heads;
  args.num_kv_heads = num_kv_heads;
  args.groups = num_heads / num_kv_heads;
  args.page_size = page_size;
  args.width = max_blocks_per_seq;
  args.head_dim = head_dim;
  args.num_blocks = num_blocks;
  {
    const int qsz = dtype_size(q_dtype);
    const int64_t per16 = 16 / qsz;
    args.q_vec = q_strides[2] == 1 && aligned(q, 16) && q_strides[0] % per16 == 0 && q_strides[1] % per16 == 0;
  }
  args.split = geo.fast ? geo.split : 0;
  args.max_splits = geo.fast ? geo.max_splits : 1;
  args.scale_log2 = scale * kLog2e;
  args.cache_dtype = cache_dtype;
#ifdef PRISM_DECODE_MEASURE
  {
    const char* dbg = getenv("PRISM_STREAM_DEBUG");
    args.debug = dbg ? atoi(dbg) : 0;
  }
#endif
  const bool page_aligned = (page_size % kTile) == 0;
  // Streaming path: canonical contiguous page layout, with scales in the
  // matching [block][token][head] layout or none (unit-scale FP8).
  // (token rows of num_kv_heads * 128 bytes, contiguous within a page)
  const int64_t tok_bytes = static_cast<int64_t>(num_kv_heads) * kHeadDim;
  const bool scale_layout = k_scale == nullptr ||
                            (ks_strides[1] == num_kv_heads && ks_strides[2] == 1 && vs_strides[1] == num_kv_heads &&
                             vs_strides[2] == 1 && ks_strides[0] == vs_strides[0] && aligned(k_scale, 16) &&
                             aligned(v_scale, 16) && ks_strides[0] % 4 == 0);
  const bool use_stream = geo.fast && geo.stream_shape && k_strides[1] == tok_bytes && k_strides[2] == kHeadDim &&
                          v_strides[1] == tok_bytes && v_strides[2] == kHeadDim &&
                          scale_layout && (cache_dtype == PRISM_DTYPE_FP8_E4M3FN || cache_dtype == q_dtype);
  if (use_stream) {
    args.plan_region = static_cast<int*>(workspace);
    args.epoch = next_split_epoch();
    args.part_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + geo.stream_acc_off);
    args.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + geo.stream_ml_off);
    args.vrow0 = geo.stream_vrow0;
    args.s_tpr = kSKv / num_kv_heads;
    args.s_ttok = kSTile * args.s_tpr;
    args.share = env_overrides().share.load();
    args.stream_nwg = geo.stream_nwg;
    args.vcols = geo.stream_vcols;
    args.plan_spin = env_overrides().plan_spin.load();
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  switch (q_dtype) {
    case PRISM_DTYPE_BF16: return launch_all<PRISM_DTYPE_BF16>(stage, args, geo, page_aligned, use_stream, stream);
    case PRISM_DTYPE_F16: return launch_all<PRISM_DTYPE_F16>(stage, args, geo, page_aligned, use_stream, stream);
    default: return launch_all<PRISM_DTYPE_F32>(stage, args, geo, page_aligned, use_stream, stream);
  }
}

extern "C" int prism_paged_decode(const void* q, int q_dtype, const int64_t q_strides[3], const void* k_cache,
                                  const void* v_cache, int cache_dtype, const int64_t k_strides[4],
                                  const int64_t v_strides[4], const float* k_scale, const float* v_scale,
                                  const int64_t ks_strides[3], const int64_t vs_strides[3],
                                  const int32_t* block_tables, const int64_t bt_strides[2],
                                  const int32_t* context_lens, const int32_t* max_context_len, void* out,
                                  const int64_t out_strides[3], int batch, int num_heads, int num_kv_heads,
                                  int head_dim, int page_size, int64_t num_blocks, int max_blocks_per_seq,
                                  float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  return prism_paged_decode_stage(0, q, q_dtype, q_strides, k_cache, v_cache, cache_dtype, k_strides, v_strides,
                                  k_scale, v_scale, ks_strides, vs_strides, block_tables, bt_strides, context_lens,
                                  max_context_len, out, out_strides, batch, num_heads, num_kv_heads, head_dim,
                                  page_size, num_blocks, max_blocks_per_seq, scale, workspace, workspace_bytes,
                                  stream);
}

// ------------------------------------------------------- allocation-free entry

namespace prism {
namespace {

// Scratch of prism_paged_decode_noalloc: the decode workspace (streaming
// plan, partials, merge counters) of callers that cannot allocate.  Each GPU
// the library runs on holds its own copy until the process ends.  Host code
// must not use the array's name as a device address: the address of each
// device's copy comes from hipGetSymbolAddress, once per device.
constexpr int64_t kNoAllocScratchBytes = int64_t{64} << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// In-flight guard of each device's scratch: the stream of the last call that
// used it and an event recorded behind that call's kernels.  A call on
// another stream while that event has not completed would overwrite the
// plan, partials and counters the running call is using, so it is refused.
struct ScratchUse {
  hipEvent_t done = nullptr;
  hipStream_t stream = nullptr;
  bool recorded = false;
};
ScratchUse g_scratch_use[kMaxDevices];

// The current device's copy of `scratch` and its guard (set up on the
// device's first call: the symbol's address and the guard's event).
int scratch_for_current_device(void** out, int* device) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "prism_paged_decode_noalloc: hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("prism_paged_decode_noalloc: device ordinal %d is out of range", dev);
    return PRISM_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                           "prism_paged_decode_noalloc: hipGetSymbolAddress"))
      return rc;
    hipEvent_t ev = nullptr;
    if (int rc = check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming),
                           "prism_paged_decode_noalloc: hipEventCreateWithFlags"))
      return rc;
    g_scratch_use[dev].done = ev;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  *device = dev;
  return PRISM_OK;
}

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

}  // namespace
}  // namespace prism

extern "C" int prism_paged_decode_noalloc(const void* q, int q_dtype, const int64_t q_strides[3],
                                          const void* k_cache, const void* v_cache, int cache_dtype,
                                          const int64_t k_strides[4], const int64_t v_strides[4],
                                          const float* k_scale, const float* v_scale,
                                          const int64_t ks_strides[3], const int64_t vs_strides[3],
                                          const int32_t* block_tables, const int64_t bt_strides[2],
                                          const int32_t* context_lens, const int32_t* max_context_len, void* out,
                                          const int64_t out_strides[3], int batch, int num_heads,
                                          int num_kv_heads, int head_dim, int page_size, int64_t num_blocks,
                                          int max_blocks_per_seq, float scale, void* stream) {
  using namespace prism;
  clear_error();
  const int64_t need = prism_paged_decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, page_size,
                                                          max_blocks_per_seq, cache_dtype);
  if (need < 0) {
    set_error("prism_paged_decode_noalloc: invalid geometry");
    return PRISM_ERR_INVALID;
  }
  if (need > kNoAllocScratchBytes) {
    set_error("prism_paged_decode_noalloc: this geometry needs %lld bytes of workspace, more than the %lld-byte "
              "scratch of the allocation-free entry point; use prism_paged_decode with a workspace",
              static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
    return PRISM_ERR_INVALID;
  }
  void* ws = nullptr;
  if (need == 0)  // no kernel of this geometry uses a workspace
    return prism_paged_decode_stage(0, q, q_dtype, q_strides, k_cache, v_cache, cache_dtype, k_strides, v_strides,
                                    k_scale, v_scale, ks_strides, vs_strides, block_tables, bt_strides,
                                    context_lens, max_context_len, out, out_strides, batch, num_heads, num_kv_heads,
                                    head_dim, page_size, num_blocks, max_blocks_per_seq, scale, nullptr, 0, stream);
  int dev = 0;
  if (int rc = scratch_for_current_device(&ws, &dev)) return rc;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  // Launches under graph capture are not guarded (the replay's timing is the
  // caller's): the guard sees eager calls only.
  const bool guarded = !stream_capturing(hs);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);  // one host thread at a time per process
  ScratchUse& use = g_scratch_use[dev];
  if (guarded && use.recorded && use.stream != hs) {
    const hipError_t q_st = hipEventQuery(use.done);
    if (q_st == hipErrorNotReady) {
      set_error("prism_paged_decode_noalloc: the device's scratch is in use by a call still running on another "
                "stream; serialise the calls (or use prism_paged_decode with a workspace per stream)");
      return PRISM_ERR_BUSY;
    }
    if (int rc = check_hip(q_st, "prism_paged_decode_noalloc: hipEventQuery")) return rc;
  }
  // Nothing in the scratch needs clearing: the streaming plan carries the key
  // of the inputs it was computed from (a stale or zero plan is rebuilt, and
  // its rebuild zeroes the merge counters), split-K chunk counters carry the
  // epoch of their call (any other value counts as zero arrivals), and
  // partials are written before they are read.
  const int rc = prism_paged_decode_stage(0, q, q_dtype, q_strides, k_cache, v_cache, cache_dtype, k_strides,
                                          v_strides, k_scale, v_scale, ks_strides, vs_strides, block_tables,
                                          bt_strides, context_lens, max_context_len, out, out_strides, batch,
                                          num_heads, num_kv_heads, head_dim, page_size, num_blocks,
                                          max_blocks_per_seq, scale, ws, need, stream);
  if (rc != PRISM_OK || !guarded) return rc;
  if (int e = check_hip(hipEventRecord(use.done, hs), "prism_paged_decode_noalloc: hipEventRecord")) return e;
  use.stream = hs;
  use.recorded = true;
  return PRISM_OK;
}
