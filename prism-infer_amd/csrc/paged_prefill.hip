// Paged prefill attention over scaled-FP8 pages (chunked / prefix-hit
// prefill): for every sequence i, query token j of its chunk sits at
// position prefix_i + j (prefix_i = context_len_i - query_len_i) and attends
// to keys 0..prefix_i + j of its paged history, which already holds the
// chunk's own K/V.  Restates prism_infer/ops/paged_attention_reference.py:
// 185-246 (gather :22-63, dequantisation :102-122, GQA :125-145): causal
// SDPA over the dequantised pages, output in q's dtype.  Dequantisation here
// is fp32 (payload * scale applied to the fp32 scores and to P), as the
// decode kernels do; the reference multiplies in q's dtype.
//
// Work layout.  A workgroup owns one kv head and one block of 32 query
// tokens of one sequence; its G waves are the G query heads of the kv head,
// so each K/V tile is read once into LDS for all of them.  Tiles of KT keys
// (one page holds whole tiles) are double buffered through LDS: the next
// tile's loads are in flight while the current one is computed.  Per
// 16-key sub-block, a wave computes S^T = K Q^T (bf16 queries: the fp8 MFMA
// 16x16x128 on the K bytes as they are, the query split into two fp8 terms
// that hold it exactly, products exact in fp32; f16 queries:
// v_mfma_f32_16x16x32_f16 on K converted to f16, exact; the key scale
// multiplies the rows of S^T), runs the online softmax per query column
// (log2 domain, lazy rescaling), and accumulates O^T += V^T P^T with
// v_mfma_f32_16x16x32_bf16 (v_mfma_f32_16x16x16_bf16 for 16-key steps), V^T
// coming from ds_read_b64_tr_b8 (fp8 -> bf16 is exact) and P * v_scale
// entering as bf16, whose fp32 exponent range holds every v scale from the
// 1e-6 floor up.  Only tiles on the diagonal apply the causal mask.
//
// Metadata stays on the device: each workgroup finds its sequence and query
// block from cu_seqlens_q with a wave scan.  Invalid lengths or block ids
// record the lowest offending sequence in status[0] (atomicMin); the host
// raises the reference's error for it.
#include "common.h"
#include "fp8_mfma.h"

namespace prism {
namespace {

constexpr int kPfD = 128;                      // head dim
constexpr int kPfCols = 16;                    // query tokens per MFMA column block
constexpr int kPfColBlocks = 2;                // column blocks per wave
constexpr int kPfQTile = kPfCols * kPfColBlocks;  // query tokens per workgroup
constexpr int kPfMaxWaves = 8;                 // GQA group size limit
constexpr float kPfRescaleThreshold = 8.0f;    // log2 units

struct PrefillArgs {
  const void* q;
  int64_t q_st, q_sh;  // elements (dim stride 1)
  const uint8_t* k;
  const uint8_t* v;
  int64_t k_sn, k_sp, k_sh, v_sn, v_sp, v_sh;  // bytes (dim stride 1)
  const float* ks;
  const float* vs;
  int64_t ks_sn, ks_sp, ks_sh, vs_sn, vs_sp, vs_sh;  // elements
  const int32_t* bt;
  int64_t bt_sb, bt_sn;
  const int32_t* ctx;
  const int32_t* cu_q;
  void* out;
  int64_t o_st, o_sh;
  int batch, num_heads, groups, page, num_blocks, width;
  float scale_log2;
  int* status;
};

// 16-byte chunk swizzle of a key row in LDS, by the key's index t.  gfx950
// LDS (measured with SQ_LDS_BANK_CONFLICT): 64 banks of 4 bytes (address bits
// 2..7); ds_read_b64 (and _tr_b8) serves lanes 0-31 and 32-63 in separate
// passes; ds_read_b128 serves 16 lanes per pass, the lanes whose bit 5 and
// parity of bits 2..4 agree.  A 128-byte key row puts bit 7 of the address
// at t & 1, so a row's 8 chunks cover one half of the banks and rows of
// opposite parity the other half.  The swizzle (GF(2)-linear in t: chunk
// ^= 4 t1 ^ 3 t2) makes both reads below conflict-free under that model: the
// K rows' b128 reads (lane (g, c): row c, chunks 2g and 2g + 1) and the V
// tiles' transposed b64 reads (lane (g, c): rows 4g + (c >> 1 & 3), chunk
// 2 jp + (c >> 3)); the previous swizzle cost 4 and 2 extra cycles per read.
__device__ __forceinline__ int pf_swz(int t) { return (((t >> 1) & 1) * 4) ^ (((t >> 2) & 1) * 3); }

// A wave-uniform pointer, moved to SGPRs.
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ void flag_sequence(const PrefillArgs& a, int seq) {
  atomicMin(a.status, seq);
}

// Inclusive wave scan of v (64 lanes).
__device__ __forceinline__ int wave_scan(int v) {
  const int lane = __lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  return v;
}

// Query blocks of sequence i (0 for a sequence with invalid lengths, which
// is flagged).
__device__ __forceinline__ int seq_blocks(const PrefillArgs& a, int i, bool flag) {
  const int q0 = a.cu_q[i];
  const int qlen = a.cu_q[i + 1] - q0;
  const int ctx = a.ctx[i];
  if (qlen <= 0 || ctx < qlen || ctx > a.width * a.page) {
    if (flag) flag_sequence(a, i);
    return 0;
  }
  return (qlen + kPfQTile - 1) / kPfQTile;
}

// Workgroup -> (sequence, query block).  Blocks are numbered in reverse so
// that the last (longest) query blocks start first.  Returns false for a
// workgroup beyond the real blocks.
__device__ bool locate(const PrefillArgs& a, int& seq, int& qblock) {
  const int lane = __lane_id();
  int total = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int i = base + lane;
    const int n = i < a.batch ? seq_blocks(a, i, blockIdx.y == 0 && blockIdx.x == 0 && threadIdx.x < 64) : 0;
    total += __shfl(wave_scan(n), 63);
  }
  const int target = total - 1 - static_cast<int>(blockIdx.x);
  if (target < 0) return false;
  int before = 0;
  for (int base = 0; base < a.batch; base += 64) {
    const int i = base + lane;
    const int n = i < a.batch ? seq_blocks(a, i, false) : 0;
    const int incl = wave_scan(n) + before;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(i < a.batch && target < incl && target >= incl - n);
    if (hit != 0) {
      const int l = __builtin_ctzll(hit);
      seq = __builtin_amdgcn_readfirstlane(base + l);
      qblock = __builtin_amdgcn_readfirstlane(target - (__shfl(incl, l) - __shfl(n, l)));
      return true;
    }
    before = __shfl(incl, 63);
  }
  return false;
}

// Query operand (B of S^T = K Q^T); lane (g, c) holds query column c's
// dims 32g..32g+31, the same dims as the K bytes it meets (row c of the
// block, LDS chunks 2g and 2g + 1); `mul` turns the column's scores into
// log2 units.
//
// bf16 queries: the fp8 MFMA (16x16x128) on the K bytes as they are.  The
// column is scaled by 2^e so that its largest |q| lies in [128, 256) and
// split into two E4M3FN terms (hi, lo).  A bf16 value there is M * 2^k with
// an 8-bit M; hi rounds it to 4 significant bits, which leaves
// (M - 16 H) * 2^k with |M - 16 H| <= 8: at most 4 significant bits, held
// exactly by lo whenever 2^k is on E4M3FN's grid (elements of 2^-2 and up,
// 2^-10 of the column's largest), and within 2^-10 below (2^-18 of the
// largest), as a third term would be.  The score is (K . (hi + lo)) * 2^-e;
// 2^-e joins the softmax scale in `mul`.
//
// f16 queries (11 bits, which two terms do not hold): K converted to f16 per
// block (exact) and v_mfma_f32_16x16x32_f16.
template <int QDT>
struct PfQOperand {
  i32x8 t[2];  // hi, lo
  float mul;   // scale_log2 * 2^-e of this lane's column
};

template <>
struct PfQOperand<PRISM_DTYPE_F16> {
  f16x8 op[4];
  float mul;  // scale_log2
};

template <int QDT>
__device__ __forceinline__ void pf_load_q(const uint16_t* src, bool valid, float scale_log2, PfQOperand<QDT>& q) {
  if constexpr (QDT == PRISM_DTYPE_F16) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const u32x4 w = valid ? *reinterpret_cast<const u32x4*>(src + 8 * cc) : u32x4{0u, 0u, 0u, 0u};
      q.op[cc] = __builtin_bit_cast(f16x8, w);
    }
    q.mul = scale_log2;
  } else {
    float x[32];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const u32x4 w = valid ? *reinterpret_cast<const u32x4*>(src + 8 * cc) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[8 * cc + 2 * e] = bf16_bits_to_f32(w[e] & 0xFFFFu);
        x[8 * cc + 2 * e + 1] = bf16_bits_to_f32(w[e] >> 16);
      }
    }
    float mx = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) mx = fmaxf(mx, fabsf(x[e]));
    mx = wave_max_across_groups(mx);
    // ilogb(mx) = frexp exponent - 1; clamped so that 2^-e stays a normal
    // fp32 number (columns of zeros, or of non-finite values, keep e = 0)
    const int e = (mx > 0.f && mx <= 3.0e38f) ? min(max(8 - __builtin_amdgcn_frexp_expf(mx), -120), 120) : 0;
    q.mul = ldexpf(scale_log2, -e);
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const float y[4] = {ldexpf(x[4 * w], e), ldexpf(x[4 * w + 1], e), ldexpf(x[4 * w + 2], e),
                          ldexpf(x[4 * w + 3], e)};
      uint32_t parts[2];
      fp8_split<2>(y, parts);
      q.t[0][w] = static_cast<int>(parts[0]);
      q.t[1][w] = static_cast<int>(parts[1]);
    }
  }
}

// Two waves per SIMD: at most 256 VGPRs + AGPRs per lane.
template <int QDT, int KT, int NW, bool SCALED>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
paged_prefill_kernel(const PrefillArgs a) {
  constexpr int kRow = kPfD;                  // one key's payload row in LDS (bytes)
  constexpr int kPayload = KT * kRow;         // K or V payload of a tile
  constexpr int kStage = 2 * kPayload + 2 * KT * 4;
  constexpr int kChunks = 2 * KT * (kRow / 16);  // 16-byte payload chunks per tile (K then V)
  constexpr int NB = KT >= 32 ? 2 : 1;            // 16-key blocks per softmax step
  constexpr int kStep = 16 * NB;                  // keys per softmax step
  static_assert(NB == 1 || KT / kStep <= 2, "the V reads below cover two steps per tile");
  using POp = typename std::conditional<NB == 2, bf16x8, shortx4>::type;  // P * v_scale, bf16 (bits for NB = 1)
  __shared__ __attribute__((aligned(256))) uint8_t stages[2 * kStage];

  int seq, qblock;
  if (!locate(a, seq, qblock)) return;
  const int h = blockIdx.y;
  constexpr int nthreads = 64 * NW;
  const int tid = threadIdx.x;
  const int wave = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid / 64);  // uniform: SGPR arithmetic below
  const int lane = tid % 64;
  const int c = lane % 16;
  const int g = lane / 16;
  const int qhead = h * a.groups + wave;

  // sequence metadata in SGPRs: every branch on it below is uniform
  const int qs = __builtin_amdgcn_readfirstlane(a.cu_q[seq]);
  const int qlen = __builtin_amdgcn_readfirstlane(a.cu_q[seq + 1]) - qs;
  const int ctx = __builtin_amdgcn_readfirstlane(a.ctx[seq]);
  const int prefix = ctx - qlen;
  const int qb0 = qblock * kPfQTile;                       // first query token of the block
  const int qcount = min(kPfQTile, qlen - qb0);
  const int kend = prefix + qb0 + qcount;                  // keys [0, kend) are needed
  const int ntiles = (kend + KT - 1) / KT;
  const int32_t* bt_row = a.bt + static_cast<int64_t>(seq) * a.bt_sb;

  // ---- query operand (B of S^T = K Q^T): column c of block cb is query
  // token qb0 + 16 cb + c; lane group g holds dims 32g .. 32g + 31.
  PfQOperand<QDT> qop[kPfColBlocks];
  bool colv[kPfColBlocks];
#pragma unroll
  for (int cb = 0; cb < kPfColBlocks; ++cb) {
    const int j = qb0 + cb * kPfCols + c;
    colv[cb] = j < qlen;
    const uint16_t* src = static_cast<const uint16_t*>(a.q) + static_cast<int64_t>(qs + (colv[cb] ? j : 0)) * a.q_st +
                          static_cast<int64_t>(qhead) * a.q_sh + 32 * g;
    pf_load_q<QDT>(src, colv[cb], a.scale_log2, qop[cb]);
  }

  // ---- tile loads, straight into LDS (load-to-LDS, 16 B per lane): K then
  // V as kChunks 16-byte chunks; chunk i of the stage lands at byte 16 i,
  // i.e. key row i / 8, LDS chunk i % 8, which holds the row's global chunk
  // (i % 8) ^ swz(row).  Scales: threads 0..2KT-1 one float each.
  // Asm so that the compiler's wait-count pass does not drain these loads
  // before each LDS read of the other stage.
  // (waves past the last chunk or scale issue nothing: the waits below are
  // vmcnt(0), so waves need not issue equal numbers of loads)
  static_assert(kChunks % 64 == 0, "whole waves of chunks");
  constexpr int kPer = (kChunks + nthreads - 1) / nthreads;  // chunks per thread
  bool tile_ok = true;
  auto issue_tile = [&](int t, uint8_t* st) {
    const int tok0 = t * KT;
    const int page = tok0 / a.page;
    const int32_t blk = bt_row[static_cast<int64_t>(page) * a.bt_sn];
    tile_ok = blk >= 0 && blk < a.num_blocks;
    if (!tile_ok) {
      if (tid == 0) flag_sequence(a, seq);
      return;
    }
    const int row0 = tok0 - page * a.page;
    const uint32_t st_lds = lds_addr(st);
    // every chunk of a wave is in one page and is all K or all V: a uniform
    // 64-bit base (SGPRs) plus a 32-bit per-lane offset (the host checks
    // that a page's bytes of one head span less than 2^31)
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int ch0 = k * nthreads + wave * 64;  // the wave's first chunk (uniform); 64 contiguous chunks
      const int ch = ch0 + lane;
      if (ch0 >= kChunks) break;
      const int isv = ch0 >= kChunks / 2;
      const int cw = ch - isv * (kChunks / 2);
      const int tok = cw / (kRow / 16);
      const int part = (cw % (kRow / 16)) ^ pf_swz(tok);
      const uint8_t* base = isv ? a.v + blk * a.v_sn + static_cast<int64_t>(row0) * a.v_sp + h * a.v_sh
                                : a.k + blk * a.k_sn + static_cast<int64_t>(row0) * a.k_sp + h * a.k_sh;
      const uint32_t off = static_cast<uint32_t>(tok * static_cast<int>(isv ? a.v_sp : a.k_sp) + part * 16);
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(st_lds + static_cast<uint32_t>(ch0) * 16);
      asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(uniform_ptr(base)),
                   "s"(m0) : "memory", "m0");
    }
    if constexpr (SCALED) {
      // threads 0..KT-1 load the K scales, KT..2KT-1 the V scales (exec-masked
      // halves of one wave share M0: the LDS address is M0 + 4 * lane)
      const int si = tid;
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(st_lds + 2 * kPayload + static_cast<uint32_t>(wave * 64) * 4);
      if (si < KT) {
        const uint8_t* base = uniform_ptr(reinterpret_cast<const uint8_t*>(
            a.ks + blk * a.ks_sn + static_cast<int64_t>(row0) * a.ks_sp + h * a.ks_sh));
        const uint32_t off = static_cast<uint32_t>(si * static_cast<int>(a.ks_sp) * 4);
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
      } else if (si < 2 * KT) {
        const uint8_t* base = uniform_ptr(reinterpret_cast<const uint8_t*>(
            a.vs + blk * a.vs_sn + static_cast<int64_t>(row0) * a.vs_sp + h * a.vs_sh));
        const uint32_t off = static_cast<uint32_t>((si - KT) * static_cast<int>(a.vs_sp) * 4);
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
      }
    } else {
      if (tid < 2 * KT) reinterpret_cast<float*>(st + 2 * kPayload)[tid] = 1.f;
    }
  };

  floatx4 acc[kPfColBlocks][8];
  float m_run[kPfColBlocks], l_run[kPfColBlocks];
#pragma unroll
  for (int cb = 0; cb < kPfColBlocks; ++cb) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[cb][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    m_run[cb] = -INFINITY;
    l_run[cb] = 0.f;
  }

  // per-lane LDS offsets inside a stage for sub-block 0 (add 16 rows per sub-block)
  const uint32_t k_off0 = c * kRow + (((2 * g) ^ pf_swz(c)) << 4);
  const uint32_t k_off1 = c * kRow + (((2 * g + 1) ^ pf_swz(c)) << 4);
  uint32_t v_off[4];
  {
    const int r = c >> 1;
    const int t = 4 * g + (r & 3);
    const int half = c & 1;
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const int chunk = 2 * jp + (r >> 2);
      v_off[jp] = kPayload + t * kRow + ((chunk ^ pf_swz(t)) << 4) + half * 8;
    }
  }
  const uint32_t stage_base = lds_addr(stages);
  const int qpos0 = prefix + qb0;  // position of query column 0 of block 0

  issue_tile(0, stages);
  bool cur_ok = tile_ok;
  __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const bool more = t + 1 < ntiles;
    // the next tile streams into the other stage, last read by tile t - 1,
    // which every wave finished before the barrier that ended that iteration
    bool next_ok = true;
    if (more) {
      issue_tile(t + 1, stages + ((t + 1) & 1) * kStage);
      next_ok = tile_ok;
    }
    const uint32_t soff = static_cast<uint32_t>(t & 1) * kStage;
    const uint8_t* st = stages + soff;
    if (cur_ok) {
#pragma unroll
      for (int sp = 0; sp < KT / kStep; ++sp) {
        const int key0 = t * KT + sp * kStep;                // first key of the step
        if (key0 > qpos0 + kPfQTile - 1) break;              // above the diagonal for every column
        // per 16-key block b: K rows, scales and the transposed V reads
        u32x4 kw[NB][2];
        floatx4 ksv[NB];
        uint64_t vt[NB][4];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int sb = sp * NB + b;
          const uint8_t* sbp = st + sb * 16 * kRow;
          kw[b][0] = *reinterpret_cast<const u32x4*>(sbp + k_off0);
          kw[b][1] = *reinterpret_cast<const u32x4*>(sbp + k_off1);
          const float* scl = reinterpret_cast<const float*>(st + 2 * kPayload) + sb * 16 + 4 * g;
          ksv[b] = *reinterpret_cast<const floatx4*>(scl);
        }
        {
          uint32_t ad[4];
#pragma unroll
          for (int jp = 0; jp < 4; ++jp) ad[jp] = stage_base + soff + v_off[jp];
          if constexpr (NB == 2) {
            if (sp == 0) lds_read_tr8_x8<0, 16 * kRow>(ad, vt[0], vt[NB - 1]);
            else lds_read_tr8_x8<2 * 16 * kRow, 3 * 16 * kRow>(ad, vt[0], vt[NB - 1]);
          } else {
#pragma unroll
            for (int jp = 0; jp < 4; ++jp) ad[jp] += sp * 16 * kRow;
            lds_read_tr8_x4(ad, vt[0]);
          }
        }
        // keys past the context end may hold any bytes: zero them in V (only
        // the context's last step can hold such keys; uniform branch)
        if (key0 + kStep > ctx) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            uint32_t keep = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) keep |= (key0 + 16 * b + 4 * g + i < ctx) ? (0xFFu << (8 * i)) : 0u;
            const uint64_t keep2 = static_cast<uint64_t>(keep) | (static_cast<uint64_t>(keep) << 32);
#pragma unroll
            for (int jp = 0; jp < 4; ++jp) vt[b][jp] &= keep2;
          }
        }
        // S^T = K Q^T for both column blocks, NB x 2 independent chains
        floatx4 sc[kPfColBlocks][NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          if constexpr (QDT == PRISM_DTYPE_F16) {
            // K converted once per block for both column blocks
            f16x8 kop[4];
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
              const u32x4& w = kw[b][cc >> 1];
              kop[cc] = fp8x8_to_f16x8(w[(cc & 1) * 2], w[(cc & 1) * 2 + 1]);
            }
#pragma unroll
            for (int cb = 0; cb < kPfColBlocks; ++cb) {
              floatx4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int cc = 0; cc < 4; ++cc) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[cc], qop[cb].op[cc], d, 0, 0, 0);
              sc[cb][b] = d;
            }
          } else {
            // the K bytes are the fp8 MFMA's A operand as they are (row =
            // key c of the block, k = dims 32g..32g+31); smaller term first
            const i32x8 ka = {static_cast<int>(kw[b][0][0]), static_cast<int>(kw[b][0][1]),
                              static_cast<int>(kw[b][0][2]), static_cast<int>(kw[b][0][3]),
                              static_cast<int>(kw[b][1][0]), static_cast<int>(kw[b][1][1]),
                              static_cast<int>(kw[b][1][2]), static_cast<int>(kw[b][1][3])};
#pragma unroll
            for (int cb = 0; cb < kPfColBlocks; ++cb) {
              floatx4 d = {0.f, 0.f, 0.f, 0.f};
              d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qop[cb].t[1], d, 0, 0, 0, 0, 0, 0);
              d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, qop[cb].t[0], d, 0, 0, 0, 0, 0, 0);
              sc[cb][b] = d;
            }
          }
        }
        // online softmax per column block -> P (A of O = P V).  One block:
        // k-slots 4g..4g+3 are keys 4g..4g+3 (16x16x16).  Two blocks: k-slots
        // 8g..8g+3 are keys 4g..4g+3 of block 0 and 8g+4..8g+7 the same keys
        // of block 1 (16x16x32), the order the score rows come out in.
        // Both column blocks go through each phase together (one branch per
        // phase), so their dependency chains interleave.
        POp pa[kPfColBlocks];
        float x[kPfColBlocks][NB][4];
#pragma unroll
        for (int cb = 0; cb < kPfColBlocks; ++cb)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[cb][b][i] = sc[cb][b][i] * ksv[b][i];  // score / softmax scale
        // causal mask: key k is visible to column c iff it is at or before
        // the query's position.  Steps wholly below the diagonal of both
        // column blocks need no mask (uniform branch); columns without a
        // query hold q = 0 there, so their scores stay finite and their rows
        // are never written.
        if (key0 + kStep - 1 > qpos0) {
#pragma unroll
          for (int cb = 0; cb < kPfColBlocks; ++cb) {
            const int qpos = qpos0 + cb * kPfCols + c;
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                x[cb][b][i] = (colv[cb] && key0 + 16 * b + 4 * g + i <= qpos) ? x[cb][b][i] : -INFINITY;
          }
        }
        float tmax[kPfColBlocks];
        bool raise[kPfColBlocks];
#pragma unroll
        for (int cb = 0; cb < kPfColBlocks; ++cb) {
          float t = fmaxf(fmaxf(x[cb][0][0], x[cb][0][1]), fmaxf(x[cb][0][2], x[cb][0][3]));
          if constexpr (NB == 2) t = fmaxf(t, fmaxf(fmaxf(x[cb][1][0], x[cb][1][1]), fmaxf(x[cb][1][2], x[cb][1][3])));
          tmax[cb] = wave_max_across_groups(t) * qop[cb].mul;  // log2 units (the multiplier is positive)
          raise[cb] = tmax[cb] > m_run[cb] + kPfRescaleThreshold;
        }
        if (__builtin_amdgcn_ballot_w64(raise[0] || raise[1]) != 0) {
#pragma unroll
          for (int cb = 0; cb < kPfColBlocks; ++cb) {
            const float m_new = raise[cb] ? tmax[cb] : m_run[cb];
            const float alpha = raise[cb] ? __builtin_amdgcn_exp2f(m_run[cb] - m_new) : 1.f;
            m_run[cb] = m_new;
            l_run[cb] *= alpha;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float ai = __shfl(alpha, 4 * g + i);
#pragma unroll
              for (int j = 0; j < 8; ++j) acc[cb][j][i] *= ai;
            }
          }
        }
        // v scales are read here, where P is formed, not with the K scales:
        // held across the QK MFMAs they push the kernel past 256 VGPRs
        floatx4 vsv[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
          vsv[b] = *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(st + 2 * kPayload) + KT +
                                                     (sp * NB + b) * 16 + 4 * g);
#pragma unroll
        for (int cb = 0; cb < kPfColBlocks; ++cb) {
          const float m_use = (m_run[cb] == -INFINITY) ? 0.f : m_run[cb];
          float p[NB][4];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              // v_exp_f32: arguments are at most 2^3 above the running max;
              // results below 2^-126 (flushed to 0) weigh nothing next to it
              p[b][i] = __builtin_amdgcn_exp2f(fmaf(x[cb][b][i], qop[cb].mul, -m_use));  // 0 where masked
              if constexpr (NB == 2) pa[cb][4 * b + i] = static_cast<__bf16>(p[b][i] * vsv[b][i]);
              else pa[cb][4 * b + i] = __builtin_bit_cast(short, static_cast<__bf16>(p[b][i] * vsv[b][i]));
            }
          }
          float ps = (p[0][0] + p[0][1]) + (p[0][2] + p[0][3]);
          if constexpr (NB == 2) ps += (p[1][0] + p[1][1]) + (p[1][2] + p[1][3]);
          l_run[cb] += ps;
        }
        // O += P V: V operand (B) for dims 16 j + c, one N-tile at a time,
        // shared by the column blocks; k-slots as P's
#pragma unroll
        for (int jp = 0; jp < 4; ++jp) {
#pragma unroll
          for (int hi = 0; hi < 2; ++hi) {
            const int j = 2 * jp + hi;
            const uint32_t w0 = static_cast<uint32_t>(vt[0][jp] >> (32 * hi));
            if constexpr (NB == 2) {
              const bf16x8 vb = fp8x8_to_bf16x8(w0, static_cast<uint32_t>(vt[NB - 1][jp] >> (32 * hi)));
#pragma unroll
              for (int cb = 0; cb < kPfColBlocks; ++cb)
                acc[cb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[cb], vb, acc[cb][j], 0, 0, 0);
            } else {
              const shortx4 v0 = fp8x4_to_bf16x4_bits(w0);
#pragma unroll
              for (int cb = 0; cb < kPfColBlocks; ++cb)
                acc[cb][j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[cb], v0, acc[cb][j], 0, 0, 0);
            }
          }
        }
      }
    }
    cur_ok = next_ok;
    __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): this wave's part of tile t + 1 has landed
    __syncthreads();
  }

  // ---- epilogue: acc[cb][j][i] is query column 4g + i of block cb, dim 16j + c
#pragma unroll
  for (int cb = 0; cb < kPfColBlocks; ++cb) {
    float l_tot = l_run[cb] + __shfl_xor(l_run[cb], 16);
    l_tot += __shfl_xor(l_tot, 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qr = 4 * g + i;
      const float li = __shfl(l_tot, qr);
      const int j = qb0 + cb * kPfCols + qr;
      if (j < qlen) {
        const float inv = li > 0.f ? 1.f / li : 0.f;
        uint16_t* dst = static_cast<uint16_t*>(a.out) + static_cast<int64_t>(qs + j) * a.o_st +
                        static_cast<int64_t>(qhead) * a.o_sh + c;
#pragma unroll
        for (int jd = 0; jd < 8; ++jd) {
          const float o = acc[cb][jd][i] * inv;
          dst[16 * jd] = (QDT == PRISM_DTYPE_F16) ? f32_to_f16_bits(o) : f32_to_bf16_bits(o);
        }
      }
    }
  }
}

template <int QDT, int KT, int NW>
int launch_prefill(const PrefillArgs& a, bool scaled, int total_q, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(total_q, kPfQTile) + a.batch),
                  static_cast<unsigned>(a.num_heads / a.groups));
  const dim3 block(64 * NW);
  if (scaled) hipLaunchKernelGGL((paged_prefill_kernel<QDT, KT, NW, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((paged_prefill_kernel<QDT, KT, NW, false>), grid, block, 0, stream, a);
  return check_launch("paged_prefill_kernel launch");
}

// Key tiles of 64, 32 or 16 keys (the largest dividing the page; at most 32
// for one or two waves); one wave per query head of the GQA group.
template <int QDT, int KT>
int dispatch_waves(const PrefillArgs& a, bool scaled, int total_q, hipStream_t stream) {
  switch (a.groups) {
    case 1: return launch_prefill<QDT, (KT > 32 ? 32 : KT), 1>(a, scaled, total_q, stream);
    case 2: return launch_prefill<QDT, (KT > 32 ? 32 : KT), 2>(a, scaled, total_q, stream);
    case 4: return launch_prefill<QDT, KT, 4>(a, scaled, total_q, stream);
    case 8: return launch_prefill<QDT, KT, 8>(a, scaled, total_q, stream);
    default:
      set_error("prism_paged_prefill: GQA group size %d is not 1, 2, 4 or 8", a.groups);
      return PRISM_ERR_LAYOUT;
  }
}

template <int QDT>
int dispatch_tile(const PrefillArgs& a, bool scaled, int total_q, hipStream_t stream) {
  // a tile lies in one page
  if (a.page % 64 == 0) return dispatch_waves<QDT, 64>(a, scaled, total_q, stream);
  if (a.page % 32 == 0) return dispatch_waves<QDT, 32>(a, scaled, total_q, stream);
  return dispatch_waves<QDT, 16>(a, scaled, total_q, stream);
}

}  // namespace

// Loads this file's code object now rather than at its first kernel launch.
int preload_paged_prefill() {
  hipFuncAttributes attr;
  return check_hip(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&paged_prefill_kernel<PRISM_DTYPE_BF16, 64, 4, true>)), "preload_paged_prefill");
}

}  // namespace prism

extern "C" int prism_paged_prefill(const void* q, int q_dtype, const int64_t q_strides[3], const void* k_cache,
                                   const void* v_cache, int cache_dtype, const int64_t k_strides[4],
                                   const int64_t v_strides[4], const float* k_scale, const float* v_scale,
                                   const int64_t k_scale_strides[3], const int64_t v_scale_strides[3],
                                   const int32_t* block_tables, const int64_t bt_strides[2],
                                   const int32_t* context_lens, const int32_t* cu_seqlens_q, void* out,
                                   const int64_t out_strides[3], int batch, int total_q, int num_heads,
                                   int num_kv_heads, int head_dim, int page_size, int num_blocks, int width,
                                   float scale, int32_t* status, void* stream_ptr) {
  using namespace prism;
  clear_error();
  if (batch < 0 || total_q < 0 || num_heads <= 0 || num_kv_heads <= 0 || page_size <= 0 || num_blocks < 0 ||
      width < 0) {
    set_error("prism_paged_prefill: invalid geometry");
    return PRISM_ERR_INVALID;
  }
  if (num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > kPfMaxWaves) {
    set_error("prism_paged_prefill: num_heads=%d / num_kv_heads=%d must be an integer group of at most %d",
              num_heads, num_kv_heads, kPfMaxWaves);
    return PRISM_ERR_LAYOUT;
  }
  if (head_dim != kPfD) {
    set_error("prism_paged_prefill: head_dim must be %d, got %d", kPfD, head_dim);
    return PRISM_ERR_LAYOUT;
  }
  if (cache_dtype != PRISM_DTYPE_FP8_E4M3FN) {
    set_error("prism_paged_prefill: the cache must be FP8 E4M3FN (dtype code %d)", cache_dtype);
    return PRISM_ERR_LAYOUT;
  }
  if (q_dtype != PRISM_DTYPE_BF16 && q_dtype != PRISM_DTYPE_F16) {
    set_error("prism_paged_prefill: q must be bf16 or float16 (dtype code %d)", q_dtype);
    return PRISM_ERR_LAYOUT;
  }
  if (page_size % 16 != 0) {
    set_error("prism_paged_prefill: page size must be a multiple of 16, got %d", page_size);
    return PRISM_ERR_LAYOUT;
  }
  if ((k_scale == nullptr) != (v_scale == nullptr)) {
    set_error("prism_paged_prefill: K/V scale caches must be provided together");
    return PRISM_ERR_INVALID;
  }
  if (!q_strides || !k_strides || !v_strides || !bt_strides || !out_strides || !status ||
      (k_scale && (!k_scale_strides || !v_scale_strides))) {
    set_error("prism_paged_prefill: null argument");
    return PRISM_ERR_INVALID;
  }
  if (q_strides[2] != 1 || k_strides[3] != 1 || v_strides[3] != 1 || out_strides[2] != 1 ||
      !aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || q_strides[0] % 8 || q_strides[1] % 8 ||
      k_strides[0] % 16 || k_strides[1] % 16 || k_strides[2] % 16 || v_strides[0] % 16 || v_strides[1] % 16 ||
      v_strides[2] % 16) {
    set_error("prism_paged_prefill: q, K/V and out need unit-stride head dims and 16-byte aligned rows");
    return PRISM_ERR_LAYOUT;
  }
  // tile loads address a page's rows of one head by a 32-bit offset
  if ((page_size - 1) * k_strides[1] + kPfD > INT32_MAX || (page_size - 1) * v_strides[1] + kPfD > INT32_MAX ||
      (k_scale && ((page_size - 1) * k_scale_strides[1] >= INT32_MAX / 4 ||
                   (page_size - 1) * v_scale_strides[1] >= INT32_MAX / 4))) {
    set_error("prism_paged_prefill: a page's token rows must span less than 2 GiB");
    return PRISM_ERR_LAYOUT;
  }
  if (batch == 0 || total_q == 0) return PRISM_OK;
  PrefillArgs a{};
  a.q = q;
  a.q_st = q_strides[0];
  a.q_sh = q_strides[1];
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.k_sn = k_strides[0], a.k_sp = k_strides[1], a.k_sh = k_strides[2];
  a.v_sn = v_strides[0], a.v_sp = v_strides[1], a.v_sh = v_strides[2];
  a.ks = k_scale;
  a.vs = v_scale;
  if (k_scale) {
    a.ks_sn = k_scale_strides[0], a.ks_sp = k_scale_strides[1], a.ks_sh = k_scale_strides[2];
    a.vs_sn = v_scale_strides[0], a.vs_sp = v_scale_strides[1], a.vs_sh = v_scale_strides[2];
  }
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sn = bt_strides[1];
  a.ctx = context_lens;
  a.cu_q = cu_seqlens_q;
  a.out = out;
  a.o_st = out_strides[0];
  a.o_sh = out_strides[1];
  a.batch = batch;
  a.num_heads = num_heads;
  a.groups = num_heads / num_kv_heads;
  a.page = page_size;
  a.num_blocks = num_blocks;
  a.width = width;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.status = status;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const bool scaled = k_scale != nullptr;
  if (q_dtype == PRISM_DTYPE_F16) return dispatch_tile<PRISM_DTYPE_F16>(a, scaled, total_q, stream);
  return dispatch_tile<PRISM_DTYPE_BF16>(a, scaled, total_q, stream);
}
