// Physical slot compaction: cache[row, dst[i], :] <- cache[row, src[i], :]
// for every row, with all reads before any write (the semantics of
// prism_infer/ops/kv_compaction.py:93-112: index_select(...).clone() then
// index_copy_).
//
// The reference always stages through a temporary (two Triton passes,
// :157-191).  Here the device decides per call whether staging is needed:
//   1. clear a bitmap over all slots and a hazard flag (fill kernel; graph safe),
//   2. mark every source slot in the bitmap,
//   3. raise the flag if some entry writes a slot that is another entry's
//      source (dst[i] marked and dst[i] != src[i]),
//   4. copy: flag clear -> move bytes directly src -> dst (one pass);
//            flag set   -> gather sources into the workspace,
//   5. scatter (flag set only): workspace -> dst.
// No host synchronisation; the flag lives in device memory.  Copies move 16
// bytes per lane when the row width allows it, 4 or 1 bytes otherwise.
#include "common.h"

#include <algorithm>

namespace prism {
namespace {

constexpr int kThreads = 256;

struct CompactWorkspace {
  uint32_t* bitmap;   // ceil(num_slots / 32) words
  uint32_t* flag;     // [0] hazard flag
  uint8_t* temp;      // rows * retained * vec_bytes
};

int64_t bitmap_words(int64_t num_slots) { return ceil_div(num_slots, 32); }

int64_t workspace_layout(int64_t rows, int64_t num_slots, int64_t vec_bytes, int64_t retained,
                         int64_t* flag_off, int64_t* temp_off) {
  const int64_t bm = align_up(bitmap_words(num_slots) * 4, 256);
  *flag_off = bm;
  *temp_off = bm + 256;
  return *temp_off + align_up(rows * retained * vec_bytes, 256);
}

__global__ void __launch_bounds__(kThreads) clear_words_kernel(uint32_t* __restrict__ words, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    words[i] = 0u;
}

// Sources of one wave that fall in the same bitmap word (plans list kept
// slots in runs, so a wave usually touches two or three words) are OR-ed
// together first: one atomic per distinct word instead of one per entry.
__global__ void __launch_bounds__(kThreads)
mark_sources_kernel(const int64_t* __restrict__ src, int64_t retained, int64_t num_slots,
                    uint32_t* __restrict__ bitmap) {
  const int lane = lane_id();
  const int64_t wave0 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) - lane;
  for (int64_t base = wave0; base < retained; base += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = base + lane;
    const int64_t sl = i < retained ? src[i] : -1;
    const bool valid = sl >= 0 && sl < num_slots;
    const int64_t w = valid ? (sl >> 5) : -1;
    const uint32_t bit = valid ? (1u << (sl & 31)) : 0u;
    uint64_t todo = __builtin_amdgcn_ballot_w64(valid);
    while (todo != 0) {  // wave-uniform loop
      const int leader = __builtin_ctzll(todo);
      const int64_t lw = __shfl(w, leader);
      const bool mine = valid && w == lw;
      uint32_t v = mine ? bit : 0u;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) v |= __shfl_xor(v, off);
      if (lane == leader) atomicOr(&bitmap[lw], v);
      todo &= ~__builtin_amdgcn_ballot_w64(mine);
    }
  }
}

__global__ void __launch_bounds__(kThreads)
detect_hazard_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t retained,
                     int64_t num_slots, const uint32_t* __restrict__ bitmap, uint32_t* __restrict__ flag) {
  bool hazard = false;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < retained;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t s = src[i];
    const int64_t d = dst[i];
    if (s < 0 || s >= num_slots || d < 0 || d >= num_slots || s == d) continue;
    if ((bitmap[d >> 5] >> (d & 31)) & 1u) hazard = true;
  }
  if (__any(hazard) && lane_id() == 0) atomicOr(flag, 1u);
}

// Element type used for the byte moves.
template <int BYTES>
struct Chunk;
template <>
struct Chunk<16> { using T = u32x4; };
template <>
struct Chunk<4> { using T = uint32_t; };
template <>
struct Chunk<1> { using T = uint8_t; };

// MODE 0: flag clear -> direct copy src -> dst; flag set -> gather src -> temp
// MODE 2: scatter temp -> dst (only when the flag is set)
//
// Grid (x: chunk ranges, y: rows).  Chunk c of a row is part c & (U - 1) of
// entry c >> USHIFT when a row vector holds U = 2^USHIFT chunks (every
// canonical shape: token rows of 1024 or 32 bytes, whole blocks), else
// c / U and c % U (USHIFT < 0).  Each thread moves four chunks per trip with
// the four loads issued before the stores, and every byte is read and
// written once, so both go through the non-temporal cache policy.
template <int BYTES, int MODE>
__global__ void __launch_bounds__(kThreads)
compact_move_kernel(uint8_t* __restrict__ cache, int64_t num_slots, int64_t vec_bytes, int ushift,
                    const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t retained,
                    uint8_t* __restrict__ temp, const uint32_t* __restrict__ flag) {
  using T = typename Chunk<BYTES>::T;
  const bool staged = *flag != 0u;
  if (MODE == 2 && !staged) return;
  const int64_t chunks_per_vec = vec_bytes / BYTES;
  const int64_t per_row = retained * chunks_per_vec;
  const int64_t row = blockIdx.y;
  const int64_t row_base = row * num_slots;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  constexpr int kUnroll = 4;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; base < per_row;
       base += kUnroll * stride) {
    T val[kUnroll];
    T* to[kUnroll];
    bool ok[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = base + u * stride;
      int64_t i, part;
      if (ushift >= 0) {
        i = c >> ushift;
        part = c & (chunks_per_vec - 1);
      } else {
        i = c / chunks_per_vec;
        part = c - i * chunks_per_vec;
      }
      ok[u] = c < per_row;
      const int64_t s = ok[u] ? src[i] : -1;
      const int64_t d = ok[u] ? dst[i] : -1;
      ok[u] = ok[u] && s >= 0 && s < num_slots && d >= 0 && d < num_slots;
      const int64_t item = row * retained + i;
      const T* from;
      if (MODE == 0) {
        from = reinterpret_cast<const T*>(cache + (row_base + s) * vec_bytes) + part;
        to[u] = staged ? reinterpret_cast<T*>(temp + item * vec_bytes) + part
                       : reinterpret_cast<T*>(cache + (row_base + d) * vec_bytes) + part;
      } else {
        from = reinterpret_cast<const T*>(temp + item * vec_bytes) + part;
        to[u] = reinterpret_cast<T*>(cache + (row_base + d) * vec_bytes) + part;
      }
      if (ok[u]) val[u] = __builtin_nontemporal_load(from);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (ok[u]) __builtin_nontemporal_store(val[u], to[u]);
  }
}

int grid_for(int64_t work, int64_t cap) {
  int64_t g = ceil_div(work, kThreads);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<int>(g);
}

template <int BYTES>
int launch_moves(uint8_t* cache, int64_t rows, int64_t num_slots, int64_t vec_bytes, const int64_t* src,
                 const int64_t* dst, int64_t retained, uint8_t* temp, const uint32_t* flag,
                 hipStream_t stream) {
  const int64_t chunks_per_vec = vec_bytes / BYTES;
  int ushift = -1;
  if ((chunks_per_vec & (chunks_per_vec - 1)) == 0) {
    ushift = 0;
    while ((int64_t{1} << ushift) < chunks_per_vec) ++ushift;
  }
  const int64_t per_row = retained * chunks_per_vec;
  // about 8 workgroups per CU in total, spread over the rows
  const int64_t cap = std::max<int64_t>(1, device_cu_count() * 8 / std::max<int64_t>(rows, 1));
  const int gx = grid_for(ceil_div(per_row, 4), cap);
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {  // grid.y limit
    const int64_t nr = std::min<int64_t>(rows - r0, 65535);
    uint8_t* c = cache + r0 * num_slots * vec_bytes;
    uint8_t* t = temp + r0 * retained * vec_bytes;
    const dim3 grid(gx, static_cast<unsigned>(nr));
    hipLaunchKernelGGL((compact_move_kernel<BYTES, 0>), grid, dim3(kThreads), 0, stream, c, num_slots, vec_bytes,
                       ushift, src, dst, retained, t, flag);
    int rc = check_launch("compact copy/gather launch");
    if (rc) return rc;
  }
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
    const int64_t nr = std::min<int64_t>(rows - r0, 65535);
    uint8_t* c = cache + r0 * num_slots * vec_bytes;
    uint8_t* t = temp + r0 * retained * vec_bytes;
    const dim3 grid(gx, static_cast<unsigned>(nr));
    hipLaunchKernelGGL((compact_move_kernel<BYTES, 2>), grid, dim3(kThreads), 0, stream, c, num_slots, vec_bytes,
                       ushift, src, dst, retained, t, flag);
    int rc = check_launch("compact scatter launch");
    if (rc) return rc;
  }
  return PRISM_OK;
}

}  // namespace

// Loads this file's code object now rather than at its first kernel launch.
int preload_kv_compaction() {
  hipFuncAttributes attr;
  return check_hip(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&clear_words_kernel)), "preload_kv_compaction");
}

}  // namespace prism

extern "C" int64_t prism_compact_slots_workspace_bytes(int64_t rows, int64_t num_slots, int64_t vec_bytes,
                                                       int64_t retained) {
  if (rows < 0 || num_slots < 0 || vec_bytes < 0 || retained < 0) return -1;
  int64_t f, t;
  return prism::workspace_layout(rows, num_slots, vec_bytes, retained, &f, &t);
}

extern "C" int prism_compact_slots(void* cache, int64_t rows, int64_t num_slots, int64_t vec_bytes,
                                   const int64_t* src, const int64_t* dst, int64_t retained,
                                   void* workspace, int64_t workspace_bytes, void* stream_ptr) {
  using namespace prism;
  clear_error();
  if (rows < 0 || num_slots < 0 || vec_bytes <= 0 || retained < 0) {
    set_error("prism_compact_slots: invalid geometry rows=%lld slots=%lld vec_bytes=%lld retained=%lld",
              static_cast<long long>(rows), static_cast<long long>(num_slots),
              static_cast<long long>(vec_bytes), static_cast<long long>(retained));
    return PRISM_ERR_INVALID;
  }
  if (retained == 0 || rows == 0 || num_slots == 0) return PRISM_OK;
  if (!cache || !src || !dst || !workspace) {
    set_error("prism_compact_slots: null pointer argument");
    return PRISM_ERR_INVALID;
  }
  int64_t flag_off, temp_off;
  const int64_t need = workspace_layout(rows, num_slots, vec_bytes, retained, &flag_off, &temp_off);
  if (workspace_bytes < need) {
    set_error("prism_compact_slots: workspace too small (%lld < %lld bytes)",
              static_cast<long long>(workspace_bytes), static_cast<long long>(need));
    return PRISM_ERR_INVALID;
  }
  if (!aligned(workspace, 256)) {
    set_error("prism_compact_slots: workspace must be 256-byte aligned");
    return PRISM_ERR_LAYOUT;
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(ws);
  uint32_t* flag = reinterpret_cast<uint32_t*>(ws + flag_off);
  uint8_t* temp = ws + temp_off;
  const int cap = device_cu_count() * 8;

  // 1. clear bitmap and flag (the flag word sits right after the bitmap's
  //    256-byte aligned extent, so one fill covers both).
  const int64_t clear_words = flag_off / 4 + 1;
  hipLaunchKernelGGL(clear_words_kernel, dim3(grid_for(clear_words, cap)), dim3(kThreads), 0, stream, bitmap,
                     clear_words);
  int rc = check_launch("compact clear launch");
  if (rc) return rc;
  // 2. mark sources, 3. detect hazards
  hipLaunchKernelGGL(mark_sources_kernel, dim3(grid_for(retained, cap)), dim3(kThreads), 0, stream, src,
                     retained, num_slots, bitmap);
  if ((rc = check_launch("compact mark launch"))) return rc;
  hipLaunchKernelGGL(detect_hazard_kernel, dim3(grid_for(retained, cap)), dim3(kThreads), 0, stream, src, dst,
                     retained, num_slots, bitmap, flag);
  if ((rc = check_launch("compact detect launch"))) return rc;
  // 4./5. moves
  uint8_t* c = static_cast<uint8_t*>(cache);
  if (vec_bytes % 16 == 0 && aligned(cache, 16))
    return launch_moves<16>(c, rows, num_slots, vec_bytes, src, dst, retained, temp, flag, stream);
  if (vec_bytes % 4 == 0 && aligned(cache, 4))
    return launch_moves<4>(c, rows, num_slots, vec_bytes, src, dst, retained, temp, flag, stream);
  return launch_moves<1>(c, rows, num_slots, vec_bytes, src, dst, retained, temp, flag, stream);
}
