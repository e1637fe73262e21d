// Physical slot compaction: cache[row, dst[i], :] <- cache[row, src[i], :]
// for every row, with all reads before any write (the semantics of
// prism_infer/ops/kv_compaction.py:93-112: index_select(...).clone() then
// index_copy_).
//
// The reference always stages every slot through a temporary (two Triton
// passes, :157-191).  Here the device decides per call whether staging is
// needed, in four launches and no host synchronisation:
//   1. mark: every source slot's tag (one uint32 per slot in the workspace)
//      gets this call's epoch;
//   2. detect: if some entry's destination is tagged (another entry's
//      source; src == dst entries are no-ops), the hazard word gets the epoch;
//   3. move: hazard word != epoch -> copy every entry src -> dst directly;
//      otherwise gather the sources into the workspace's temporary;
//   4. scatter (hazard word == epoch only): temporary -> destinations.
// Nothing needs clearing: tags and the hazard word are compared with the
// call's epoch, a value that differs from call to call and from the small
// integers recycled memory often holds; a stale value that matches by chance
// only makes the call stage, which gives the same bytes.  Copies move 16
// bytes per lane when the row width allows it, 4 or 1 bytes otherwise.
#include "common.h"

#include <algorithm>
#include <atomic>

namespace prism {
namespace {

constexpr int kThreads = 256;
#ifndef PRISM_MOVE_WG_PER_CU
#define PRISM_MOVE_WG_PER_CU 4
#endif
#ifndef PRISM_MOVE_UNROLL
#define PRISM_MOVE_UNROLL 4
#endif
// Move grid: workgroups per CU (over all rows) and chunks in flight per lane.
// Config 5's payload + scale calls, cold, with the pipelined slot indices:
// 4 / 4 321 us; 8 / 4 346, 4 / 8 331, 2 / 8 334, 1 / 8 344 us (the loop
// without the pipelining, 8 / 4: 338 us; 1 / 8: 650 us).
constexpr int kMoveWgPerCu = PRISM_MOVE_WG_PER_CU;
constexpr int kMoveUnroll = PRISM_MOVE_UNROLL;

// Workspace: tags (one uint32 per slot), the hazard word, the temporary.
int64_t workspace_layout(int64_t rows, int64_t num_slots, int64_t vec_bytes, int64_t retained, int64_t* flag_off,
                         int64_t* temp_off) {
  *flag_off = align_up(num_slots * 4, 256);
  *temp_off = *flag_off + 256;
  return *temp_off + align_up(rows * retained * vec_bytes, 256);
}

// This call's tag value: a process-wide counter passed through a bijective
// 32-bit mixer, so that consecutive calls' tags are far apart and unlike the
// small integers recycled memory often holds (a tag that matches by chance
// only costs staging); never 0.
unsigned int next_compaction_epoch() {
  static std::atomic<unsigned int> counter{0};
  for (;;) {
    uint32_t x = counter.fetch_add(1, std::memory_order_relaxed) + 0x9E3779B9u;
    x ^= x >> 16;
    x *= 0x7FEB352Du;
    x ^= x >> 15;
    x *= 0x846CA68Bu;
    x ^= x >> 16;
    if (x != 0u) return x;
  }
}

__global__ void __launch_bounds__(kThreads)
mark_sources_kernel(const int64_t* __restrict__ src, int64_t retained, int64_t num_slots,
                    uint32_t* __restrict__ tags, uint32_t epoch) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < retained;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t s = src[i];
    if (s >= 0 && s < num_slots) tags[s] = epoch;
  }
}

// Whether entry (s, d) moves anything.
__device__ __forceinline__ bool entry_live(int64_t s, int64_t d, int64_t num_slots) {
  return s >= 0 && s < num_slots && d >= 0 && d < num_slots && s != d;
}

__global__ void __launch_bounds__(kThreads)
detect_hazard_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t retained,
                     int64_t num_slots, const uint32_t* __restrict__ tags, uint32_t* __restrict__ flag,
                     uint32_t epoch) {
  bool hazard = false;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < retained;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t s = src[i];
    const int64_t d = dst[i];
    if (entry_live(s, d, num_slots) && tags[d] == epoch) hazard = true;
  }
  if (__any(hazard) && lane_id() == 0) *flag = epoch;  // every writer stores the same value
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

// MODE 0: hazard word != epoch -> direct copy src -> dst; else gather src -> temp
// MODE 2: scatter temp -> dst (only when the hazard word == epoch)
//
// Grid (x: chunk ranges, y: rows).  Chunk c of a row is part c & (U - 1) of
// entry c >> USHIFT when a row vector holds U = 2^USHIFT chunks (every
// canonical shape: token rows of 1024 or 32 bytes, whole blocks), else
// c / U and c % U (USHIFT < 0).  Each thread moves kMoveUnroll chunks per
// trip with all loads issued before the stores, and every byte is read and
// written once, so both go through the non-temporal cache policy.  The
// entries' slot indices are software-pipelined: a trip's data loads go out
// with the next trip's index loads behind them, so the only round trip per
// trip is the data's (the index loads of a trip would otherwise precede its
// data loads as a second, dependent one).
template <int BYTES, int MODE>
__global__ void __launch_bounds__(kThreads)
compact_move_kernel(uint8_t* __restrict__ cache, int64_t num_slots, int64_t vec_bytes, int ushift,
                    const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t retained,
                    uint8_t* __restrict__ temp, const uint32_t* __restrict__ flag, uint32_t epoch) {
  using T = typename Chunk<BYTES>::T;
  const bool staged = *flag == epoch;
  if (MODE == 2 && !staged) return;
  const int64_t chunks_per_vec = vec_bytes / BYTES;
  const int64_t per_row = retained * chunks_per_vec;
  const int64_t row = blockIdx.y;
  const int64_t row_base = row * num_slots;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  auto entry_of = [&](int64_t c, int64_t& i, int64_t& part) {
    if (ushift >= 0) {
      i = c >> ushift;
      part = c & (chunks_per_vec - 1);
    } else {
      i = c / chunks_per_vec;
      part = c - i * chunks_per_vec;
    }
  };
  // slot indices of a trip's chunks (-1: past the end)
  int64_t s[kMoveUnroll], d[kMoveUnroll];
  auto load_indices = [&](int64_t b) {
#pragma unroll
    for (int u = 0; u < kMoveUnroll; ++u) {
      const int64_t c = b + u * stride;
      int64_t i, part;
      entry_of(c, i, part);
      const bool in = c < per_row;
      s[u] = in ? src[i] : -1;
      d[u] = in ? dst[i] : -1;
    }
  };
  int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (base < per_row) load_indices(base);
  for (; base < per_row; base += kMoveUnroll * stride) {
    T val[kMoveUnroll];
    T* to[kMoveUnroll];
    bool ok[kMoveUnroll];
#pragma unroll
    for (int u = 0; u < kMoveUnroll; ++u) {
      const int64_t c = base + u * stride;
      int64_t i, part;
      entry_of(c, i, part);
      ok[u] = entry_live(s[u], d[u], num_slots);
      T* tmp = reinterpret_cast<T*>(temp + (row * retained + i) * vec_bytes) + part;
      T* direct = reinterpret_cast<T*>(cache + (row_base + d[u]) * vec_bytes) + part;
      const T* from = MODE == 0 ? reinterpret_cast<const T*>(cache + (row_base + s[u]) * vec_bytes) + part : tmp;
      to[u] = (MODE == 0 && staged) ? tmp : direct;
      if (ok[u]) val[u] = __builtin_nontemporal_load(from);
    }
    const int64_t next = base + kMoveUnroll * stride;
    if (next < per_row) load_indices(next);
#pragma unroll
    for (int u = 0; u < kMoveUnroll; ++u)
      if (ok[u]) __builtin_nontemporal_store(val[u], to[u]);
  }
}

int grid_for(int64_t work, int64_t cap) {
  int64_t g = ceil_div(work, kThreads);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<int>(g);
}

// Launches both passes of one kernel family over the rows, in chunks of the
// grid.y limit.
template <typename Launch>
int launch_passes(int64_t rows, Launch&& launch) {
  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
      launch(pass, r0, std::min<int64_t>(rows - r0, 65535));
      if (int rc = check_launch(pass == 0 ? "compact move launch" : "compact scatter launch")) return rc;
    }
  }
  return PRISM_OK;
}

template <int BYTES>
int launch_moves(uint8_t* cache, int64_t rows, int64_t num_slots, int64_t vec_bytes, const int64_t* src,
                 const int64_t* dst, int64_t retained, uint8_t* temp, const uint32_t* flag, uint32_t epoch,
                 hipStream_t stream) {
  const int64_t chunks_per_vec = vec_bytes / BYTES;
  int ushift = -1;
  if ((chunks_per_vec & (chunks_per_vec - 1)) == 0) {
    ushift = 0;
    while ((int64_t{1} << ushift) < chunks_per_vec) ++ushift;
  }
  const int64_t per_row = retained * chunks_per_vec;
  const int64_t cap = std::max<int64_t>(1, device_cu_count() * kMoveWgPerCu / std::max<int64_t>(rows, 1));
  const int gx = grid_for(ceil_div(per_row, kMoveUnroll), cap);
  return launch_passes(rows, [&](int pass, int64_t r0, int64_t nr) {
    uint8_t* c = cache + r0 * num_slots * vec_bytes;
    uint8_t* t = temp + r0 * retained * vec_bytes;
    const dim3 grid(gx, static_cast<unsigned>(nr));
    if (pass == 0)
      hipLaunchKernelGGL((compact_move_kernel<BYTES, 0>), grid, dim3(kThreads), 0, stream, c, num_slots, vec_bytes,
                         ushift, src, dst, retained, t, flag, epoch);
    else
      hipLaunchKernelGGL((compact_move_kernel<BYTES, 2>), grid, dim3(kThreads), 0, stream, c, num_slots, vec_bytes,
                         ushift, src, dst, retained, t, flag, epoch);
  });
}

}  // namespace

// Loads this file's code object now rather than at its first kernel launch.
int preload_kv_compaction() {
  hipFuncAttributes attr;
  return check_hip(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&mark_sources_kernel)),
                   "preload_kv_compaction");
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
  uint32_t* tags = reinterpret_cast<uint32_t*>(ws);
  uint32_t* flag = reinterpret_cast<uint32_t*>(ws + flag_off);
  uint8_t* temp = ws + temp_off;
  const uint32_t epoch = next_compaction_epoch();
  const int grid = grid_for(retained, device_cu_count() * 8);
  // 1. mark the sources, 2. detect hazards
  hipLaunchKernelGGL(mark_sources_kernel, dim3(grid), dim3(kThreads), 0, stream, src, retained, num_slots, tags, epoch);
  if (int rc = check_launch("compact mark launch")) return rc;
  hipLaunchKernelGGL(detect_hazard_kernel, dim3(grid), dim3(kThreads), 0, stream, src, dst, retained, num_slots, tags,
                     flag, epoch);
  if (int rc = check_launch("compact detect launch")) return rc;
  // 3./4. move, then scatter when staged
  uint8_t* c = static_cast<uint8_t*>(cache);
  if (vec_bytes % 16 == 0 && aligned(cache, 16))
    return launch_moves<16>(c, rows, num_slots, vec_bytes, src, dst, retained, temp, flag, epoch, stream);
  if (vec_bytes % 4 == 0 && aligned(cache, 4))
    return launch_moves<4>(c, rows, num_slots, vec_bytes, src, dst, retained, temp, flag, epoch, stream);
  return launch_moves<1>(c, rows, num_slots, vec_bytes, src, dst, retained, temp, flag, epoch, stream);
}
