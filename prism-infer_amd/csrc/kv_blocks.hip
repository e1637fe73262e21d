// Whole-block KV moves between two paged caches of the same layout, one of
// which may live in pinned host memory (swap out / swap in).  A block is
// `block_bytes` contiguous bytes in each of `rows` rows ([kv, layer] pairs)
// whose pitch is the cache's bytes per row, so one strided DMA copy
// (hipMemcpy2DAsync) moves a block of every row at once; no kernel and no
// staging.  Block moves inside one device cache go through the compaction
// kernels instead (all reads before writes).
#include "common.h"

#include <algorithm>

extern "C" int prism_copy_blocks(void* dst, const void* src, int64_t rows, int64_t dst_row_pitch,
                                 int64_t src_row_pitch, int64_t block_bytes, int64_t dst_blocks,
                                 int64_t src_blocks, const int64_t* dst_ids, const int64_t* src_ids, int64_t n,
                                 void* stream_ptr) {
  prism::clear_error();
  if (n < 0 || rows <= 0 || block_bytes <= 0 || dst_blocks <= 0 || src_blocks <= 0) {
    prism::set_error("prism_copy_blocks: invalid sizes (rows=%lld block_bytes=%lld n=%lld)",
                     static_cast<long long>(rows), static_cast<long long>(block_bytes), static_cast<long long>(n));
    return PRISM_ERR_INVALID;
  }
  if (dst_row_pitch < dst_blocks * block_bytes || src_row_pitch < src_blocks * block_bytes) {
    prism::set_error("prism_copy_blocks: row pitch smaller than blocks * block_bytes");
    return PRISM_ERR_INVALID;
  }
  if (n == 0) return PRISM_OK;
  if (!dst || !src || !dst_ids || !src_ids) {
    prism::set_error("prism_copy_blocks: null pointer");
    return PRISM_ERR_INVALID;
  }
  for (int64_t i = 0; i < n; ++i) {
    if (dst_ids[i] < 0 || dst_ids[i] >= dst_blocks || src_ids[i] < 0 || src_ids[i] >= src_blocks) {
      prism::set_error("prism_copy_blocks: entry %lld: block ids (%lld -> %lld) out of range", static_cast<long long>(i),
                       static_cast<long long>(src_ids[i]), static_cast<long long>(dst_ids[i]));
      return PRISM_ERR_INVALID;
    }
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  for (int64_t i = 0; i < n; ++i) {
    uint8_t* d = static_cast<uint8_t*>(dst) + dst_ids[i] * block_bytes;
    const uint8_t* s = static_cast<const uint8_t*>(src) + src_ids[i] * block_bytes;
    int rc = prism::check_hip(hipMemcpy2DAsync(d, static_cast<size_t>(dst_row_pitch), s,
                                               static_cast<size_t>(src_row_pitch), static_cast<size_t>(block_bytes),
                                               static_cast<size_t>(rows), hipMemcpyDefault, stream),
                              "prism_copy_blocks: hipMemcpy2DAsync");
    if (rc) return rc;
  }
  return PRISM_OK;
}

// Streaming device-to-device copy: the read + write ceiling that the store
// and compaction kernels are measured against (each touches every byte once,
// as this copy does).  A grid of `workgroups_per_cu` workgroups per CU walks
// the buffer in trips of kCopyUnroll 16-byte chunks per lane, all loads of a
// trip issued before its stores, with the non-temporal policy on both sides.
namespace prism {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 8;

__global__ void __launch_bounds__(kCopyThreads)
stream_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src, int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kCopyThreads;
  const int64_t trip = stride * kCopyUnroll;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kCopyThreads + threadIdx.x;
  for (; i + (kCopyUnroll - 1) * stride < n16; i += trip) {  // whole trips
    u32x4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) __builtin_nontemporal_store(v[u], dst + i + u * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace
}  // namespace prism

extern "C" int prism_device_copy(void* dst, const void* src, int64_t nbytes, int workgroups_per_cu,
                                 void* stream_ptr) {
  prism::clear_error();
  if (nbytes < 0 || (nbytes % 16) != 0 || workgroups_per_cu < 1 || workgroups_per_cu > 64) {
    prism::set_error("prism_device_copy: nbytes must be a non-negative multiple of 16 and workgroups_per_cu in "
                     "[1, 64] (got %lld, %d)", static_cast<long long>(nbytes), workgroups_per_cu);
    return PRISM_ERR_INVALID;
  }
  if (!prism::aligned(dst, 16) || !prism::aligned(src, 16)) {
    prism::set_error("prism_device_copy: dst and src must be 16-byte aligned");
    return PRISM_ERR_LAYOUT;
  }
  if (nbytes == 0) return PRISM_OK;
  const int64_t n16 = nbytes / 16;
  const int64_t want = static_cast<int64_t>(prism::device_cu_count()) * workgroups_per_cu;
  const int blocks = static_cast<int>(std::max<int64_t>(1, std::min(want, prism::ceil_div(n16, prism::kCopyThreads))));
  hipLaunchKernelGGL(prism::stream_copy_kernel, dim3(blocks), dim3(prism::kCopyThreads), 0,
                     static_cast<hipStream_t>(stream_ptr), static_cast<prism::u32x4*>(dst),
                     static_cast<const prism::u32x4*>(src), n16);
  return prism::check_launch("stream_copy_kernel launch");
}
