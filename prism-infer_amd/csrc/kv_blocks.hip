// Whole-block KV moves between two paged caches of the same layout, one of
// which may live in pinned host memory (swap out / swap in).  A block is
// `block_bytes` contiguous bytes in each of `rows` rows ([kv, layer] pairs)
// whose pitch is the cache's bytes per row, so one strided DMA copy
// (hipMemcpy2DAsync) moves a block of every row at once; no kernel and no
// staging.  Block moves inside one device cache go through the compaction
// kernels instead (all reads before writes).
#include "common.h"

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
