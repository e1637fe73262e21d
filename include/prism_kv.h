/*
 * prism_kv.h -- C ABI of libprism_mi355x.so, the MI355X (gfx950) scaled-FP8
 * paged-KV hot path.
 *
 * Conventions
 *   - Every entry point returns PRISM_OK (0) on success or a negative status;
 *     prism_last_error() then returns a thread-local message.
 *   - Pointers are device pointers (already including storage offsets) unless
 *     stated otherwise.  Strides are in ELEMENTS of the pointed-to type.
 *   - `stream` is a hipStream_t passed as void*; all work is enqueued on it and
 *     no call synchronises the host.  Nothing here allocates or frees device
 *     memory: scratch comes in through a caller-owned `workspace`.
 *   - Device-side metadata (slot_mapping, block tables, context lengths,
 *     max_context_len) is read by the kernels at run time, so a call captured
 *     into a HIP graph follows updated contents on replay.
 *
 * dtype codes (PRISM_DTYPE_*) name the element type of a buffer.
 */
#ifndef PRISM_KV_H
#define PRISM_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRISM_OK 0
#define PRISM_ERR_INVALID (-1) /* contract violation (shape, dtype, size)   */
#define PRISM_ERR_LAYOUT (-2)  /* unsupported layout / alignment / stride   */
#define PRISM_ERR_HIP (-3)     /* a HIP runtime call failed                 */
#define PRISM_ERR_BUSY (-4)    /* a shared resource is in use by a running call */

#define PRISM_DTYPE_F32 0
#define PRISM_DTYPE_BF16 1
#define PRISM_DTYPE_F16 2
#define PRISM_DTYPE_FP8_E4M3FN 3

/* ABI version of this header (bumped on any signature change). */
int prism_abi_version(void);

/* Message for the most recent failing call on this thread ("" if none). */
const char* prism_last_error(void);

/* Number of compute units of the current device (used for work sizing). */
int prism_device_cu_count(void);

/*
 * Load every kernel's code object on the current device now (HIP otherwise
 * loads a code object at the first launch of one of its kernels, which stalls
 * that call for tens of milliseconds).  No counterpart in the reference (its
 * Triton kernels compile on first call); for hosts that want the first
 * decode step to run at speed.  Returns PRISM_OK or PRISM_ERR_HIP.
 */
int prism_preload(void);

/*
 * KV store.  Replaces the kernels behind
 *   store_kvcache(key, value, k_cache, v_cache, slot_mapping,
 *                 k_scale_cache=None, v_scale_cache=None)
 *   (prism_infer/ops/kv_cache_store.py:419-476; scaled kernel :81-167,
 *    dense kernel :58-78, eager semantics :170-230).
 *
 * key/value   : [num_tokens, num_heads, head_dim] of in_dtype (F32/BF16/F16);
 *               strides {token, head, dim}; head and dim must be dense
 *               (stride_dim == 1, stride_head == head_dim).
 * k/v_cache   : contiguous [num_slots, num_heads, head_dim] of cache_dtype.
 * k/v_scale   : contiguous [num_slots, num_heads] fp32, or both NULL.
 *               Non-NULL requires cache_dtype == FP8_E4M3FN and selects the
 *               per-token, per-head scaled quantiser:
 *                 s = max(amax|x| / 448, 1e-6);  q = e4m3fn(clamp(x / s, +-448))
 *               NULL with an FP8 cache stores a unit-scale RNE cast; NULL with
 *               a F32/BF16/F16 cache stores a plain cast.
 * slot_mapping: int32 [num_tokens]; slot < 0 (padding) and slot >= num_slots
 *               are skipped.
 */
int prism_kv_store(const void* key, const void* value, int in_dtype, const int64_t key_strides[3],
                   const int64_t value_strides[3], void* k_cache, void* v_cache, int cache_dtype,
                   float* k_scale, float* v_scale, const int32_t* slot_mapping, int64_t num_tokens,
                   int num_heads, int head_dim, int64_t num_slots, void* stream);

/*
 * Paged decode attention (one query token per sequence, GQA).  Replaces the
 * kernel behind
 *   paged_decode_attention(q, k_cache, v_cache, block_tables, context_lens,
 *                          scale, *, k_scale_cache=None, v_scale_cache=None,
 *                          max_context_len=None, block_n=32)
 *   (prism_infer/ops/paged_decode.py:443-485; kernel :42-180).
 *
 * q          : [batch, num_heads, head_dim] of q_dtype (F32/BF16/F16), strides q_strides.
 * k/v_cache  : [num_blocks, page_size, num_kv_heads, head_dim] of cache_dtype
 *              (FP8_E4M3FN, or F32/BF16/F16 for unscaled caches), strides
 *              k_strides / v_strides {block, token, head, dim}; dim stride 1.
 * k/v_scale  : [num_blocks, page_size, num_kv_heads] fp32 or both NULL;
 *              strides ks_strides / vs_strides.
 * block_tables: int32 [>= batch, max_blocks_per_seq], strides bt_strides.
 *              Block ids < 0 (and >= num_blocks) are skipped, not errors.
 * context_lens: int32 [>= batch]; max_context_len: int32 [1].  A token t of
 *              sequence b is attended iff t < min(context_lens[b],
 *              *max_context_len, max_blocks_per_seq * page_size) and its block
 *              id is valid.  A sequence with no attended token outputs zeros.
 * out        : [batch, num_heads, head_dim] of q_dtype, strides out_strides.
 * workspace  : device scratch of at least prism_paged_decode_workspace_bytes()
 *              bytes for the same geometry; may be NULL when that function
 *              returns 0.  It holds split-K partials with their arrival
 *              counters (tagged per call, so leftovers of any other call or
 *              use count as zero) and, for the streaming kernel, two work
 *              plans (prefix-sharing groups, tile ranges), each with the
 *              inputs it was computed from, behind a plan word; a call whose
 *              block tables and context lengths equal those of the current
 *              plan reuses it, otherwise one workgroup of the call builds the
 *              other plan and publishes it.  Any initial contents are valid.
 *              Calls that share a workspace must be ordered on one stream.
 */
int64_t prism_paged_decode_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim,
                                           int page_size, int max_blocks_per_seq, int cache_dtype);

int prism_paged_decode(const void* q, int q_dtype, const int64_t q_strides[3], const void* k_cache,
                       const void* v_cache, int cache_dtype, const int64_t k_strides[4],
                       const int64_t v_strides[4], const float* k_scale, const float* v_scale,
                       const int64_t ks_strides[3], const int64_t vs_strides[3],
                       const int32_t* block_tables, const int64_t bt_strides[2],
                       const int32_t* context_lens, const int32_t* max_context_len, void* out,
                       const int64_t out_strides[3], int batch, int num_heads, int num_kv_heads,
                       int head_dim, int page_size, int64_t num_blocks, int max_blocks_per_seq,
                       float scale, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Allocation-free paged decode.  NO COUNTERPART IN THE REFERENCE: for callers
 * that cannot allocate device memory or pass a workspace (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).
 * Same arguments, semantics and results as prism_paged_decode minus the
 * workspace: the library keeps a file-scope 64 MiB (67,108,864-byte) scratch
 * array per GPU (held until the process ends) and uses it as the workspace.
 * A geometry whose prism_paged_decode_workspace_bytes() exceeds 64 MiB is
 * rejected with PRISM_ERR_INVALID (e.g. B = 256 at 32k tokens needs about
 * 36 MiB and fits).  Calls no hipMalloc, hipFree or allocating library
 * routine.  Every call on one GPU shares that GPU's scratch, so calls must
 * not overlap on one GPU.  The entry point refuses, with PRISM_ERR_BUSY, a
 * call on another stream while the previous call's kernels have not
 * finished (checked with an event recorded behind each call; the event is
 * created with the scratch's address on the device's first call).  Calls on
 * the same stream are ordered by the stream and always accepted.  Launches
 * recorded under graph capture are not checked: replays of a captured graph
 * that overlap other calls on the same GPU race.
 */
int prism_paged_decode_noalloc(const void* q, int q_dtype, const int64_t q_strides[3],
                               const void* k_cache, const void* v_cache, int cache_dtype,
                               const int64_t k_strides[4], const int64_t v_strides[4],
                               const float* k_scale, const float* v_scale,
                               const int64_t ks_strides[3], const int64_t vs_strides[3],
                               const int32_t* block_tables, const int64_t bt_strides[2],
                               const int32_t* context_lens, const int32_t* max_context_len, void* out,
                               const int64_t out_strides[3], int batch, int num_heads, int num_kv_heads,
                               int head_dim, int page_size, int64_t num_blocks, int max_blocks_per_seq,
                               float scale, void* stream);

/*
 * Stage selector for measurement: the same as prism_paged_decode but runs only
 * one part of it.  stage 0 runs everything and is identical to
 * prism_paged_decode; stage 1 runs the decode kernel (every family is one
 * launch that merges its own partials and, for the streaming kernel, checks
 * and if needed builds its plan, so stage 1 is the whole decode and stage 2
 * launches nothing); stage 3 only builds the streaming kernel's plan in the
 * workspace, as a separate one-workgroup launch (nothing for the other
 * kernels).
 */
int prism_paged_decode_stage(int stage, const void* q, int q_dtype, const int64_t q_strides[3],
                             const void* k_cache, const void* v_cache, int cache_dtype,
                             const int64_t k_strides[4], const int64_t v_strides[4],
                             const float* k_scale, const float* v_scale,
                             const int64_t ks_strides[3], const int64_t vs_strides[3],
                             const int32_t* block_tables, const int64_t bt_strides[2],
                             const int32_t* context_lens, const int32_t* max_context_len,
                             void* out, const int64_t out_strides[3], int batch, int num_heads,
                             int num_kv_heads, int head_dim, int page_size, int64_t num_blocks,
                             int max_blocks_per_seq, float scale, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* Tokens per split-K work item chosen for a geometry (0 = no split-K path). */
int prism_paged_decode_split_tokens(int batch, int num_heads, int num_kv_heads, int head_dim,
                                    int page_size, int max_blocks_per_seq, int cache_dtype);

/*
 * Kernel family a scaled-FP8 geometry selects: 0 generic, 1 per-split (split-K
 * partials + combine), 2 streaming (tile-balanced persistent kernel + merge).
 * Family 2 additionally needs the canonical dense cache layout at call time
 * (otherwise family 1 runs).  A forced family (see below) applies where the
 * geometry allows it.
 */
int prism_paged_decode_kernel_family(int batch, int num_heads, int num_kv_heads, int head_dim,
                                     int page_size, int max_blocks_per_seq, int cache_dtype);

/*
 * Process-wide kernel-family overrides (no counterpart in the reference, whose
 * Triton op has one kernel; used by tests to run every family on the same
 * inputs).  path: 0 automatic, 1 per-split, 2 streaming; split_tokens: 0
 * automatic, else tokens per split (rounded up to 32); share: 1 analyse
 * shared prefixes on the device, 0 treat every page as private.  Initial
 * values come from PRISM_DECODE_PATH / PRISM_DECODE_SPLIT / PRISM_DECODE_SHARE,
 * read once at the first call.  No override skips work or changes results
 * beyond the decode tolerance.
 */
int prism_paged_decode_set_overrides(int path, int split_tokens, int share);
void prism_paged_decode_get_overrides(int out[3]);

/*
 * Test hook of the streaming decode kernel's plan wait (no counterpart in the
 * reference).  A workgroup that waits for another workgroup's plan build
 * gives up after `polls` polls (default prism_paged_decode_default_plan_wait_limit(),
 * far beyond any build); it then writes NaN to the call's output rows and
 * counts the give-up in the workspace's plan header, which makes the next
 * call rebuild the plan.  Setting 0 makes every waiting workgroup give up at
 * once, so the path can be exercised from the host with kernels that all
 * exit normally.  Returns the previous limit, or -1 for polls < 0.
 */
int prism_paged_decode_set_plan_wait_limit(int polls);
int prism_paged_decode_default_plan_wait_limit(void);

/*
 * Physical slot compaction.  Replaces the kernels behind
 *   compact_kv_slots(cache, source_slots, destination_slots)
 *   (prism_infer/ops/kv_compaction.py:93-112; gather/scatter kernels :33-86).
 *
 * cache      : contiguous [rows, num_slots, vec_bytes] bytes (a payload cache
 *              [kv, layers, slots, heads, dim] or a scale cache
 *              [kv, layers, slots, heads] viewed as bytes).
 * src, dst   : int64 [retained] slot indices.  Semantics: every destination
 *              slot receives the bytes its source slot held BEFORE the call
 *              (all reads precede all writes), for every row.  Entries whose
 *              source or destination is outside [0, num_slots) are skipped.
 *              Duplicate destinations leave which source wins unspecified.
 * workspace  : prism_compact_slots_workspace_bytes() bytes of device scratch.
 *              The library detects on the device whether any destination
 *              aliases a different entry's source; only then does it stage
 *              the sources through the workspace (two passes), otherwise it
 *              copies in one pass.
 */
int64_t prism_compact_slots_workspace_bytes(int64_t rows, int64_t num_slots, int64_t vec_bytes,
                                            int64_t retained);

int prism_compact_slots(void* cache, int64_t rows, int64_t num_slots, int64_t vec_bytes,
                        const int64_t* src, const int64_t* dst, int64_t retained, void* workspace,
                        int64_t workspace_bytes, void* stream);

/*
 * Whole-block moves between two caches of the same layout, either of which may
 * be pinned host memory.  Replaces the per-block copies of
 *   ModelRunner.swap_blocks(swap_map, direction)
 *   (prism_infer/engine/model_runner.py:1001-1031).
 *
 * dst, src    : caches viewed as [rows][row_pitch bytes]; block i of a row is
 *               the block_bytes bytes at i * block_bytes (a [kv, layers,
 *               blocks, ...] cache has rows = kv * layers and row_pitch =
 *               blocks * block_bytes).
 * dst_ids, src_ids : HOST int64 [n] block ids, each in [0, dst_blocks) or
 *               [0, src_blocks); entry i copies block src_ids[i] of every row
 *               to block dst_ids[i] (one strided async DMA copy per entry, in
 *               entry order).  Host memory must be pinned (page-locked).
 */
int prism_copy_blocks(void* dst, const void* src, int64_t rows, int64_t dst_row_pitch, int64_t src_row_pitch,
                      int64_t block_bytes, int64_t dst_blocks, int64_t src_blocks, const int64_t* dst_ids,
                      const int64_t* src_ids, int64_t n, void* stream);

/*
 * Streaming device-to-device copy of nbytes (a multiple of 16; both pointers
 * 16-byte aligned) with `workgroups_per_cu` workgroups per CU (1-64),
 * non-temporal 16-byte loads and stores, eight in flight per lane.  NO
 * COUNTERPART IN THE REFERENCE: it is the measured read + write ceiling that
 * the store and compaction kernels, which touch every byte once, are
 * compared with.  Returns PRISM_OK, PRISM_ERR_INVALID or PRISM_ERR_LAYOUT.
 */
int prism_device_copy(void* dst, const void* src, int64_t nbytes, int workgroups_per_cu, void* stream);

/*
 * Paged prefill attention (chunked / prefix-hit prefill) over paged FP8
 * K/V.  Replaces
 *   paged_prefill_attention_reference(q, k_cache, v_cache, context, *,
 *       num_heads, num_kv_heads, scale, k_scale_cache=None, v_scale_cache=None)
 *   (prism_infer/ops/paged_attention_reference.py:185-246).
 *
 * q          : [total_q, num_heads, head_dim] of q_dtype (BF16/F16), strides
 *              q_strides {token, head, dim}; dim stride 1, rows 16-byte aligned.
 *              Sequence i owns rows [cu_seqlens_q[i], cu_seqlens_q[i + 1]).
 * k/v_cache  : [num_blocks, page_size, num_kv_heads, head_dim] FP8_E4M3FN,
 *              strides k_strides / v_strides {block, token, head, dim}; dim
 *              stride 1.  head_dim 128; page_size a multiple of 16; GQA group
 *              num_heads / num_kv_heads of 1, 2, 4 or 8.
 * k/v_scale  : [num_blocks, page_size, num_kv_heads] fp32 or both NULL (unit
 *              scale); strides ks_strides / vs_strides.
 * block_tables, context_lens, cu_seqlens_q : int32 device arrays ([>= batch,
 *              width], [>= batch], [>= batch + 1]).  context_lens[i] counts the
 *              sequence's whole history including its query tokens, which are
 *              already stored in the cache; query token j of sequence i sits
 *              at position context_lens[i] - query_len_i + j and attends to
 *              keys 0 .. that position.
 * out        : [total_q, num_heads, head_dim] of q_dtype, strides out_strides.
 * status     : device int32[1], set by the caller to INT32_MAX.  A sequence
 *              whose lengths are invalid (query_len <= 0, context_len <
 *              query_len, context_len > width * page_size) or whose needed
 *              block ids are negative or >= num_blocks records its index
 *              there (atomic min); its output rows are unspecified.
 */
int prism_paged_prefill(const void* q, int q_dtype, const int64_t q_strides[3], const void* k_cache,
                        const void* v_cache, int cache_dtype, const int64_t k_strides[4],
                        const int64_t v_strides[4], const float* k_scale, const float* v_scale,
                        const int64_t ks_strides[3], const int64_t vs_strides[3],
                        const int32_t* block_tables, const int64_t bt_strides[2],
                        const int32_t* context_lens, const int32_t* cu_seqlens_q, void* out,
                        const int64_t out_strides[3], int batch, int total_q, int num_heads,
                        int num_kv_heads, int head_dim, int page_size, int num_blocks, int width,
                        float scale, int32_t* status, void* stream);

/*
 * Test hook with no counterpart in the reference: converts n fp32 values to
 * E4M3FN bytes with the exact device routine the scaled store uses (native
 * gfx950 conversion plus the NaN rule), so the rounding can be checked
 * exhaustively against the CPU oracle.
 */
int prism_debug_fp8_encode(const float* in, uint8_t* out, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PRISM_KV_H */
