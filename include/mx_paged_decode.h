/*
 * mx_paged_decode.h -- C ABI of the MI355X (gfx950) paged GQA decode attention library
 * (libmxattn.so).
 *
 * Operator (reference task.md:138-148): for every sequence b, query token i < seqlen_q and
 * query head h,
 *   kv      = h / (num_heads / num_kv_heads)
 *   keys    = the first L = seq_lens[b] tokens of sequence b; token t lives in physical page
 *             block_table[b, t / page_size] at in-page offset t % page_size.  With causal = 1
 *             query token i sees only keys t < L - seqlen_q + i + 1 (the causal mask aligned to
 *             the end of the cache, as flash_attn_with_kvcache does for the reference's
 *             seqlen_q / causal arguments, task.md:47, 53); a query row that sees no key is
 *             written as zeros, as is every row of an empty sequence (L <= 0).
 *   out[b,i,h,:] = softmax(q[b,i,h,:] . K[keys,kv,:]^T * scale) . V[keys,kv,:]
 *
 * Layouts (all contiguous, row-major):
 *   q, out       [batch, seqlen_q, num_heads, head_dim]  bf16  (seqlen_q == 1 is the decode step)
 *   k/v cache    [num_pages, page_size, num_kv_heads, head_dim]  bf16
 *   seq_lens     [batch]                                  int32
 *   block_table  [batch, max_pages_per_seq]               int32
 * Only the first ceil(seq_lens[b] / page_size) entries of a block_table row are read; the
 * padding entries after them are never touched (reference task.md:8-10, 61, 92).
 *
 * Supported shapes: head_dim in {64, 128, 256}; page_size in {16, 32, 64, 128, 256};
 * num_heads % num_kv_heads == 0 and num_heads / num_kv_heads <= 128; seqlen_q >= 1 with
 * batch * seqlen_q <= 65535; causal 0 or 1.  The seqlen_q * (num_heads / num_kv_heads) query
 * rows of one KV head are processed in groups of 16 rows (32 when there are more than 16 and
 * head_dim <= 128): every further group streams that head's K/V once more.
 *
 * Every call is asynchronous on the given stream (NULL = the legacy default stream) and never
 * synchronises.  Calls that share one workspace (including the library's internal one) must
 * be ordered on one stream.
 */
#ifndef MX_PAGED_DECODE_H
#define MX_PAGED_DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by the int-returning entry points (also kept for mx_last_status()). */
#define MX_STATUS_OK 0
#define MX_STATUS_NULL_POINTER (-1)         /* a required pointer is NULL                    */
#define MX_STATUS_INVALID_SHAPE (-2)        /* sizes inconsistent (e.g. Hq % Hkv != 0)       */
#define MX_STATUS_UNSUPPORTED (-3)          /* valid but not implemented (D, page size, ...) */
#define MX_STATUS_WORKSPACE_TOO_SMALL (-4)  /* caller workspace smaller than required        */
#define MX_STATUS_HIP_ERROR (-5)            /* HIP runtime reported an error                 */
#define MX_STATUS_ALLOC_FAILED (-6)         /* internal workspace allocation failed          */
#define MX_STATUS_INVALID_ARGUMENT (-7)     /* bad non-shape argument (phase, scale, ...)    */

/* Bits of the device status word (sticky; read with mx_read_device_status). */
#define MX_DEVICE_BAD_PAGE_ID 1u    /* a valid block_table slot held an id outside [0, num_pages) */
#define MX_DEVICE_SEQ_TOO_LONG 2u   /* seq_lens[b] exceeded the capacity the call was planned for */
#define MX_DEVICE_WORKSPACE_STATE 4u /* the workspace's counter region was not zero at launch (a
                                        workspace not zero-filled, or shared by overlapping calls):
                                        that call's output is not valid                         */

/* Schedules reported by mx_paged_gqa_decode_plan. */
#define MX_SCHEDULE_SPLIT_GRID 0   /* grid (Hkv * row groups, batch, splits); the splits of
                                      each unit merge through an in-kernel tree of arrival
                                      counters, or, when splits > 4096 or batch * Hkv * row
                                      groups * ceil(splits / 8) > 12288, in a combine kernel
                                      that follows                                                */
#define MX_SCHEDULE_BALANCED 1     /* one launch of a fixed number of workgroups that divide the
                                      batch's K/V chunks evenly from seq_lens on the device and
                                      merge split sequences themselves                            */
#define MX_SCHEDULE_SPLIT_GRID_PAIRED 2 /* the split grid over pairs of adjacent KV heads, two
                                      waves of each workgroup per head: automatic plans on bf16
                                      and fp8 caches, head_dim 128, an even num_kv_heads >= 8,
                                      2 * seqlen_q * group <= 16, and splits of >= 896 tokens     */
#define MX_SCHEDULE_BALANCED_PAIRED 3 /* the balanced schedule over pairs of adjacent KV heads,
                                      on the same shapes as MX_SCHEDULE_SPLIT_GRID_PAIRED, and
                                      on fp8 caches also with 4 or 6 KV heads when the pairs of
                                      the batch are at least the workgroups; on bf16 caches of
                                      4 KV heads, pairs of heads 0 and 3, 1 and 2 when the
                                      pairs of the batch outnumber the workgroups               */

/* Phase flags for mx_paged_gqa_decode (0 = run everything). */
#define MX_PHASE_MAIN_ONLY 1        /* split grid: run only the split-KV kernel, partials stay in
                                       the workspace (balanced schedule: the whole call)          */
#define MX_PHASE_COMBINE_ONLY 2     /* split grid: run only the combine over the partials of an
                                       identical MAIN_ONLY call (balanced schedule: nothing)      */

/*
 * Drop-in replacement for the reference's C500 kernel entry point, same name, argument order
 * and meaning: reference task.md:38-54, implementation submission_clean.cu:432-447, bound by
 * verify_real.py:12-14 / bench_all.py:98-100 as argtypes [c_void_p]*6 + [c_int64]*9.
 *   - scale is derived as 1/sqrt(headdim) (submission_clean.cu:451);
 *   - block_table row width = num_blocks / batch_size (submission_clean.cu:449, task.md:61);
 *   - the K/V pools hold num_blocks pages (task.md:57-58): page ids outside [0, num_blocks)
 *     are flagged (MX_DEVICE_BAD_PAGE_ID) and read as page 0, where the reference reads
 *     outside the pool;
 *   - seqlen_k is the capacity used for split planning (task.md:7, 131);
 *   - launches on the legacy default stream, no synchronisation (task.md:67);
 *   - uses a library-owned, grow-only workspace per device (submission_clean.cu:478-491);
 *   - seqlen_q >= 1 and causal (0 or 1) are honoured with the operator semantics above (the
 *     reference fixes them at 1 and 0, task.md:64, 66, and its kernel ignores them).
 * Returns nothing, as the reference does; on invalid arguments nothing is launched, a message
 * is printed to stderr and the status is kept for mx_last_status() / mx_last_error().
 */
void run_kernel(const void* q, const void* k_cache_paged, const void* v_cache_paged,
                void* output, const int32_t* cache_seqlens, const int32_t* block_table,
                int64_t batch_size, int64_t seqlen_k, int64_t seqlen_q, int64_t num_heads,
                int64_t num_heads_k, int64_t headdim, int64_t page_block_size,
                int64_t num_blocks, int64_t causal);

/*
 * Extended entry point (replaces the same run_kernel, submission_clean.cu:432-504, with an
 * explicit scale, table width, pool size, split override, workspace and stream, and a status).
 *   seqlen_q           query tokens per sequence (1 = decode).
 *   num_pages          pool size; page ids outside [0, num_pages) are flagged and read as page 0.
 *                      0 = unknown (only negative ids are flagged).
 *   max_pages_per_seq  block_table row width.
 *   max_seq_len        capacity the split plan is sized for (<= 0: max_pages_per_seq*page_size).
 *                      seq_lens[b] beyond the planned capacity (max_seq_len rounded up to whole
 *                      splits, at most max_pages_per_seq*page_size) are clamped and flagged
 *                      (MX_DEVICE_SEQ_TOO_LONG).
 *   causal             0, or 1 for the end-aligned causal mask of multi-token queries.
 *   num_splits         0 = automatic: the balanced schedule when batch <= 512,
 *                      64 <= units <= 8192 (units = batch * num_kv_heads * query row
 *                      groups; a row group is 16 rows, or 32 when seqlen_q * num_heads /
 *                      num_kv_heads > 16 and head_dim <= 128) and the capacity is at least
 *                      2048 tokens (1024 with 512+ units); else the split grid with a
 *                      CU-count-driven split count (1, or 4+ splits of >= 128 tokens);
 *                      > 0 = split grid with that many splits per sequence (clamped to the
 *                      number of pages of max_seq_len);
 *                      < 0 = balanced schedule with exactly -num_splits workgroups.
 *   workspace          device memory of >= mx_paged_gqa_decode_workspace_size() bytes,
 *                      zero-filled once by the caller before first use (its first 229 632
 *                      bytes hold a status word, workgroup claim masks and merge counters
 *                      that every call leaves at zero); NULL = library-owned: one per device, grown on demand
 *                      (doubling; earlier allocations are kept, never freed, so graphs
 *                      captured with them stay valid).  A call that needs it to grow fails
 *                      with MX_STATUS_INVALID_ARGUMENT on a capturing stream.
 *   phase              0, MX_PHASE_MAIN_ONLY or MX_PHASE_COMBINE_ONLY.
 *   stream             hipStream_t (NULL = legacy default stream).
 * q, k_cache and v_cache must be 16-byte aligned and out 8-byte aligned (MX_STATUS_INVALID_ARGUMENT
 * otherwise).
 * Returns MX_STATUS_OK or a negative MX_STATUS_* code; nothing is launched on error.
 */
int mx_paged_gqa_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                        const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                        int64_t seqlen_q, int64_t num_heads, int64_t num_kv_heads,
                        int64_t head_dim, int64_t page_size, int64_t num_pages,
                        int64_t max_pages_per_seq, int64_t max_seq_len, int32_t causal,
                        float scale, int64_t num_splits, void* workspace, int64_t workspace_bytes,
                        int32_t phase, void* stream);

/*
 * mx_paged_gqa_decode for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  No counterpart in the
 * reference.  Arguments as mx_paged_gqa_decode (phase 0), without a workspace: the call uses a
 * library-owned device array of MX_NOALLOC_SCRATCH_BYTES per GPU, which the HIP runtime places
 * on each device when the library's code is first loaded there and holds until the process
 * ends.  The call never allocates (no hipMalloc, hipFree or allocating library routine); the
 * first call on a device also launches a clear of the array's status word and counters on
 * `stream`, ahead of its decode.  A call whose mx_paged_gqa_decode_workspace_size exceeds
 * MX_NOALLOC_SCRATCH_BYTES is rejected with MX_STATUS_UNSUPPORTED before anything is launched.
 * Every such call on one GPU shares that GPU's array: calls that overlap in time on one GPU
 * (different streams without ordering, or different host threads) race on it, so order them
 * on one stream.  The device status flags of these calls (a bad page id read as page 0, a
 * sequence clamped to the capacity) go to the array's own status word, which
 * mx_read_device_status reads when passed MX_NOALLOC_WORKSPACE; it is sticky until read with
 * reset != 0.  Returns MX_STATUS_*.
 */
#define MX_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
/* The workspace argument of mx_read_device_status that names the current device's no-alloc
 * array (a sentinel, never dereferenced as a host or device address). */
#define MX_NOALLOC_WORKSPACE ((void*)(intptr_t)-1)
int mx_paged_gqa_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                void* out, const int32_t* seq_lens, const int32_t* block_table,
                                int64_t batch, int64_t seqlen_q, int64_t num_heads,
                                int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_pages, int64_t max_pages_per_seq,
                                int64_t max_seq_len, int32_t causal, float scale,
                                int64_t num_splits, void* stream);

/*
 * The decode over an fp8 K/V cache: k_cache and v_cache hold OCP e4m3fn bytes (torch
 * float8_e4m3fn) in the same [num_pages, page_size, num_kv_heads, head_dim] layout, and the
 * keys and values are k_scale and v_scale times the stored values (per-tensor scales, as in
 * vLLM's fp8 KV cache).  q and out stay bf16; every other argument is as mx_paged_gqa_decode's.
 * The kernels read half the bytes of a bf16 cache and widen the values to bf16 in registers
 * (exact: every e4m3fn value is a bf16 value) before the same MFMA path.  k_scale and v_scale
 * must be finite.
 * With head_dim 64, an even num_kv_heads and seqlen_q * (num_heads / num_kv_heads) <= 16, the
 * kernels read adjacent KV heads in pairs as one head of dim 128 (a 64-dim fp8 row is half a
 * 128-byte line; unpaired, each line would be fetched once per head).  The workspace size and
 * plan of this call: mx_paged_gqa_decode_workspace_size (which covers both cache formats) and
 * mx_paged_gqa_decode_plan_fp8kv.
 * No counterpart in the reference, whose cache is bf16 only; it is the same operator on a
 * narrower cache format.
 */
int mx_paged_gqa_decode_fp8kv(const void* q, const void* k_cache, const void* v_cache,
                              void* out, const int32_t* seq_lens, const int32_t* block_table,
                              int64_t batch, int64_t seqlen_q, int64_t num_heads,
                              int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                              int64_t num_pages, int64_t max_pages_per_seq, int64_t max_seq_len,
                              int32_t causal, float scale, float k_scale, float v_scale,
                              int64_t num_splits, void* workspace, int64_t workspace_bytes,
                              int32_t phase, void* stream);

/*
 * Partial decode of one shard of the keys (the split phase of the reference's split-KV decode,
 * optimized_c500_flash_attn.cu:537-551 and the partial (m, l, O) rows it leaves for
 * combine_splits, exposed for a caller-chosen key range).  Arguments as mx_paged_gqa_decode,
 * with seq_lens / block_table describing this shard's keys only; instead of the bf16 output
 * it writes, per query row (b, t, h):
 *   o_partial    [batch, seqlen_q, num_heads, head_dim] fp32, 16-byte aligned: the row's
 *                attention output over this shard's keys (normalised);
 *   lse_partial  [batch, seqlen_q, num_heads] fp32: log(sum_t exp(scale * q . k_t)) over them.
 * A row that sees no key of the shard (empty shard; causal rows before their first key) gets
 * O = 0 and lse = -inf.  With causal = 1 the end-aligned mask is applied to the shard's own
 * length, which is the global mask when the shard holds the last keys of the sequence and
 * earlier shards end at or before L - seqlen_q + 1 (pass causal = 0 for those).  Workspace:
 * mx_paged_gqa_decode_workspace_size of the same arguments.  Returns MX_STATUS_*.
 */
int mx_paged_gqa_decode_partial(const void* q, const void* k_cache, const void* v_cache,
                                float* o_partial, float* lse_partial, const int32_t* seq_lens,
                                const int32_t* block_table, int64_t batch, int64_t seqlen_q,
                                int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                                int64_t max_seq_len, int32_t causal, float scale,
                                int64_t num_splits, void* workspace, int64_t workspace_bytes,
                                void* stream);

/*
 * Log-sum-exp merge of gathered partials (replaces combine_splits,
 * optimized_c500_flash_attn.cu:666-728, over partials the caller holds, e.g. after an
 * all-gather of every shard's mx_paged_gqa_decode_partial output):
 *   out[r] = sum_p exp(lse[p, r] - M) o[p, r] / sum_p exp(lse[p, r] - M),  M = max_p lse[p, r].
 *   o_parts    [num_parts, rows, head_dim] fp32, 16-byte aligned.
 *   lse_parts  [num_parts, rows] fp32 (natural log; -inf = the part saw no key, weight 0).
 *   out        [rows, head_dim] bf16, 8-byte aligned; a row no part saw a key for is zeros.
 * head_dim 64, 128 or 256; rows <= 2^25.  Asynchronous on `stream`.  Returns MX_STATUS_*.
 */
int mx_lse_merge(const float* o_parts, const float* lse_parts, int64_t num_parts, int64_t rows,
                 int64_t head_dim, void* out, void* stream);

/*
 * Host-only planning (no HIP call when num_cus > 0): validates the shape and reports the
 * schedule (MX_SCHEDULE_*), the splits per sequence and tokens per split (split grid; 0 for the
 * balanced schedule), the workgroups launched and the workspace bytes a call with these
 * arguments would use.  Replaces the reference's split policy choose_num_splits
 * (submission_clean.cu:375-430) and its page-rounding of splits (submission_clean.cu:456-461).
 * num_cus <= 0 queries the current device.  Any of the out pointers may be NULL.
 */
int mx_paged_gqa_decode_plan(int64_t batch, int64_t seqlen_q, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             int64_t max_pages_per_seq, int64_t max_seq_len, int64_t num_splits,
                             int64_t num_cus, int64_t* schedule_out, int64_t* splits_out,
                             int64_t* tokens_per_split_out, int64_t* workgroups_out,
                             int64_t* workspace_bytes_out);

/* The plan of the same call through mx_paged_gqa_decode_fp8kv (arguments and outputs as
 * mx_paged_gqa_decode_plan's).  No counterpart in the reference (bf16 caches only). */
int mx_paged_gqa_decode_plan_fp8kv(int64_t batch, int64_t seqlen_q, int64_t num_heads,
                                   int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                   int64_t max_pages_per_seq, int64_t max_seq_len,
                                   int64_t num_splits, int64_t num_cus, int64_t* schedule_out,
                                   int64_t* splits_out, int64_t* tokens_per_split_out,
                                   int64_t* workgroups_out, int64_t* workspace_bytes_out);

/* Workspace bytes a call needs (replaces the grow-only sizing of submission_clean.cu:463,
 * 478-491), on a bf16 or an fp8 cache; negative MX_STATUS_* on invalid arguments.  Queries the
 * current device's CU count when num_splits == 0. */
int64_t mx_paged_gqa_decode_workspace_size(int64_t batch, int64_t seqlen_q, int64_t num_heads,
                                           int64_t num_kv_heads, int64_t head_dim,
                                           int64_t page_size, int64_t max_pages_per_seq,
                                           int64_t max_seq_len, int64_t num_splits);

/*
 * Paged KV-cache append: writes seqlen_new new tokens per sequence into their page slots, the
 * step that fills the layout the decode reads.  No counterpart in the reference, whose harness
 * fills pages with torch.randn (bench_all.py:31-33); the semantics are those of the k / v
 * arguments of flash_attn_with_kvcache, which the reference's harness passes as None
 * (verify_real.py:40-41): token j of sequence b is stored at position
 * pos = max(seq_lens[b], 0) + j, i.e. page block_table[b, pos / page_size], offset
 * pos % page_size.
 *   k_new, v_new   [batch, seqlen_new, num_kv_heads, head_dim] bf16, 16-byte aligned.
 *   k_cache, v_cache, block_table, page_size, max_pages_per_seq: as for the decode.
 *   seq_lens       lengths BEFORE the append; not modified (the caller adds seqlen_new).
 *   num_pages      pool size (required, >= 1): a page id outside [0, num_pages) is flagged
 *                  (MX_DEVICE_BAD_PAGE_ID) and its token skipped; a position past the table
 *                  row is flagged (MX_DEVICE_SEQ_TOO_LONG) and skipped.  Nothing is written
 *                  outside the pool.
 *   workspace      any decode workspace (its status word receives the flags), NULL = the
 *                  library's.
 * Asynchronous on `stream`; head_dim must be a multiple of 8.  Returns MX_STATUS_*.
 */
int mx_paged_kv_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                       const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                       int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim,
                       int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                       void* workspace, void* stream);

/*
 * Append-and-attend: the step flash_attn_with_kvcache performs when given k / v (the
 * reference's oracle, called with k = v = None by its harness, verify_real.py:40-41).  Writes
 * k_new / v_new [batch, seqlen_new, num_kv_heads, head_dim] bf16 at positions
 * max(seq_lens[b], 0) + j of each sequence's block-table row (as mx_paged_kv_append), and
 * decodes q over the max(seq_lens[b], 0) + seqlen_new keys of each sequence (with causal = 1,
 * query token i of seqlen_q sees keys t < L_new - seqlen_q + i + 1, L_new the count after the
 * append).  seq_lens are the lengths BEFORE the append and are not modified.  Other arguments
 * as mx_paged_gqa_decode (max_seq_len is the capacity after the append) and
 * mx_paged_kv_append (num_pages is required; slots past the table row or outside the pool are
 * skipped and flagged, and the output of a flagged call is unspecified).  The workspace is the
 * decode's (mx_paged_gqa_decode_workspace_size).
 * For 1 <= seqlen_new <= 16 this is ONE launch: the new keys are read from k_new / v_new as one
 * more chunk of each (sequence, KV head) and written to the cache by the same kernel, whose
 * attention never reads those slots.  The pools then equal mx_paged_kv_append's bit for bit;
 * the output differs from the two-call sequence only by summation order.  Longer appends run
 * the append kernel, then the decode (bit-identical to the two calls).  Nothing is launched on
 * error.  Returns MX_STATUS_*.
 * No counterpart in the reference's own code; the semantics are flash_attn_with_kvcache's.
 */
int mx_paged_gqa_decode_append(const void* q, const void* k_new, const void* v_new,
                               void* k_cache, void* v_cache, void* out, const int32_t* seq_lens,
                               const int32_t* block_table, int64_t batch, int64_t seqlen_q,
                               int64_t seqlen_new, int64_t num_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t page_size, int64_t num_pages,
                               int64_t max_pages_per_seq, int64_t max_seq_len, int32_t causal,
                               float scale, int64_t num_splits, void* workspace,
                               int64_t workspace_bytes, void* stream);

/*
 * The paged append into an fp8 (e4m3fn) cache: as mx_paged_kv_append, with k_new / v_new bf16
 * and k_cache / v_cache holding one e4m3fn byte per element.  Each value x is stored as the
 * e4m3fn value nearest to x / k_scale (x / v_scale for V; the correctly rounded fp32 quotient,
 * ties to even), the quotient saturated to [-448, 448] first; NaN stays NaN.  k_scale and
 * v_scale must be finite and > 0.  These are the scales the fp8 decode multiplies back.
 * No counterpart in the reference (bf16 caches only).
 */
int mx_paged_kv_append_fp8kv(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                             const int32_t* seq_lens, const int32_t* block_table, int64_t batch,
                             int64_t seqlen_new, int64_t num_kv_heads, int64_t head_dim,
                             int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                             float k_scale, float v_scale, void* workspace, void* stream);

/*
 * Append-and-attend on an fp8 cache: what mx_paged_kv_append_fp8kv and then
 * mx_paged_gqa_decode_fp8kv over seq_lens[b] + seqlen_new keys do, with
 * mx_paged_gqa_decode_append's arguments plus the two scales.  Up to 16 new tokens it is one
 * launch: the attention kernel quantizes the new rows, writes them and attends the quantized
 * values.  Longer appends run the append kernel first.
 * No counterpart in the reference (bf16 caches only).
 */
int mx_paged_gqa_decode_append_fp8kv(const void* q, const void* k_new, const void* v_new,
                                     void* k_cache, void* v_cache, void* out,
                                     const int32_t* seq_lens, const int32_t* block_table,
                                     int64_t batch, int64_t seqlen_q, int64_t seqlen_new,
                                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                     int64_t page_size, int64_t num_pages,
                                     int64_t max_pages_per_seq, int64_t max_seq_len,
                                     int32_t causal, float scale, float k_scale, float v_scale,
                                     int64_t num_splits, void* workspace, int64_t workspace_bytes,
                                     void* stream);

/* Copies the sticky device status word (MX_DEVICE_* bits) of a workspace (NULL = the library's
 * workspace of the current device, MX_NOALLOC_WORKSPACE = the current device's no-alloc array)
 * to *flags_out after synchronising the stream; clears it when reset != 0.  Not part of the
 * reference (which validates nothing on the device). */
int mx_read_device_status(void* workspace, int32_t reset, void* stream, int32_t* flags_out);

/* Status and message of the last failing call on this host thread (reference has none). */
int mx_last_status(void);
const char* mx_last_error(void);

/* Library version string. */
const char* mx_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MX_PAGED_DECODE_H */
