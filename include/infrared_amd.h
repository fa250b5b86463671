/*
 * infrared_amd — C ABI of the MI355X (gfx950) paged-attention hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, element strides and sizes (no framework types);
 *   - launches asynchronously on the caller's `stream` and never synchronises,
 *     allocates or frees device memory, so calls are hipGraph-capturable;
 *   - returns 0 on success or a negative IR_E* code, with a thread-local
 *     message readable through ir_last_error(); it never aborts or throws.
 *
 * Data layout (kept identical to the reference pool so callers that address
 * `pool.k[layer, slot]` directly keep working):
 *   K/V cache of one layer: [num_slots, num_kv_heads, head_dim], slot = block_id *
 *   block_size + offset, head_dim contiguous (reference:
 *   infrared/cache/paged_kv_cache.py:44-46).
 *
 * Device-side bounds problems (a slot or block id outside the pool, a context
 * longer than the block table) never fault: the offending element is skipped
 * and a bit is OR-ed into *err_flags (when err_flags is non-NULL) so the host
 * can check it later without a synchronising call in the hot loop.
 */
#ifndef INFRARED_AMD_H
#define INFRARED_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ir_stream_t; /* a hipStream_t; NULL is the null stream */

/* dtype codes */
enum {
  IR_DTYPE_F32 = 0,
  IR_DTYPE_F16 = 1,
  IR_DTYPE_BF16 = 2
};

/* return codes */
enum {
  IR_OK = 0,
  IR_EINVAL = -1,       /* bad argument (shape, stride, alignment, dtype) */
  IR_EUNSUPPORTED = -2, /* valid request this build has no kernel for */
  IR_EWORKSPACE = -3,   /* workspace missing or too small */
  IR_ELAUNCH = -4       /* the HIP runtime rejected the launch */
};

/* bits OR-ed into *err_flags by the kernels */
enum {
  IR_ERR_SLOT_RANGE = 1,     /* scatter slot >= num_slots (write skipped) */
  IR_ERR_BLOCK_RANGE = 2,    /* block id outside [0, num_blocks) (block masked) */
  IR_ERR_CONTEXT_RANGE = 4,  /* context_len > max_blocks*block_size (clamped) or < 0 */
  IR_ERR_GATHER_RANGE = 8,   /* gather slot outside [0, num_slots) (key masked) */
  IR_ERR_PLAN = 16,          /* a decode plan with sequence pairs run without IR_PLAN_SHARE_GROUPS
                                (nothing written) */
  IR_ERR_WRITE_SLOT = 32     /* a fused prefill's new token written elsewhere than its block-table
                                slot (the call attended the new row itself) */
};

/* flags of ir_paged_prefill_plan, ir_paged_decode_plan and ir_paged_decode_planned */
enum {
  IR_PLAN_SHARE_GROUPS = 1, /* prefill: keep each shared-prefix group's KV head on one XCD;
                               decode: run sequence pairs that share prefix blocks as one unit */
  IR_PLAN_F32 = 2           /* prefill: a plan for an fp32 call (the fp32 kernel's 64-column
                               items); a 16-bit call takes only a plan built without it */
};

/* flags of ir_decode_form */
enum {
  IR_FORM_CLEAR_ON_FAIL = 1 /* after the check, set every context length to 0 when *bad is set */
};

/* Message of the last failed call on this thread ("" if none). */
const char* ir_last_error(void);

/* Version string of the library build. */
const char* ir_version(void);

/*
 * Identity of the stream capture in progress on `stream`: *capture_id = 0 when
 * the stream is not capturing, else a value unique to that capture (the HIP
 * capture sequence id + 1). No counterpart in the reference: the seam uses it
 * to record its reference-form checks once per captured graph
 * (infrared/engine/cuda_graph.py:263-285 captures the decode forward with the
 * reference's own metadata).
 */
int ir_stream_capture_id(ir_stream_t stream, uint64_t* capture_id);

/*
 * KV-slot scatter: k_cache[slot_mapping[i]] = k[i]; v_cache[slot_mapping[i]] = v[i].
 *
 * Replaces PagedKVPool.write (infrared/cache/paged_kv_cache.py:48-57), i.e. the
 * two index_put_ calls `self.k[layer_idx, slots] = k`, and the store_kvcache
 * skeleton of docs/research/t4-triton-cudagraph-api.md:134-158.
 *   k, v:        [n_tokens, num_kv_heads, head_dim], strides in elements
 *                (token, head); head_dim stride is 1.
 *   k_cache, v_cache: one layer of the pool, strides (slot, head) in elements.
 *   slot_mapping: [n_tokens] int64 flat slot ids. A negative slot skips the row
 *                (padding sentinel); a slot >= num_slots is skipped and flagged.
 * Bit-exact copy semantics; duplicated slots must carry identical rows (the
 * pad-by-repeat convention of infrared/engine/cuda_graph.py:22-25).
 */
int ir_kv_scatter(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                  const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                  void* k_cache, void* v_cache, int64_t cache_slot_stride,
                  int64_t cache_head_stride, int64_t num_slots,
                  const int64_t* slot_mapping, int64_t n_tokens, int num_kv_heads,
                  int head_dim, int dtype, int32_t* err_flags, ir_stream_t stream);

/*
 * Slot gather: out_k[i] = k_cache[slots[i]], out_v[i] = v_cache[slots[i]].
 *
 * Replaces PagedKVPool.gather (infrared/cache/paged_kv_cache.py:59-72), the
 * `self.k[layer_idx, flat]` indexing over gather_slots. Outputs are
 * [n, num_kv_heads, head_dim] contiguous; a slot outside [0, num_slots) reads
 * as zeros and is flagged with IR_ERR_GATHER_RANGE.
 */
int ir_gather_slots(const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                    int64_t cache_head_stride, int64_t num_slots, const int64_t* slots,
                    int64_t n, int num_kv_heads, int head_dim, int dtype, void* out_k,
                    void* out_v, int32_t* err_flags, ir_stream_t stream);

/*
 * Paged gather through a block table (test/debug utility that shares the
 * decode kernel's token -> slot address function):
 *   out_k[b, t] = k_cache[block_tables[b, t / bs] * bs + t % bs] for t < context_lens[b],
 *   zero for context_lens[b] <= t < max_ctx.
 * Restates PagedKVPool.gather (infrared/cache/paged_kv_cache.py:59-72) with the
 * gather_slots closed form of infrared/engine/paged_engine.py:306-314.
 *   out_k, out_v: [num_seqs, max_ctx, num_kv_heads, head_dim] contiguous.
 */
int ir_paged_gather(const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                    int64_t cache_head_stride, int64_t num_blocks, int block_size,
                    const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                    const int32_t* context_lens, int num_seqs, int max_ctx,
                    int num_kv_heads, int head_dim, int dtype, void* out_k, void* out_v,
                    int32_t* err_flags, ir_stream_t stream);

/*
 * Bytes of device workspace ir_paged_decode needs for this shape (0 when one
 * partition covers the longest context): the split-KV partials, unnormalised
 * accumulators [num_seqs, num_q_heads, parts, head_dim] and running max / sum
 * [num_seqs, num_q_heads, parts, 2], fp32. Scratch: no initial contents.
 * Calls sharing a workspace must be stream-ordered.
 */
int64_t ir_paged_decode_workspace_size(int num_seqs, int num_q_heads, int num_kv_heads,
                                       int head_dim, int max_blocks_per_seq, int block_size,
                                       int partition_tokens);

/*
 * Arrival counters the split decode needs: one int32 per sequence x KV head x
 * group of <= 16 query heads. The caller zero-fills the counters buffer once;
 * every call (ir_paged_decode, ir_paged_decode_planned) leaves the counters it
 * used at zero, so one counters buffer serves calls of any shape. Kept apart
 * from the workspace because partial rows are scratch whose layout changes
 * with the shape.
 */
int64_t ir_paged_decode_num_counters(int num_seqs, int num_q_heads, int num_kv_heads);

/* The partition size (tokens) ir_paged_decode picks when partition_tokens == 0. */
int ir_paged_decode_default_partition(int num_seqs, int num_kv_heads, int max_blocks_per_seq,
                                      int block_size);

/*
 * GQA paged decode attention, one query token per sequence.
 *
 * Replaces the decode use of _paged_attention_triton / _paged_attention_naive
 * (infrared/model/triton_attention.py:110-129, :310-358) with the
 * (block_tables, context_lens) signature of
 * docs/research/t4-triton-cudagraph-api.md:79-127:
 *   out[b, h] = softmax_t(scale * q[b, h] . K[b, t, h / n_rep]) @ V[b, t, h / n_rep],
 *   t in [0, context_lens[b]), K/V rows addressed through block_tables[b].
 *   q, out:       [num_seqs, num_q_heads, head_dim] (strides seq, head in elements).
 *   block_tables: [num_seqs, bt_stride] int32 block ids, first max_blocks_per_seq used.
 *   context_lens: [num_seqs] int32 (0 gives a zero output row).
 *   partition_tokens: split-KV partition length in tokens (multiple of 16,
 *                 at most 4096; 0 = ir_paged_decode_default_partition). A sequence longer
 *                 than one partition is split across workgroups; the last of them to
 *                 finish (counted on `counters`) merges their fp32 partials with
 *                 log-sum-exp weights.
 *   counters:     >= ir_paged_decode_num_counters(...) int32, zero-filled before
 *                 first use (required when a sequence can span partitions).
 *   workspace:    >= ir_paged_decode_workspace_size(...) bytes, 256-byte aligned.
 * head_dim in {64, 128}; num_q_heads % num_kv_heads == 0; dtype f32/f16/bf16.
 */
int ir_paged_decode(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                    const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                    int64_t cache_head_stride, int64_t num_blocks, int block_size,
                    const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                    const int32_t* context_lens, void* out, int64_t out_seq_stride,
                    int64_t out_head_stride, int num_seqs, int num_q_heads,
                    int num_kv_heads, int head_dim, float scale, int dtype,
                    int partition_tokens, int32_t* counters, int64_t num_counters,
                    void* workspace, int64_t workspace_bytes, int32_t* err_flags,
                    ir_stream_t stream);

/*
 * ir_paged_decode without a caller workspace, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference: it is
 * ir_paged_decode with the same arguments, minus counters and workspace, whose
 * split-KV arrival counters and fp32 partial rows live in a 16 MiB device array
 * inside the library (64 KiB of counters, the rest partial rows), held by
 * every GPU the library runs on until the process ends. A call whose
 * ir_paged_decode_workspace_size exceeds 16 MiB - 64 KiB, or that needs more
 * than 16,384 counters, returns IR_EWORKSPACE. All calls on one GPU share that
 * array: calls that overlap on one GPU (other streams, concurrent graph
 * replays) race; calls ordered on one stream do not. Allocates nothing.
 */
int ir_paged_decode_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                            const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                            int64_t cache_head_stride, int64_t num_blocks, int block_size,
                            const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                            const int32_t* context_lens, void* out, int64_t out_seq_stride,
                            int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
                            int head_dim, float scale, int dtype, int partition_tokens,
                            int32_t* err_flags, ir_stream_t stream);

/*
 * Planned decode: the same attention as ir_paged_decode (one query token per
 * sequence over block_tables / context_lens), on a work-balanced schedule that
 * ir_paged_decode_plan builds once per batch of decode metadata and every
 * layer's ir_paged_decode_planned reuses. Replaces the same reference seam as
 * ir_paged_decode (infrared/model/triton_attention.py:110-129 via
 * PagedKVPool/PagedContext, infrared/cache/paged_kv_cache.py:25-72); the
 * plan/run split has no counterpart in the reference, whose metadata is also
 * built once per step (infrared/engine/paged_engine.py:290-332) and shared by
 * every layer.
 *
 * The call's 16-key tiles (per sequence, per KV head and group of <= 16 query
 * heads) are cut into one equal slice per CU, so every CU reads the same
 * number of keys whatever the spread of context lengths; sequences cut by a
 * slice boundary are merged in the same launch (log-sum-exp of fp32
 * partials, the last-arriving slice merges).
 *
 * ir_paged_decode_plan_bytes: bytes of plan for this shape, 0 when the shape
 *   is not plannable (batch 1..1024, block_size a multiple of 16).
 * ir_paged_decode_planned_workspace_bytes: bytes of workspace (fp32 partial
 *   rows, scratch) the run needs; its arrival counters are
 *   ir_paged_decode_num_counters(...) int32 of a zero-filled counters buffer,
 *   which the run leaves at zero.
 * ir_paged_decode_plan: writes the plan for (block_tables, context_lens) and a
 *   pool with the given slot/head strides (elements) and dtype. Context
 *   lengths outside [0, max_blocks * block_size] are clamped and flagged
 *   (IR_ERR_CONTEXT_RANGE); block ids outside [0, num_blocks) are flagged
 *   (IR_ERR_BLOCK_RANGE) and their keys masked, as in ir_paged_decode.
 * ir_paged_decode_planned: runs one layer over the plan. Shapes and cache
 *   strides must be those the plan was built for; q/out as in ir_paged_decode.
 *   Calls sharing a workspace must be stream-ordered; a plan may be rebuilt
 *   only after the runs that read it.
 * flags: IR_PLAN_SHARE_GROUPS (plan and run alike; taken when a KV head has at
 *   most 8 query heads) pairs sequences b, b + 1 whose block tables begin with
 *   the same block ids -- the blocks the prefix cache hands sequences with a
 *   common prompt prefix (infrared/cache/block_manager.py:209-234,
 *   match_prefix) -- into one unit per KV head: both sequences' query heads in
 *   the MFMA columns one sequence leaves empty, so the shared blocks (those
 *   wholly inside both contexts) are read once for the pair. Runs of
 *   consecutive sharing sequences pair from their start. Outputs are the same
 *   attention (each column sees exactly its sequence's keys). A plan that
 *   holds pairs run without the flag writes nothing and sets IR_ERR_PLAN.
 */
int64_t ir_paged_decode_plan_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                   int max_blocks_per_seq, int block_size);
int64_t ir_paged_decode_planned_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                                int head_dim);
int ir_paged_decode_plan(const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                         const int32_t* context_lens, int num_seqs, int num_q_heads,
                         int num_kv_heads, int block_size, int64_t num_blocks,
                         int64_t cache_slot_stride, int64_t cache_head_stride, int dtype,
                         int flags, void* plan, int64_t plan_bytes, int32_t* err_flags,
                         ir_stream_t stream);
int ir_paged_decode_planned(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                            const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                            void* out, int64_t out_seq_stride, int64_t out_head_stride,
                            int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                            int max_blocks_per_seq, int block_size, float scale, int dtype,
                            int flags, const void* plan, int32_t* counters, int64_t num_counters,
                            void* workspace, int64_t workspace_bytes, int32_t* err_flags,
                            ir_stream_t stream);

/*
 * Paged attention over the reference's own per-forward metadata: per-key flat
 * slot ids plus an additive mask. This is the exact contract of
 * _paged_attention_triton / _paged_attention_naive
 * (infrared/model/triton_attention.py:110-129, :310-358; mask semantics of
 * infrared/model/layers.py:102-118), so every caller of the reference seam
 * (eager decode, prefill with prefix hit, packed mixed steps, graph decode)
 * runs unchanged.
 *   q, out:       [B, Sq, num_q_heads, head_dim] (strides b, s, h in elements).
 *   gather_slots: [B, T] int64 (strides b, t) flat slot ids; slots outside the
 *                 pool are flagged and masked out.
 *   mask:         additive, element (b, s, t) at mask + b*mb + s*ms + t*mt, of
 *                 dtype mask_dtype (f32/f16/bf16); strides may be 0 (broadcast).
 * Scores are q.k*scale + mask; a row whose keys are all masked with finfo.min
 * averages V uniformly, as the reference softmax does.
 *   run_if:       null, or a device int32 read by every workgroup first: the
 *                 call does nothing (writes no output) while it is 0. A graph
 *                 captured over the reference's decode metadata records this
 *                 kernel gated on ir_decode_form's *bad.
 */
int ir_paged_attention_masked(const void* q, int64_t q_b_stride, int64_t q_s_stride,
                              int64_t q_h_stride, const void* k_cache, const void* v_cache,
                              int64_t cache_slot_stride, int64_t cache_head_stride,
                              int64_t num_slots, const int64_t* gather_slots,
                              int64_t gs_b_stride, int64_t gs_t_stride, const void* mask,
                              int64_t mask_b_stride, int64_t mask_s_stride,
                              int64_t mask_t_stride, int mask_dtype, void* out,
                              int64_t out_b_stride, int64_t out_s_stride,
                              int64_t out_h_stride, int batch, int seq_q, int seq_k,
                              int num_q_heads, int num_kv_heads, int head_dim, float scale,
                              int dtype, int32_t* err_flags, const int32_t* run_if,
                              ir_stream_t stream);

/*
 * Block tables from the reference engine's own decode metadata, so unchanged
 * callers of the seam reach the block-table decode kernels. The reference's
 * eager decode passes gather_slots[i, p] = bt_i[p / bs] * bs + p % bs (0 past
 * ctx_i) and the mask 0 for p < ctx_i, finfo.min after
 * (infrared/engine/paged_engine.py:306-314, :630-638, via PagedContext,
 * infrared/cache/paged_kv_cache.py:75-91). Writes context_lens[i] (the mask's
 * zeros) and block_tables[i, j] = gather_slots[i, j * bs] / bs (0 past the
 * context), and sets bad[0] to 1 unless the metadata has exactly that form,
 * else 0: the zeros a prefix, later mask values <= -6e4, at least one zero,
 * every slot below ctx_i the closed form, every block id in [0, num_blocks).
 * With bad[0] clear the decode kernels over these tables compute what
 * ir_paged_attention_masked computes. bad: int32 [batch + 1], no clearing
 * needed (bad[1..batch] is working space).
 *   flags: IR_FORM_CLEAR_ON_FAIL also sets every context_lens[i] to 0 when the
 *   check failed (for a caller that does not wait for bad[0], as under graph
 *   capture: the block-table decode then reads no key and the mask kernel,
 *   gated on bad[0], computes the call).
 *   host_verdict: null, or pinned host memory from the HIP host allocator
 *   (one uint64): receives (uint64)tag << 32 | bad[0] from the device at the
 *   end of the call in one 8-byte store, so the host can read the verdict of
 *   the call it tagged when it arrives, without synchronising.
 *   gather_slots: [batch, seq_k] int64 (strides b, t); mask: element (b, t) at
 *   mask + b*mask_b_stride + t*mask_t_stride, dtype mask_dtype.
 *   block_tables: [batch, bt_stride] int32, max_blocks_per_seq >= ceil(seq_k / bs).
 */
int ir_decode_form(const int64_t* gather_slots, int64_t gs_b_stride, int64_t gs_t_stride,
                   const void* mask, int64_t mask_b_stride, int64_t mask_t_stride, int mask_dtype,
                   int batch, int seq_k, int block_size, int64_t num_blocks, int32_t* block_tables,
                   int64_t bt_stride, int max_blocks_per_seq, int32_t* context_lens, int32_t* bad,
                   int flags, uint64_t* host_verdict, uint32_t tag, ir_stream_t stream);

/*
 * Prefill metadata from the reference engine's packed prefill / mixed-step
 * form, so unchanged callers of the seam reach ir_paged_prefill. The reference
 * hands the seam one frame of num_q query tokens, a key axis concatenating each
 * scheduled sequence's history [0, start + q) in order, per-key slots
 * gather_slots[k_off + p] = bt[p / bs] * bs + p % bs and the additive mask of
 * build_varlen_mask / build_attention_mask (0 where the key is the query's own
 * sequence at or before its position, finfo.min elsewhere)
 * (infrared/engine/paged_engine.py:194-206, :461-516;
 * infrared/model/inputs.py:33-85). One call before the host's one read
 * (ir_varlen_form_tables only when the tables did not fit):
 *   ir_varlen_form_scan: reads every mask element once (element (r, k) at
 *     mask + r*mask_q_stride + k*mask_k_stride; a contiguous 16-byte-aligned
 *     mask as one flat array) and every key's slot; writes cu_seqlens_q
 *     [num_q + 1], q_start [num_q] and seq_k_offsets [num_q] for the sequences
 *     found, and info[0..5] (no clearing needed): info[1..3] = sequence count,
 *     longest chunk, widest block table (blocks); info[0] = 0 if each row's
 *     visible keys are one contiguous range, every other value <= -6e4, the
 *     rows of a sequence each see one key more than the last, the sequences'
 *     key ranges tile [0, num_k) in order, and every slot
 *     gather_slots[k_off_i + p] (stride gs_k_stride) has the closed form with a
 *     block id in [0, num_blocks); else 1. info[5] is working space. info[4]
 *     = 1 when the call also wrote the block tables: block_tables (null or
 *     int32 [tables_capacity]) holds them as [info[1], W] with
 *     W = max(info[3], 1) when info[0] is clear and info[1] * W <=
 *     tables_capacity. host_record (null, or pinned host memory
 *     from the HIP host allocator, at least 2*num_q + 9 int32) receives, from
 *     the device at the end of the call, info[0..4] at [0..4], then
 *     cu_seqlens_q[0..n] at [8..8+n] and q_start[0..n) at [9+n..9+2n)
 *     (n = info[1]; written only when info[0] is clear) and, last, once the
 *     rest is visible to the host, `tag` at [7]: a host that waits for word 7
 *     to hold a tag its earlier calls did not pass reads the whole record
 *     without synchronising the stream (a stream synchronisation works too;
 *     nothing is written when num_q is 0). row_records: [4*num_q] int32
 *     scratch, 16-byte aligned, zero before the first call; every call leaves
 *     it zero (calls sharing it must be stream-ordered).
 *   ir_varlen_form_tables: block_tables[i, j] = gather_slots[k_off_i + j*bs] / bs
 *     ([num_seqs, bt_stride] int32, max_blocks_per_seq >= info[3]).
 * With info[0] clear after the scan, ir_paged_prefill over this metadata
 * computes what ir_paged_attention_masked computes from the frame.
 */
int ir_varlen_form_scan(const void* mask, int64_t mask_q_stride, int64_t mask_k_stride, int mask_dtype,
                        int num_q, int num_k, const int64_t* gather_slots, int64_t gs_k_stride, int block_size,
                        int64_t num_blocks, int32_t* row_records, int32_t* cu_seqlens_q, int32_t* q_start,
                        int32_t* seq_k_offsets, int32_t* info, int32_t* block_tables, int64_t tables_capacity,
                        int32_t* host_record, int64_t host_capacity, int32_t tag, ir_stream_t stream);
int ir_varlen_form_tables(const int64_t* gather_slots, int64_t gs_k_stride, const int32_t* seq_k_offsets,
                          const int32_t* cu_seqlens_q, const int32_t* q_start, int num_seqs, int block_size,
                          int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq, ir_stream_t stream);

/*
 * Chunked prefill / prefix-hit prefill / packed mixed step over block tables
 * (16-bit dtypes, MFMA). Replaces the Sq > 1 uses of
 * _paged_attention_triton / _paged_attention_naive
 * (infrared/model/triton_attention.py:110-129, :310-358) with the
 * (block_tables, cu_seqlens_q, q_start) form of the engine's prefill and mixed
 * steps (infrared/engine/paged_engine.py:194-207, :461-516):
 *   query token i of sequence b (packed row cu_seqlens_q[b] + i) is at
 *   position q_start[b] + i and attends keys t <= q_start[b] + i of sequence b,
 *   K/V rows addressed through block_tables[b] -- the causal-with-offset mask of
 *   infrared/model/inputs.py:33-54 and, per sequence, the varlen mask of
 *   infrared/model/inputs.py:57-85 (a decode row is a one-token sequence).
 *   q, out:       [total_q, num_q_heads, head_dim] (strides token, head in elements).
 *   cu_seqlens_q: [num_seqs + 1] int32, non-decreasing, cu_seqlens_q[num_seqs] <= total_q.
 *   q_start:      [num_seqs] int32, tokens already cached (the first query's position).
 *   max_q_len:    upper bound of the per-sequence query counts (sizes the grid; a chunk
 *                 longer than it sets IR_ERR_CONTEXT_RANGE and its rows past the bound
 *                 are not written).
 *   plan:         null, or the plan ir_paged_prefill_plan wrote for this call's
 *                 cu_seqlens_q / q_start, shapes and dtype (IR_PLAN_F32 for fp32,
 *                 without it for bf16 / f16; plan_bytes as sized by
 *                 ir_paged_prefill_plan_bytes): workgroups then run the heaviest work
 *                 first, and items heavier than the mean load of a workgroup slot are cut
 *                 into key-range pieces merged in the same launch. The plan also holds
 *                 the pieces' arrival counters and partial rows, so calls on one plan
 *                 must be stream-ordered. Results agree with the unplanned call within
 *                 fp32 rounding of the merge (identical when nothing is cut).
 * Keys q_start[b] + q_len_b beyond the table (max_blocks_per_seq * block_size) set
 * IR_ERR_CONTEXT_RANGE and are clamped; a bad block id sets IR_ERR_BLOCK_RANGE and
 * that block's keys read as zeros. head_dim in {64, 128}; dtype bf16, f16 or fp32. fp32
 * (the reference's fp32 path: fp32 scores, softmax and PV product) runs on its own
 * kernel of 64-column workgroups: at most 64 query heads per KV head (more returns
 * IR_EUNSUPPORTED), planned by a plan built with IR_PLAN_F32, the fused write as its
 * own launch first; its q, out, cache and new-row strides are multiples of 16 bytes and
 * out 16-byte aligned.
 * Fused K/V write (the step's PagedKVPool.write folded into the call; k_new null: none):
 *   k_new, v_new: [n_write, num_kv_heads, head_dim] (strides token, head in elements;
 *                 16-byte aligned, 16-byte strides), rows written to the caches at
 *                 write_slots[row] (int64 [n_write]; a negative slot is skipped, one
 *                 past the pool is flagged IR_ERR_SLOT_RANGE), as ir_kv_scatter would --
 *                 by workgroups of the same launch, so the caches are written here.
 *   src_row0:     rows src_row0 .. src_row0 + total_q - 1 are this call's query tokens
 *                 in packed order; their keys (positions >= q_start[b]) are read from
 *                 those rows, not from the pool. Equal to ir_kv_scatter followed by the
 *                 unfused call when each such row's write slot is its block-table slot;
 *                 a row whose slot differs sets IR_ERR_WRITE_SLOT.
 */
int ir_paged_prefill(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                     const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                     int64_t cache_head_stride, int64_t num_blocks, int block_size,
                     const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                     const int32_t* cu_seqlens_q, const int32_t* q_start, int num_seqs,
                     int total_q, int max_q_len, void* out, int64_t out_tok_stride,
                     int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim,
                     float scale, int dtype, void* plan, int64_t plan_bytes,
                     const void* k_new, int64_t k_new_tok_stride, int64_t k_new_head_stride,
                     const void* v_new, int64_t v_new_tok_stride, int64_t v_new_head_stride,
                     const int64_t* write_slots, int64_t n_write, int64_t src_row0,
                     int32_t* err_flags, ir_stream_t stream);

/*
 * Work plan for ir_paged_prefill, built on the device from the call's metadata
 * (no host synchronisation, so it can be captured). Like the decode plan it
 * has no counterpart in the reference, which builds a step's prefill metadata
 * once (infrared/engine/paged_engine.py:194-207, :461-516) and shares it across
 * layers; so is this plan: build it once per step, pass it to every layer's
 * ir_paged_prefill.
 * ir_paged_prefill_plan_bytes: bytes of plan for these shapes (0 when there is
 *   nothing to plan), enough for a plan of either kind (IR_PLAN_F32 or not).
 * ir_paged_prefill_plan: writes the plan (one workgroup: weighs every (sequence,
 *   query block) item by the key tiles it walks, cuts the heaviest, places the
 *   pieces, clears the arrival counters). Arguments as for ir_paged_prefill,
 *   plus flags; IR_PLAN_F32 plans an fp32 call, whose items are the fp32
 *   kernel's (64 / n_rep query tokens, at most 64 query heads per KV head), and
 *   only an fp32 call reads such a plan. Default placement: one global
 *   heaviest-first order, a piece's
 *   KV heads on consecutive workgroups. IR_PLAN_SHARE_GROUPS: consecutive
 *   sequences whose block tables begin with the same block id form a share
 *   group -- the prefix cache of infrared/cache/block_manager.py:209-234
 *   (match_prefix) hands every sequence with a common cached prefix the same
 *   blocks for it, registered by :258-283 (register_full_blocks) -- and each
 *   (share group, KV head) runs on one XCD (when the KV heads divide the XCD
 *   count and the groups balance), so a shared prefix's K/V is fetched into
 *   one L2 for the whole group: fewer bytes from memory, for callers whose
 *   prefill shares HBM with other work. Only block_tables' first column is
 *   read (bt_stride elements between rows); the placement changes the
 *   schedule, never a result bit.
 * ir_paged_prefill_plan_xcds: XCDs the plan lays its grid out for on the
 *   current device (the plan's size depends on it).
 */
int64_t ir_paged_prefill_plan_bytes(int num_seqs, int max_q_len, int num_q_heads, int num_kv_heads,
                                    int head_dim);
int ir_paged_prefill_plan(const int32_t* cu_seqlens_q, const int32_t* q_start,
                          const int32_t* block_tables, int64_t bt_stride, int num_seqs,
                          int total_q, int max_q_len, int max_blocks_per_seq, int block_size,
                          int num_q_heads, int num_kv_heads, int head_dim, int flags, void* plan,
                          int64_t plan_bytes, ir_stream_t stream);
int ir_paged_prefill_plan_xcds(void);

/*
 * Fused rotary embedding + KV-slot scatter. Replaces, per layer,
 * apply_rotary_pos_emb (infrared/model/layers.py:79-89, called at :164) followed by
 * PagedKVPool.write (infrared/cache/paged_kv_cache.py:48-57, called from
 * infrared/model/triton_attention.py:101-104):
 *   q_out[i, h] = rope(q[i, h]);  k_cache[slot_mapping[i], h] = rope(k[i, h]);
 *   v_cache[slot_mapping[i], h] = v[i, h],
 *   rope(x) = x * c + rotate_half(x) * s, rotate_half(x) = (-x[D/2:], x[:D/2]),
 *   c, s = cos[i], sin[i] rounded to the activation dtype first, every product and
 *   the sum rounded to the dtype (the reference's tensor ops; bit-identical).
 *   q, q_out: [n_tokens, num_q_heads, head_dim] (q_out may alias q); k, v:
 *   [n_tokens, num_kv_heads, head_dim]; cos, sin: fp32 [n_tokens, head_dim] rows
 *   (cs_tok_stride elements apart), as RotaryEmbedding returns them.
 * Slot semantics as ir_kv_scatter (negative = skip, >= num_slots = skip + flag).
 * head_dim a multiple of 16; all rows (cos/sin included) 16-byte aligned.
 */
int ir_rope_kv_scatter(const void* q, int64_t q_tok_stride, int64_t q_head_stride, void* q_out,
                       int64_t qo_tok_stride, int64_t qo_head_stride, const void* k,
                       int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                       int64_t v_tok_stride, int64_t v_head_stride, const float* cos,
                       const float* sin, int64_t cs_tok_stride, void* k_cache, void* v_cache,
                       int64_t cache_slot_stride, int64_t cache_head_stride, int64_t num_slots,
                       const int64_t* slot_mapping, int64_t n_tokens, int num_q_heads,
                       int num_kv_heads, int head_dim, int dtype, int32_t* err_flags,
                       ir_stream_t stream);

/*
 * Read-only HBM streaming roof (a measurement utility; no counterpart in the
 * reference, which publishes no bandwidth figure): reads `bytes` of `src` with
 * the decode kernels' load form (non-temporal 16-byte loads, 1 KiB contiguous
 * per wavefront instruction) and discards them. Timing a call gives the read
 * bandwidth the decode's achieved KV GB/s is held against.
 * ir_hbm_read_granule: `bytes` must be a positive multiple of this.
 * ir_hbm_read: `sink` is one uint32 the kernel may write (a value no caller
 * should rely on); workgroups 0 = 8 per CU.
 */
int64_t ir_hbm_read_granule(void);
int ir_hbm_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups, ir_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* INFRARED_AMD_H */
