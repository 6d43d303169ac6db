/*
 * seqattn_hip.h - C ABI of the MI355X (gfx950) streamed exact-attention library.
 *
 * The library is libseqattn_hip.so, built from stream-attn_amd/csrc/.  Every entry
 * point takes plain device or pinned-host pointers, element strides and sizes;
 * no C++ type or exception crosses this boundary.  The caller owns all memory:
 * the library never allocates or frees caller buffers.  A pipeline object owns
 * only its own HIP streams and events.
 *
 * Return codes: 0 on success, a positive hipError_t when the HIP runtime
 * failed, or one of the negative SA_ERR_* codes when an argument was rejected.
 * sa_last_error() returns a message describing the most recent failure on the
 * calling thread.
 *
 * Tensor layouts follow the reference: packed [tokens, heads, head_dim] with
 * the head_dim stride equal to 1; every other stride is passed in elements.
 */
#ifndef SEQATTN_HIP_H
#define SEQATTN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: pipeline state in 16-row groups (sa_pipeline_create); fused finalize in
 * the pipeline's last chunk launches.  3: head-group pipelines
 * (sa_pipeline_create_head_groups). */
#define SA_ABI_VERSION 3

/* dtype codes for Q/K/V/output element types */
#define SA_DTYPE_BF16 0
#define SA_DTYPE_FP16 1

/* sa_update_attention_state flags */
#define SA_FLAG_CAUSAL 1
#define SA_FLAG_INITIALIZE 2

/* negative error codes (positive codes are hipError_t values) */
#define SA_ERR_INVALID_ARGUMENT (-1)
#define SA_ERR_UNSUPPORTED_DTYPE (-2)
#define SA_ERR_UNSUPPORTED_HEAD_DIM (-3)
#define SA_ERR_BAD_STATE (-4)

/* ABI version of the loaded library; equals SA_ABI_VERSION when it matches
 * this header. */
int32_t sa_abi_version(void);

/* Message for the most recent failure on the calling thread ("" if none). */
const char* sa_last_error(void);

/*
 * One K/V chunk's online-softmax update of the FP32 state (m, l, acc) of a
 * resident query block.
 *
 * Replaces update_attention_state (reference src/seqattn_core/kernels/streaming.py:205-271),
 * which launches _streaming_attention_update_kernel (same file, lines 19-156).
 *
 *   q    [q_tokens, q_heads, head_dim]      bf16/fp16, strides (stride_qt, stride_qh, 1)
 *   k, v [kv_tokens, kv_heads, head_dim]    same dtype, strides (stride_kt, stride_kh, 1) / (stride_vt, stride_vh, 1)
 *   running_max, running_sum [q_tokens, q_heads]  fp32, shared strides (stride_st, stride_sh)
 *   accumulator [q_tokens, q_heads, head_dim]     fp32, strides (stride_at, stride_ah, 1)
 *
 * Logits are q.k * softmax_scale * log2(e) (base-2 domain).  With
 * SA_FLAG_CAUSAL, key kv_local_offset + j is visible to query q_local_offset + i
 * iff kv_local_offset + j <= q_local_offset + i + causal_shift.  With
 * SA_FLAG_INITIALIZE the state starts at m = -inf, l = 0, acc = 0 instead of
 * being read.  q_heads must be a multiple of kv_heads (query head h reads K/V
 * head h / (q_heads / kv_heads)).  head_dim is a multiple of 8 in [16, 256].
 * The launch is asynchronous on `stream` (a hipStream_t, NULL = default stream).
 */
int32_t sa_update_attention_state(
    const void* q, const void* k, const void* v,
    float* running_max, float* running_sum, float* accumulator,
    int64_t stride_qt, int64_t stride_qh,
    int64_t stride_kt, int64_t stride_kh,
    int64_t stride_vt, int64_t stride_vh,
    int64_t stride_st, int64_t stride_sh,
    int64_t stride_at, int64_t stride_ah,
    int32_t q_tokens, int32_t kv_tokens,
    int32_t q_heads, int32_t kv_heads, int32_t head_dim,
    int32_t q_local_offset, int32_t kv_local_offset, int32_t causal_shift,
    double softmax_scale, int32_t flags, int32_t dtype,
    void* stream);

/*
 * The update above with INT8 K/V and per-group fp16 scales.
 *
 * Replaces update_attention_state_int8 (reference
 * src/seqattn_core/kernels/streaming.py:274-342; dequantization at lines 113-120).
 *
 *   k, v     [kv_tokens, kv_heads, head_dim] int8, strides (stride_kt, stride_kh, 1), multiples of 16
 *   k_scales, v_scales  fp16, element (g, h) at scales[g * stride_?sg + h * stride_?sh]
 *
 * Key j of K/V head h is dequantized as dtype(float(k[j, h, :]) * float(scale))
 * with scale = k_scales[(storage_token_offset + j) / quant_group_tokens, h]
 * (quant_group_tokens a power of two; the reference's pages use 64), which is
 * the reference's rounding: the result equals sa_update_attention_state on the
 * dequantized K/V.  head_dim is a multiple of 16 in [16, 128].  Other
 * arguments as in sa_update_attention_state.
 */
int32_t sa_update_attention_state_int8(
    const void* q, const void* k, const void* v,
    const void* k_scales, const void* v_scales,
    float* running_max, float* running_sum, float* accumulator,
    int64_t stride_qt, int64_t stride_qh,
    int64_t stride_kt, int64_t stride_kh,
    int64_t stride_vt, int64_t stride_vh,
    int64_t stride_ksg, int64_t stride_ksh,
    int64_t stride_vsg, int64_t stride_vsh,
    int64_t stride_st, int64_t stride_sh,
    int64_t stride_at, int64_t stride_ah,
    int32_t q_tokens, int32_t kv_tokens,
    int32_t q_heads, int32_t kv_heads, int32_t head_dim,
    int32_t q_local_offset, int32_t kv_local_offset, int32_t storage_token_offset,
    int32_t causal_shift, double softmax_scale, int32_t flags, int32_t dtype,
    int32_t quant_group_tokens, void* stream);

/*
 * out = acc / l where l > 0, else 0, cast to dtype; optionally
 * lse = ln(sum exp(logits)) = (m + log2 l) * ln 2 (natural log), -inf where l == 0.
 *
 * Replaces finalize_attention (reference src/seqattn_core/kernels/streaming.py:345-371),
 * which launches _finalize_attention_kernel (lines 158-202); the LSE output has
 * no counterpart in the reference.
 *
 *   accumulator [q_tokens, q_heads, head_dim] fp32, strides (stride_at, stride_ah, 1)
 *   running_max, running_sum [q_tokens, q_heads] fp32, strides (stride_st, stride_sh)
 *   out [q_tokens, q_heads, head_dim] dtype, strides (stride_ot, stride_oh, 1)
 *   lse (may be NULL) fp32, element (h, t) at lse[h * lse_stride_h + lse_token_offset + t]
 *
 * running_max may be NULL when lse is NULL.  `out` may alias the query buffer
 * that fed the update (device-consumer mode): this kernel reads only the state.
 */
int32_t sa_finalize_attention(
    const float* accumulator, const float* running_max, const float* running_sum,
    void* out, float* lse,
    int64_t stride_at, int64_t stride_ah,
    int64_t stride_st, int64_t stride_sh,
    int64_t stride_ot, int64_t stride_oh,
    int64_t lse_stride_h, int64_t lse_token_offset,
    int32_t q_tokens, int32_t q_heads, int32_t head_dim, int32_t dtype,
    void* stream);

/* ------------------------------------------------------------------------ */
/* Transfer pipeline: pinned host Q/K/V -> HBM workspace -> pinned host out. */
/* ------------------------------------------------------------------------ */

typedef struct sa_pipeline sa_pipeline;

typedef struct sa_pipeline_stats {
    int64_t h2d_bytes;
    int64_t d2h_bytes;
    int64_t q_chunks;
    int64_t kv_tiles;
    int64_t max_resident_q_tokens;
} sa_pipeline_stats;

/*
 * Bind a pipeline to caller-owned device workspace buffers (the layout of
 * CudaWorkspace, reference src/seqattn_core/streaming/workspace.py:8-50) and
 * its two copy streams (H2D, D2H), and create its ready/free events.
 *
 *   q_buffer      [q_chunk_tokens, q_heads, head_dim] dtype
 *   k_slots[i], v_slots[i]  [kv_chunk_tokens, kv_heads, head_dim] dtype, i < num_kv_buffers (1..3)
 *   running_max, running_sum  q_rows * q_heads fp32
 *   accumulator   q_rows * q_heads * head_dim fp32
 *                 with q_rows = q_chunk_tokens rounded up to a multiple of 16.
 *                 The pipeline keeps this state in the update kernel's
 *                 row-group layout (16-row groups in lane order, so every
 *                 state load and store moves whole contiguous blocks), not in
 *                 the strided [token][head] layout of sa_update_attention_state;
 *                 only this pipeline's launches read it.  Buffers sized for
 *                 q_chunk_tokens rows only are too small whenever
 *                 q_chunk_tokens is not a multiple of 16 and q_heads > 1.
 *   out_slots     NULL (device-consumer mode: no raw output buffers) or
 *                 num_output_buffers pointers to [q_chunk_tokens, q_heads, head_dim] dtype
 *   num_output_buffers  1..2: output ready/free event pairs (and slots when out_slots != NULL)
 *   h2d_stream, d2h_stream  caller hipStream_t handles for the copies, or NULL
 *                 for streams the pipeline creates (default priority) and
 *                 destroys with itself.  Caller streams must outlive the
 *                 pipeline; a caller whose allocator tracks stream uses of
 *                 its buffers (torch record_stream) must pass its own streams.
 * All buffers are contiguous.
 */
int32_t sa_pipeline_create(
    sa_pipeline** out_pipeline, int32_t device,
    void* q_buffer, void* const* k_slots, void* const* v_slots, int32_t num_kv_buffers,
    float* running_max, float* running_sum, float* accumulator,
    void* const* out_slots, int32_t num_output_buffers,
    int32_t q_chunk_tokens, int32_t kv_chunk_tokens,
    int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t dtype,
    void* h2d_stream, void* d2h_stream);

/*
 * Bind a pipeline to the buffer sets of the head-group schedule.  No
 * counterpart in the reference, whose resident Q super-block spans every head
 * of a token range and streams all of K and V once per block (planner.py:187-325,
 * streaming/executor.py:18-188).  Here a unit is every token of a group of
 * group_kv_heads K/V heads and their q_heads / kv_heads query heads per K/V
 * head, so each byte of Q, K and V crosses PCIe once per run.
 *
 *   qo_sets[i]   [max_q_tokens, group_kv_heads * (q_heads / kv_heads), head_dim] dtype:
 *                a unit's Q columns, then its output
 *   k_sets[i], v_sets[i]  [max_kv_tokens, group_kv_heads, head_dim] dtype
 *   vt_sets      NULL, or num_sets device buffers of vt_bytes each: V of a
 *                segment transposed per K/V head for head_dim 128, as for
 *                sa_pipeline_attach_resident_scratch (used when a segment's
 *                group_kv_heads * 128 * roundup(keys, 64) * 2 bytes fit)
 *   num_sets     1 or 2; with 2, unit u uses set u % 2 and units alternate
 *                between compute_stream and a second stream of the pipeline,
 *                and the units' sizes ramp up 1, 2, 4, ... K/V heads and back
 *                down at the end, with units of at most group_kv_heads,
 *                evened out, between (the first unit's copies and the last
 *                units' output copies are the exposed ones); with 1, units
 *                of at most group_kv_heads, evened out
 *   kv_chunk_tokens  where the row sums merge, as in a token-block pipeline of
 *                that K/V chunk, whose sa_pipeline_run output this matches bit
 *                for bit; a segment longer than one chunk needs a chunk that is
 *                a multiple of 64
 *   h2d_stream, d2h_stream  as for sa_pipeline_create
 * Buffers are contiguous and 16-byte aligned.  sa_pipeline_run on such a
 * pipeline runs the head-group schedule: per unit, strided H2D copies of its
 * K and V columns of every token (after the set's previous launches) and of
 * its Q columns (after the set's previous output copy),
 * one fused update launch per segment writing the output over the unit's Q
 * rows and the LSE, and a strided D2H of the output columns.  Inputs may
 * hold at most max_q_tokens / max_kv_tokens rows.  The step API
 * (load_q ... d2h, attach_int8_scales) returns SA_ERR_BAD_STATE;
 * sa_pipeline_run_resident works for segments its single fused launch
 * covers.
 */
int32_t sa_pipeline_create_head_groups(
    sa_pipeline** out_pipeline, int32_t device,
    void* const* qo_sets, void* const* k_sets, void* const* v_sets, void* const* vt_sets, int64_t vt_bytes,
    int32_t num_sets, int64_t max_q_tokens, int64_t max_kv_tokens, int32_t group_kv_heads,
    int32_t kv_chunk_tokens, int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t dtype,
    void* h2d_stream, void* d2h_stream);

/*
 * Head-group pipelines only: page-locked host memory through which
 * sa_pipeline_run copies the output when out_host is pageable (strided
 * copies between pageable memory and the device are staged by the runtime
 * row by row).  Each unit's output goes through it in row chunks, in order
 * on the D2H stream: a chunk's copy, then a host function
 * (hipLaunchHostFunc) that scatters the chunk into the host rows, then the
 * next chunk; the calling thread does not wait for them until the run ends.
 * The buffer must hold at least one output row of a unit
 * (group_kv_heads * q_heads / kv_heads * head_dim * 2 bytes).  NULL and 0
 * detach it; the pipeline keeps the pointer until then.  No counterpart in
 * the reference.
 */
int32_t sa_pipeline_attach_host_staging(sa_pipeline* pipeline, void* staging, int64_t bytes);

/* Wait for all pending copies of the pipeline, then release its events and the streams it created. */
int32_t sa_pipeline_destroy(sa_pipeline* pipeline);

/*
 * Whole tensor-mode schedule with host output (reference
 * src/seqattn_core/streaming/executor.py:18-188 without output_transform):
 * for each segment, for each Q super-block: Q H2D on the H2D stream, then per
 * K/V chunk an H2D into the next ring slot (fenced by that slot's free event)
 * and an update launch on compute_stream (fenced by the slot's ready event),
 * then the finalized block is copied into out_host on the D2H stream.  With
 * one output slot (or none, output_mode host_aliased) the block's last chunk
 * launches write the output and the LSE in their epilogue, into the buffer
 * that held the block's Q, in place of a state store and a finalize launch;
 * with two slots a finalize launch writes the output slot.  Without output
 * slots the block's output leaves, and the next block's Q rows arrive, in
 * row pieces of the block (multiples of the update kernel's workgroup tile)
 * as the block's last chunk launches finish piece by piece, and the next
 * block's first chunk is copied ahead of its Q rows and applied to each
 * piece as its rows land; every row still sees the same chunks in the same
 * order.  Returns after the D2H stream has drained.  An error return comes
 * after the pipeline's copy streams and second stream have drained, so no
 * copy still reads or writes the host buffers; launches already enqueued on
 * compute_stream may still run.
 *
 *   q_host/k_host/v_host/out_host: contiguous pinned host [tokens, heads, head_dim] dtype
 *   cu_seqlens_q/k: num_segments + 1 host int64 boundaries
 *   lse (may be NULL): device fp32 [q_heads, lse_stride_h >= total_q_tokens]
 *   stats (may be NULL): counters are ADDED to it
 */
int32_t sa_pipeline_run(
    sa_pipeline* pipeline,
    const void* q_host, const void* k_host, const void* v_host, void* out_host,
    float* lse, int64_t lse_stride_h,
    const int64_t* cu_seqlens_q, const int64_t* cu_seqlens_k, int32_t num_segments,
    double softmax_scale, int32_t causal,
    void* compute_stream, sa_pipeline_stats* stats);

/*
 * Head-group pipelines only: sa_pipeline_run with the output in device
 * memory.  out [total_q_tokens, q_heads, head_dim] dtype with strides
 * (stride_ot, stride_oh, 1), 16-byte aligned, strides multiples of 8; each
 * unit's fused launches write the rows of its heads straight into it, and no
 * output copy is made.  Enqueued on compute_stream (and the pipeline's
 * second stream, joined back into it); returns once the host inputs have
 * been copied, before the launches end: later work on compute_stream sees
 * the output and the LSE.  An error return comes after the copy streams and
 * the second stream have drained, as for sa_pipeline_run.  No counterpart in
 * the reference (its device outputs go through output_transform,
 * executor.py:145-172).
 */
int32_t sa_pipeline_run_device_output(
    sa_pipeline* pipeline,
    const void* q_host, const void* k_host, const void* v_host,
    void* out, int64_t stride_ot, int64_t stride_oh,
    float* lse, int64_t lse_stride_h,
    const int64_t* cu_seqlens_q, const int64_t* cu_seqlens_k, int32_t num_segments,
    double softmax_scale, int32_t causal,
    void* compute_stream, sa_pipeline_stats* stats);

/*
 * Step interface used by device-consumer mode (reference executor.py:44-186
 * with output_transform): the caller runs one Q super-block at a time and may
 * consume the finalized device tile between finalize and D2H.  sa_pipeline_run
 * is these steps in a loop.
 *
 * sa_pipeline_load_q: H2D of q_tokens rows from q_host (already offset to the
 * super-block start) into q_buffer on the H2D stream, after the Q-free event
 * of the previous super-block; compute_stream then waits for the copy.
 */
int32_t sa_pipeline_load_q(sa_pipeline* pipeline, const void* q_host, int32_t q_tokens,
                           void* compute_stream, sa_pipeline_stats* stats);

/* Stream one segment's K/V (k_host/v_host offset to the segment start,
 * k_length rows) through the ring in kv_chunk_tokens chunks and apply every
 * chunk to the resident Q block (executor.py:68-123). */
int32_t sa_pipeline_stream_kv(sa_pipeline* pipeline, const void* k_host, const void* v_host,
                              int32_t k_length, int32_t q_tokens, int32_t q_local_offset,
                              int32_t causal_shift, double softmax_scale, int32_t causal,
                              void* compute_stream, sa_pipeline_stats* stats);

/*
 * Stream one contiguous K/V span of a segment: host rows k_host/v_host hold
 * segment positions [kv_local_offset, kv_local_offset + kv_tokens).  The span
 * goes through the ring in chunks of at most kv_chunk_tokens rows and every
 * chunk updates the resident Q block.  Paged mode coalesces consecutive
 * pages of a segment into one span (replaces the per-page loop of
 * paged/runtime/triton.py:109-238, whose kernel launches cover one page each).
 * *initialize: in, nonzero while the state still has to be defined by the
 * next launch (the first span of a Q block); out, 0 once a launch did.  With
 * kv_tokens == 0 and *initialize set, the state is initialized to "no keys".
 * Ring slots rotate across calls; the H2D copies are on the pipeline's H2D
 * stream, so an event recorded there after this call marks the host rows as
 * consumed.
 */
int32_t sa_pipeline_stream_kv_span(sa_pipeline* pipeline, const void* k_host, const void* v_host,
                                   int32_t kv_tokens, int32_t kv_local_offset,
                                   int32_t* initialize, int32_t q_tokens,
                                   int32_t q_local_offset, int32_t causal_shift,
                                   double softmax_scale, int32_t causal, void* compute_stream,
                                   sa_pipeline_stats* stats);

/*
 * Gathered form of sa_pipeline_stream_kv_span for paged sources: the span's
 * host rows are split over num_fragments contiguous fragments (one per
 * page: K rows k_fragments[i], V rows v_fragments[i], fragment_tokens[i]
 * rows each), in segment order starting at kv_local_offset.  Fragments are
 * packed into ring slots of up to kv_chunk_tokens rows with one H2D copy per
 * piece, and each slot is one update launch (the reference copies a page
 * into a pinned stage and launches per page, paged/runtime/triton.py:119-238).
 * Fragment memory must stay valid and unmodified until an event recorded on
 * the H2D stream after this call has completed.
 */
int32_t sa_pipeline_stream_kv_gather(sa_pipeline* pipeline, const void* const* k_fragments,
                                     const void* const* v_fragments,
                                     const int32_t* fragment_tokens, int32_t num_fragments,
                                     int32_t kv_local_offset, int32_t* initialize,
                                     int32_t q_tokens, int32_t q_local_offset,
                                     int32_t causal_shift, double softmax_scale, int32_t causal,
                                     void* compute_stream, sa_pipeline_stats* stats);

/*
 * INT8 K/V pages (PagedAttentionConfig.kv_storage_dtype == "int8"): give the
 * pipeline one fp16 scale buffer per ring slot for K and for V, each holding
 * kv_chunk_tokens * kv_heads values (row-major [row, kv_head]).  num_slots
 * must equal the ring size; head_dim must be a multiple of 16 up to 128.
 * No counterpart in the reference, whose paged workspace allocates per-slot
 * group-scale tensors itself (paged/runtime/staging.py:97-107).
 */
int32_t sa_pipeline_attach_int8_scales(sa_pipeline* pipeline, void* const* k_scale_slots,
                                       void* const* v_scale_slots, int32_t num_slots);

/*
 * sa_pipeline_stream_kv_gather for INT8 pages: fragment i holds
 * fragment_tokens[i] int8 rows of kv_heads * head_dim bytes (K and V) and one
 * fp16 scale per (row, K/V head) (k_scale_fragments[i], v_scale_fragments[i],
 * kv_heads values per row).  Rows and scales are gathered into a ring slot
 * and its scale slots and each slot is one INT8 update launch that
 * dequantizes in the kernel, as update_attention_state_int8 does for a page
 * (reference paged/runtime/triton.py:139-200).  Requires
 * sa_pipeline_attach_int8_scales.
 */
int32_t sa_pipeline_stream_kv_gather_int8(sa_pipeline* pipeline, const void* const* k_fragments,
                                          const void* const* v_fragments,
                                          const void* const* k_scale_fragments,
                                          const void* const* v_scale_fragments,
                                          const int32_t* fragment_tokens, int32_t num_fragments,
                                          int32_t kv_local_offset, int32_t* initialize,
                                          int32_t q_tokens, int32_t q_local_offset,
                                          int32_t causal_shift, double softmax_scale,
                                          int32_t causal, void* compute_stream,
                                          sa_pipeline_stats* stats);

/*
 * HBM-resident execution: Q/K/V and out are device tensors (strides in
 * elements, unit stride over head_dim), so nothing crosses PCIe.  Same Q
 * super-block / K/V chunk decomposition as sa_pipeline_run, using the
 * pipeline's state buffers; K/V chunks and Q blocks are read in place and
 * each block is finalized straight into out (and lse when non-NULL, layout
 * [q_heads, total_q] with row stride lse_stride_h).  When kv_chunk_tokens is
 * a multiple of 64 and out is 16-byte aligned with strides that are multiples
 * of 8, each segment is one update launch over all of its queries and keys
 * that finalizes in its epilogue and merges the row sums at every chunk
 * boundary, so the result equals sa_pipeline_run's bit for bit; the state
 * buffers are then untouched.  Enqueued on compute_stream; returns without
 * waiting.  The reference accepts host
 * tensors only (validation.py:13-14); this is the device-input extension.
 */
int32_t sa_pipeline_run_resident(sa_pipeline* pipeline, const void* q, const void* k,
                                 const void* v, void* out, float* lse, int64_t stride_qt,
                                 int64_t stride_qh, int64_t stride_kt, int64_t stride_kh,
                                 int64_t stride_vt, int64_t stride_vh, int64_t stride_ot,
                                 int64_t stride_oh, int64_t lse_stride_h,
                                 const int64_t* cu_seqlens_q, const int64_t* cu_seqlens_k,
                                 int32_t num_segments, double softmax_scale, int32_t causal,
                                 void* compute_stream, sa_pipeline_stats* stats);

/*
 * Attach caller-owned device scratch for sa_pipeline_run_resident (NULL and 0
 * detach it).  No counterpart in the reference.  With head_dim 128, a fused
 * resident launch whose segment has kv_tokens keys first copies V into it,
 * transposed per K/V head ([kv_heads][128][keys padded to a multiple of 64],
 * 16-bit), when kv_heads * 128 * roundup(kv_tokens, 64) * 2 bytes fit; the
 * update kernel then reads V^T fragments with half the LDS instructions.
 * Results are identical with or without it.  The pipeline keeps the pointer
 * until it is replaced or the pipeline is destroyed; runs on one pipeline
 * share it, in stream order.
 */
int32_t sa_pipeline_attach_resident_scratch(sa_pipeline* pipeline, void* scratch, int64_t bytes);

/*
 * Finalize the resident state on compute_stream (executor.py:125-142).
 * slot >= 0: into output slot `slot`; the Q-free event is recorded first (the
 * next Q H2D may start) and finalize waits for the slot's previous D2H.
 * slot == -1: into q_buffer itself (device-consumer Q reuse); Q stays held
 * until sa_pipeline_d2h(release_q=1) or sa_pipeline_release_q.
 * lse as in sa_finalize_attention (NULL for none).
 */
int32_t sa_pipeline_finalize(sa_pipeline* pipeline, int32_t slot, int32_t q_tokens,
                             float* lse, int64_t lse_stride_h, int64_t lse_token_offset,
                             void* compute_stream);

/*
 * Finalize the resident state straight into a caller device buffer `dest`
 * with strides (stride_ot, stride_oh, 1) on compute_stream: the output stays
 * in HBM and no D2H is issued.  The Q-free event is recorded first.
 */
int32_t sa_pipeline_finalize_into(sa_pipeline* pipeline, void* dest, int64_t stride_ot,
                                  int64_t stride_oh, int32_t q_tokens, float* lse,
                                  int64_t lse_stride_h, int64_t lse_token_offset,
                                  void* compute_stream);

/* Record the Q-free event on compute_stream (a consumer produced a new tensor
 * and no longer needs the Q buffer, executor.py:170-172). */
int32_t sa_pipeline_release_q(sa_pipeline* pipeline, void* compute_stream);

/*
 * D2H of `bytes` from device `src` to pinned host `dst_host` on the D2H stream
 * after everything enqueued on compute_stream so far (executor.py:173-184).
 * Output events of `event_slot` (0 <= event_slot < num_output_buffers) fence
 * the next finalize into that slot; release_q != 0 (src lives in q_buffer)
 * records the Q-free event on the D2H stream.
 */
int32_t sa_pipeline_d2h(sa_pipeline* pipeline, void* dst_host, const void* src, int64_t bytes,
                        int32_t event_slot, int32_t release_q, void* compute_stream,
                        sa_pipeline_stats* stats);

/* Block until the D2H stream has drained. */
int32_t sa_pipeline_synchronize(sa_pipeline* pipeline);

/*
 * Kernel timing of the update launches: with enable != 0, every later update
 * launch of the pipeline is bracketed by a pair of timing events on the
 * stream it is launched on (the compute stream, or the pipeline's second
 * stream for the concurrent half of a split chunk update).
 * sa_pipeline_kernel_timing waits for the recorded launches, returns their
 * summed duration (ms) and count, and resets the record.
 * sa_pipeline_kernel_busy does the same and also returns the length of the
 * union of the launch intervals (ms): the time at least one update launch
 * was running, in which overlapping half-launches count once.
 */
int32_t sa_pipeline_set_kernel_timing(sa_pipeline* pipeline, int32_t enable);

/*
 * Host-side trace ranges: with enable != 0 the pipeline brackets the enqueue
 * of each stage with ROCm tracer (roctx) ranges named like the reference's
 * NVTX ranges (streaming/executor.py:53-174, enabled there by
 * config.enable_nvtx): "seqattn:q_h2d", "seqattn:kv_h2d",
 * "seqattn:fused_update", "seqattn:fused_finalize", "seqattn:output_d2h".
 * The tracer library is loaded on first use; SA_ERR_BAD_STATE when it is
 * missing.
 */
int32_t sa_pipeline_set_trace_ranges(sa_pipeline* pipeline, int32_t enable);
int32_t sa_pipeline_kernel_timing(sa_pipeline* pipeline, double* total_ms, int64_t* launches);
int32_t sa_pipeline_kernel_busy(sa_pipeline* pipeline, double* busy_ms, double* total_ms,
                                int64_t* launches);

/*
 * sa_run_resident_noalloc: attention over HBM-resident Q/K/V into a
 * caller-owned device output (and LSE), allocating nothing.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It computes what sa_pipeline_run_resident computes for
 * head_dim 128 with transposed-V scratch attached, bit for bit (same
 * launches: a V transpose per segment, then one fused update launch whose
 * row sums merge at every kv_chunk_tokens boundary), but the transposed V
 * lives in a fixed 64 MiB device array inside the library (one per GPU,
 * held until the process ends) instead of caller-provided scratch.
 * Limits: head_dim 128; per segment kv_heads * 128 * (keys rounded up to
 * 64) * 2 bytes <= 64 MiB (for example 8 K/V heads x 32,768 keys), larger
 * segments are rejected before anything is enqueued.  Calls on one GPU share
 * its array: calls that overlap on that GPU (other streams or threads) race.
 * Strides are in elements; lse may be NULL.  Enqueued on `stream`.
 */
int32_t sa_run_resident_noalloc(const void* q, const void* k, const void* v, void* out, float* lse,
                                int64_t stride_qt, int64_t stride_qh, int64_t stride_kt,
                                int64_t stride_kh, int64_t stride_vt, int64_t stride_vh,
                                int64_t stride_ot, int64_t stride_oh, int64_t lse_stride_h,
                                const int64_t* cu_seqlens_q, const int64_t* cu_seqlens_k,
                                int32_t num_segments, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, int32_t dtype, int32_t kv_chunk_tokens,
                                double softmax_scale, int32_t causal, void* stream);

/* hipStream_t of the pipeline's H2D (which == 0) or D2H (which == 1) copy stream. */
void* sa_pipeline_stream(sa_pipeline* pipeline, int32_t which);

/* Device pointers: output slot `index` (NULL without slots) and the Q buffer. */
void* sa_pipeline_output_slot(sa_pipeline* pipeline, int32_t index);
void* sa_pipeline_q_buffer(sa_pipeline* pipeline);

#ifdef __cplusplus
}
#endif

#endif /* SEQATTN_HIP_H */
