/*
 * rq_hip.h - C ABI of the MI355X-native ResidualQuant packed KV-cache path.
 *
 * One shared library (residualquant_amd/librq_hip.so, built for gfx950 with
 * hipcc) exports these symbols.  Every entry point takes plain device
 * pointers, sizes and strides (in elements), enqueues on the caller's HIP
 * stream and returns 0 on success or a negative RQ_E* code; the message of
 * the last failure on the calling thread is rq_last_error().  Validation of
 * sizes, schedules and alignment happens on the host before any device work.
 *
 * Reference interface (heejunkim00/ResidualQuant, paths relative to
 * plugins/residual_quantization/csrc/): the pybind11 ops attention()/quantize()
 * declared at common/api.h:11-31 and exported at dispatch/binding.cpp:19-38.
 */
#ifndef RQ_HIP_H
#define RQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RQ_OK = 0,
    RQ_EINVAL = -1,    /* invalid argument (TORCH_CHECK in the reference) */
    RQ_ENOKERNEL = -2, /* no kernel for this geometry/schedule (kernel_registry.h:66-72) */
    RQ_ELAUNCH = -3,   /* HIP launch or runtime error */
    RQ_ENOSPACE = -4   /* workspace smaller than rq_attention_workspace_bytes() */
};

/* reference_mode */
enum { RQ_MODE_ANCHOR = 0, RQ_MODE_ADJACENT = 1 };
/* coefficient_method (quantize/types.h:4: Unit, Norm, LeastSquares) */
enum { RQ_COEF_UNIT = 0, RQ_COEF_NORM = 1, RQ_COEF_LS = 2 };

/* Library version, (major << 16) | minor. */
int rq_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* rq_last_error(void);

/*
 * Bytes of one token row of a packed page: sum over records of
 * D*bits/8 + 2*D/group + 2.  Replaces QuantizationRecord::Bytes /
 * PackedLayout::PageWidth (common/cache.cuh:14-17, :78-80) and
 * DeferredKVGroup.page_width (src/residual_quantization/install_model.py:34-38).
 * Returns a negative code for an invalid schedule.
 */
int rq_page_width(int head_dim, int records, const int* bits, const int* groups);

/*
 * Quantize-on-write of one completed loop group into the paged cache.
 * Replaces quantize() (quantize/api.cpp:8-95 -> launch_quantize,
 * quantize/launch.cuh:43-86 -> quantize_kernel, quantize/kernel.cuh:332-355).
 *
 * key_ptrs[r], value_ptrs[r]: BF16 [rows_r, heads, head_dim], channel stride
 *   1, head stride head_dim, token stride key_strides[r] / value_strides[r]
 *   (elements); input_rows = min over inputs of rows_r (must be >= tokens).
 * kv_cache: UINT8 [2, num_blocks, heads, page_tokens, page_width], contiguous.
 * slot_mapping: INT64 [tokens]; slot < 0 leaves the cache untouched.
 * key_rotation / value_rotation: FP16 [heads, D, D] or NULL (y = x . R).
 * key_mean: FP32 [records, heads, D] or NULL (subtracted from K after rotation).
 * bits[r], groups[r]: record schedule in loop order.
 */
int rq_quantize(int records, const void* const* key_ptrs, const int64_t* key_strides,
                const void* const* value_ptrs, const int64_t* value_strides, int64_t input_rows,
                void* kv_cache, int64_t num_blocks, int heads, int page_tokens, int page_width,
                const int64_t* slot_mapping, int64_t tokens, int head_dim,
                const void* key_rotation, const void* value_rotation, const float* key_mean,
                const int* bits, const int* groups, int reference_mode, int anchor_index,
                int coefficient, hipStream_t stream);

/*
 * Device workspace that rq_attention needs for `rows` query rows (query.size(0))
 * and a page table of `max_pages` columns (block_table.size(1)).  Depends
 * only on host shapes, so a captured graph can reuse one allocation.
 */
size_t rq_attention_workspace_bytes(int64_t rows, int heads, int head_dim, int64_t max_pages,
                                    int page_tokens);

/*
 * Split-K paged decode attention over packed pages for loop `loop_index`.
 * Replaces attention() (attention/api.cpp:8-115 -> launch_attention,
 * attention/launch.cuh:33-132 -> prepare/compute/merge kernels).
 *
 * query, key, value, output: BF16 [rows, heads, head_dim] with the given
 *   token strides (elements); key/value are the current token (not yet in
 *   the cache).  Row i belongs to the request b with
 *   query_start_loc[b] <= i < query_start_loc[b+1] and attends to
 *   seq_lens[b]-1 history tokens read through block_table[b][t/page_tokens].
 * block_table: INT32 [>= requests, max_pages], row stride block_table_stride.
 * workspace: device memory of at least rq_attention_workspace_bytes(...).
 */
int rq_attention(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                 const void* value, int64_t value_stride, void* output, int64_t output_stride,
                 int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                 int page_tokens, int page_width, const int32_t* query_start_loc,
                 const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                 int64_t block_table_stride, int64_t max_pages, const void* key_rotation,
                 const void* value_rotation, const float* key_mean, int records,
                 const int* bits, const int* groups, int reference_mode, int anchor_index,
                 int loop_index, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Attention of each request's last n tokens over its packed history: request
 * b's rows query_start_loc[b]..query_start_loc[b+1] (n of them) are its last
 * n of seq_lens[b] tokens; row r attends to the first seq_lens[b] - n tokens
 * through block_table and, causally, to the request's new key/value rows
 * 0..r.  The prefill of a prompt chunk over a packed prefix: no counterpart
 * in the reference, whose scheduler forbids partial prefill and cached
 * prefixes (src/residual_quantization/scheduler.py:11-18).  Arguments,
 * validation and workspace (rq_attention_workspace_bytes) are those of
 * rq_attention (head_dim 96 or 128, anchor or adjacent mode).  A request
 * may have no new rows.  rq_attention itself routes calls with an average
 * of 2 or more rows per request (3 in the anchor-only loop) to the same
 * multi-row kernels (each row then sees seq_lens[b] - 1 history tokens and
 * its own key/value, the reference's semantics).
 */
int rq_packed_prefill_attention(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                                const void* value, int64_t value_stride, void* output, int64_t output_stride,
                                int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                                int page_tokens, int page_width, const int32_t* query_start_loc,
                                const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                                int64_t block_table_stride, int64_t max_pages, const void* key_rotation,
                                const void* value_rotation, const float* key_mean, int records, const int* bits,
                                const int* groups, int reference_mode, int anchor_index, int loop_index,
                                void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * rq_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, whose
 * attention() allocates its temporaries per call (attention/launch.cuh:85-98).
 * Same arguments, semantics, kernels and results as rq_attention; the
 * workspace is a static device array of RQ_ATTENTION_NOALLOC_MAX_BYTES per
 * GPU, held until the process ends.  A call whose route needs more returns
 * RQ_ENOSPACE before any device work: the per-row decode kernels need
 * (272 + 130 x splits) x 4 bytes per (row, head), about 5 000 (row, head)
 * pairs at one split; the multi-row kernels (2 or more rows per request)
 * (132 x splits + 1) x 4 bytes, about 2 000 pairs at eight splits.
 * (rq_attention_workspace_bytes covers both routes, so it may exceed the
 * scratch for a call that still fits.)
 * Every noalloc call on one GPU shares that array.  Eager calls are ordered
 * by the library, across streams and host threads: a call on another stream
 * than the previous call first makes its stream wait for the previous
 * call's kernels (one event per GPU, created with the scratch lookup on the
 * first call on that GPU; it holds no device memory).  Calls captured into a
 * graph are not ordered against work outside the graph: replays of a graph
 * holding noalloc calls race with other noalloc work on the same GPU and
 * must be serialized by the caller.  Calls no hipMalloc/hipFree and records
 * no timing events.
 */
#define RQ_ATTENTION_NOALLOC_MAX_BYTES ((size_t)8 << 20)
int rq_attention_noalloc(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                         const void* value, int64_t value_stride, void* output, int64_t output_stride,
                         int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                         int page_tokens, int page_width, const int32_t* query_start_loc,
                         const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                         int64_t block_table_stride, int64_t max_pages, const void* key_rotation,
                         const void* value_rotation, const float* key_mean, int records, const int* bits,
                         const int* groups, int reference_mode, int anchor_index, int loop_index,
                         hipStream_t stream);

/*
 * Restore the BF16 K/V of `loop_index` at the given slots (rotated space,
 * K including its mean): the record value the quantizer keeps as its
 * reference (quantize/kernel.cuh:160-203; attention/compute.cuh:28-197).
 * key_out / value_out: BF16 [tokens, heads, head_dim], contiguous; slot < 0
 * gives zeros.  No counterpart op in the reference's Python surface; it
 * exposes the reconstruction both reference kernels perform internally.
 */
int rq_dequantize(const void* kv_cache, int64_t num_blocks, int heads, int page_tokens,
                  int page_width, const int64_t* slots, int64_t tokens, int head_dim,
                  const float* key_mean, int records, const int* bits, const int* groups,
                  int reference_mode, int anchor_index, int loop_index, void* key_out,
                  void* value_out, hipStream_t stream);

/*
 * BF16 paged decode attention with the same split-K skeleton: the
 * comparison baseline of the decode metric.  Cache BF16
 * [2, num_blocks, heads, page_tokens, head_dim], contiguous.  No counterpart
 * in the reference (it compares against vLLM's own BF16 backend).
 */
int rq_paged_attention_bf16(const void* query, int64_t query_stride, const void* key,
                            int64_t key_stride, const void* value, int64_t value_stride,
                            void* output, int64_t output_stride, int64_t rows, int heads,
                            int head_dim, const void* cache, int64_t num_blocks, int page_tokens,
                            const int32_t* query_start_loc, const int32_t* seq_lens,
                            int64_t requests, const int32_t* block_table,
                            int64_t block_table_stride, int64_t max_pages, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/*
 * Causal (or full) varlen prefill attention over raw BF16 Q/K/V:
 * out[i] = softmax(softmax_scale * q_i K_j^T over keys j <= i + len_k - len_q) V
 * per sequence s = [cu_seqlens[s], cu_seqlens[s + 1]) and head (query head h
 * reads key/value head h / (heads_q / heads_k)).  Replaces the
 * flash_attn_varlen_func(q, k, v, out, cu_seqlens_q, cu_seqlens_k,
 * max_seqlen_q, max_seqlen_k, softmax_scale, causal) call of the full-prompt
 * branch, src/residual_quantization/packed_backend.py:63-77 (vLLM 0.10.2).
 * Q/K/V/output rows [tokens, heads, head_dim] with element strides per token,
 * 8-byte aligned; cu_seqlens int32 [batch + 1] on the device; max_seqlen_q
 * and max_seqlen_k must be at least every sequence's query and key length.
 * head_dim 96 or 128.  `workspace` holds rq_prefill_workspace_bytes(...)
 * bytes of device memory (may be null when that is 0).
 */
int rq_prefill_attention(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                         const void* value, int64_t value_stride, void* output, int64_t output_stride,
                         int heads_q, int heads_k, int head_dim, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int64_t batch, int64_t max_seqlen_q,
                         int64_t max_seqlen_k, float softmax_scale, int causal, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/*
 * Workspace bytes rq_prefill_attention needs for these host shapes.  The
 * current kernels merge within their workgroups and return 0; callers that
 * allocate what this returns keep working if a later plan needs scratch.
 * same_lengths = 1 when cu_seqlens_q and cu_seqlens_k are the same array.
 * No counterpart in the reference (flash-attn sizes its own scratch).
 */
size_t rq_prefill_workspace_bytes(int64_t batch, int heads_q, int head_dim, int64_t max_seqlen_q,
                                  int64_t max_seqlen_k, int causal, int same_lengths);

/*
 * Elementwise callers on either side of the packed attention in one layer of
 * the looped (Ouro) decoder, plugins/looped_transformers/src/looped_transformers/ouro.py:101-157.
 *
 * rq_rms_norm replaces vLLM's RMSNorm (layernorm.py), used as
 * input_layernorm / input_layernorm_2 / post_attention_layernorm(_2)
 * (ouro.py:132-157) and the loop's final norm (ouro.py:240): with a residual,
 * total = bf16(x + residual) is written to residual_out (which may alias
 * residual) and normalized; without one, x is normalized.
 * y = bf16(bf16(total * rsqrt(mean(total^2) + eps)) * weight), mean over the
 * hidden channels in FP32.  With pre_weight, x is first replaced by its own
 * RMSNorm with pre_weight (same eps), which fuses a norm that feeds a fused
 * add (input_layernorm_2 -> post_attention_layernorm, ouro.py:154-155, and
 * post_attention_layernorm_2 -> the next layer's input_layernorm or the
 * final norm) into one launch.  BF16 rows, 16-byte aligned, strides
 * multiples of 8 elements; hidden a multiple of 8 up to 2048.
 */
int rq_rms_norm(const void* x, int64_t x_stride, const void* pre_weight, const void* residual,
                int64_t residual_stride, void* residual_out, int64_t residual_out_stride, const void* weight, void* y,
                int64_t y_stride, int64_t rows, int hidden, float eps, hipStream_t stream);

/*
 * Rotate-half rotary embedding of the Q and K of fused [q | k | v] BF16 rows
 * (the rotary_emb(positions, query, key) call, ouro.py:93-99, :109, with
 * rotary_dim = head_dim): for i < head_dim / 2,
 * out[i] = x[i] cos - x[i + d/2] sin, out[i + d/2] = x[i + d/2] cos + x[i] sin,
 * cos/sin FP32 tables [table_rows, head_dim / 2] indexed by the int64
 * position of each row (clamped to the table).  Optionally also writes the
 * rotated K and the raw V to key_stage / value_stage rows (the loop-group
 * staging of the packed backend, src/residual_quantization/packed_backend.py:101-137).
 */
int rq_rope_qkv(const void* qkv, int64_t qkv_stride, const int64_t* positions, const float* cos_table,
                const float* sin_table, int64_t table_rows, int heads, int head_dim, int64_t rows, void* query,
                int64_t query_stride, void* key, int64_t key_stride, void* key_stage, void* value_stage,
                int64_t stage_stride, hipStream_t stream);

/*
 * out = bf16(silu(gate) * up) over [gate | up] BF16 rows of 2 * width: the
 * SiluAndMul activation of Qwen2MLP (ouro.py:125-131).
 */
int rq_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride, int64_t rows, int width,
                hipStream_t stream);

/*
 * y = bf16(x . weight^T) for 1-8 BF16 rows x [rows, in_features] and a
 * contiguous BF16 weight [out_features, in_features] (a linear layer's
 * weight as nn.Linear holds it), FP32 accumulation: the QKV, O, gate/up and
 * down projections of a decode step at small batch (ouro.py:101-131 runs
 * them through vLLM's linear layers), where the product is a stream of the
 * weights.  in_features a multiple of 8 up to 6144; x and weight 16-byte
 * aligned, x_stride a multiple of 8.  More rows return RQ_ENOKERNEL.
 */
int rq_linear_rows(const void* x, int64_t x_stride, const void* weight, void* y, int64_t y_stride, int64_t rows,
                   int64_t out_features, int64_t in_features, hipStream_t stream);

/*
 * Kernel timing for measurement: when enabled, rq_attention and
 * rq_paged_attention_bf16 record HIP events around their split-K kernel on
 * the caller's stream; rq_timing_read() synchronizes the recorded events and
 * returns the summed milliseconds and the launch count, then clears them.
 */
void rq_timing_enable(int enabled);
int rq_timing_read(double* milliseconds, int64_t* launches);

/* Split-K sizing: target number of split-K workgroups per launch (0 = default). */
void rq_set_split_target(int workgroups);

#ifdef __cplusplus
}
#endif

#endif /* RQ_HIP_H */
