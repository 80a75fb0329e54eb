// Launch parameters shared between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rq_device.h"

namespace rq {

// Workgroups of `threads` threads of `kernel` that one compute unit holds at
// once (its registers and LDS decide), at least 1.
inline int resident_per_cu(const void* kernel, int threads) {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, 0) != hipSuccess || blocks < 1)
        return 1;
    return blocks;
}

// Coefficient methods (same values as RQ_COEF_* in include/rq_hip.h).
constexpr int RQ_COEF_UNIT_ = 0;
constexpr int RQ_COEF_NORM_ = 1;
constexpr int RQ_COEF_LS_ = 2;

struct QuantizeParams {
    const uint16_t* key_ptrs[kMaxRecords];
    const uint16_t* value_ptrs[kMaxRecords];
    int64_t key_strides[kMaxRecords];
    int64_t value_strides[kMaxRecords];
    uint8_t* cache;
    int64_t plane_stride;  // num_blocks * heads * page_tokens * page_width
    int64_t num_blocks;
    const int64_t* slots;
    int64_t tokens;
    const uint16_t* key_rotation;  // FP16 bits [heads, D, D] or null
    const uint16_t* value_rotation;
    const float* key_mean;  // FP32 [records, heads, D] or null
    int heads, page_tokens, page_width, records, anchor, adjacent, coefficient;
    int page_shift;     // log2(page_tokens): page tokens are 16 or 32
    int compute_units;  // of the launching device, for grid sizing
    RecordRegion region[kMaxRecords];
};

hipError_t launch_quantize(const QuantizeParams& p, int head_dim, hipStream_t stream);

struct RestoreParams {
    const uint8_t* cache;
    int64_t plane_stride, num_blocks;
    int heads, page_tokens, page_width, head_dim;
    const int64_t* slots;
    int64_t tokens;
    const float* key_mean;
    int chain_length;            // records restored in order
    int chain[kMaxRecords];      // record indices, base first
    RecordRegion region[kMaxRecords];
    uint16_t* key_out;
    uint16_t* value_out;
};

hipError_t launch_restore(const RestoreParams& p, hipStream_t stream);

struct PrefillParams {
    const uint16_t* query;   // BF16 [tokens_q, heads_q, D], token stride query_stride
    int64_t query_stride;
    const uint16_t* key;     // BF16 [tokens_k, heads_k, D]
    int64_t key_stride;
    const uint16_t* value;
    int64_t value_stride;
    uint16_t* output;        // BF16 [tokens_q, heads_q, D]
    int64_t output_stride;
    const int32_t* cu_seqlens_q;  // [batch + 1]
    const int32_t* cu_seqlens_k;
    int batch;
    int heads_q;
    int group;               // heads_q / heads_k
    int head_dim;
    int max_seqlen_q;
    int causal;
    float softmax_scale;
    // Plan (prefill_plan in prefill.hip): each workgroup takes a pair of
    // 128-query blocks of one (sequence, head) and merges within itself, so
    // no workspace is needed.
    int query_blocks;         // ceil(max_seqlen_q / 128)
    int items;                // block pairs per (head, sequence)
};

constexpr int kPrefillBlockQueries = 128;
constexpr int kPrefillBlockKeys = 64;

// Fills the plan fields of `p` from its shape fields; returns the workspace bytes.
size_t prefill_plan(PrefillParams& p, int64_t max_seqlen_k);
hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream);

// Fused elementwise kernels of the looped-model decode step (step_ops.hip).
struct StepNormParams {
    const uint16_t* x;          // BF16 [rows, hidden]
    int64_t x_stride;
    const uint16_t* pre_weight; // optional: x is first RMS-normalized with this weight
    const uint16_t* residual;   // optional BF16 [rows, hidden] added to x first
    int64_t residual_stride;
    uint16_t* residual_out;     // optional: receives bf16(x + residual) (may alias residual)
    int64_t residual_out_stride;
    const uint16_t* weight;     // BF16 [hidden]
    uint16_t* y;
    int64_t y_stride;
    int64_t rows;
    int hidden;                 // multiple of 8, at most 2048
    float eps;
};

struct StepRopeParams {
    const uint16_t* qkv;        // BF16 [rows, 3 * heads * head_dim]
    int64_t qkv_stride;
    const int64_t* positions;   // [rows]
    const float* cos_table;     // [positions, head_dim / 2]
    const float* sin_table;
    int64_t table_rows;         // positions are clamped to [0, table_rows - 1]
    int heads, head_dim;
    int64_t rows;
    uint16_t* q;
    int64_t q_stride;
    uint16_t* k;
    int64_t k_stride;
    uint16_t* k_stage;          // optional copies of the rotated K and of V
    uint16_t* v_stage;
    int64_t stage_stride;
};

hipError_t launch_rms_norm(const StepNormParams& p, hipStream_t stream);
hipError_t launch_rope(const StepRopeParams& p, hipStream_t stream);
// y = bf16(x . w^T) for 1 <= rows <= kLinearMaxRows rows of x [rows, in],
// w [out, in] contiguous; in_features a multiple of 8 up to 6144.
constexpr int kLinearMaxRows = 8;
hipError_t launch_linear_rows(const uint16_t* x, int64_t x_stride, const uint16_t* w, uint16_t* y, int64_t y_stride,
                              int rows, int out_features, int in_features, hipStream_t stream);
hipError_t launch_silu_mul(const uint16_t* gate_up, int64_t gate_up_stride, uint16_t* out, int64_t out_stride,
                           int64_t rows, int width, hipStream_t stream);

// Per (row, head) prepared query block in the workspace (floats).
constexpr int kPrepScalars = 16;   // [0] delta [1] live score [2] q'.mu_A [3..10] Q16 [11..14] Q32
constexpr int kPrepQuery = 128;    // q' FP32 in log2 units
constexpr int kPrepPlanes = 64;    // 4 nibble planes x up to 16 words (each order)
constexpr int kPrepFloats = kPrepScalars + kPrepQuery + 2 * kPrepPlanes;
constexpr int kMaxSplits = 64;

struct AttentionParams {
    const uint16_t* query;
    int64_t query_stride;
    const uint16_t* key;
    int64_t key_stride;
    const uint16_t* value;
    int64_t value_stride;
    uint16_t* output;
    int64_t output_stride;
    int64_t rows;
    int heads;
    int head_dim;
    const uint8_t* cache;      // packed UINT8 or BF16 pages (baseline)
    int64_t plane_stride;      // bytes between the K and V planes
    int64_t num_blocks;
    int page_tokens;
    int page_width;            // bytes per token row of a page (packed)
    const int32_t* query_start_loc;
    const int32_t* seq_lens;
    int64_t requests;
    const int32_t* block_table;
    int64_t block_table_stride;
    int64_t max_pages;
    const uint16_t* key_rotation;
    const uint16_t* value_rotation;
    const float* key_mean_loop;    // mu of the current loop [heads, D] or null
    const float* key_mean_anchor;  // mu of the anchor [heads, D] or null (residual loops only)
    RecordRegion anchor;
    RecordRegion residual;
    int has_residual;
    int32_t* row_request;  // workspace [rows]
    int32_t* arrivals;     // workspace [rows, heads]: finished splits (zeroed by prepare)
    float* prep;           // workspace [rows, heads, kPrepFloats]
    float* partials;       // workspace [rows, heads, splits, D + 2]
    int splits;
    int fused_prepare;     // 1: each decode workgroup prepares its own query (requires splits == 1)
    int compute_units;     // of the launching device
    int stream_priority;   // set by the launch: the grid fits the device at once, so its waves take StreamPriority
    // Adjacent mode, loop L > 0: records 0..L of the restore chain (chain_length = L + 1, else 0)
    // and the key means of every record [records, heads, D] (or null).
    RecordRegion chain[kMaxRecords];
    int chain_length;
    const float* key_mean_all;
};

hipError_t launch_attention(const AttentionParams& p, hipStream_t stream, hipEvent_t begin,
                            hipEvent_t end);

// Several query rows per request over packed pages (D = 96 or 128, anchor
// and adjacent mode): one workgroup per (request, head, row tile of 32 rows,
// history split) streams the split's pages once for all the tile's rows on
// MFMA tiles, then a finish launch per (row, head) merges the splits,
// applies R_v^T and adds the live tokens.  causal = 0: the reference decode
// semantics (history seq_len - 1, the row's own live token); causal = 1: the
// rows are the request's last n tokens (history seq_len - n, live tokens
// j <= r).
constexpr int kMultiRowEntry = 132;        // per (row, head, split): m, l, 2 unused, O[D <= 128] (log2 units)
constexpr int kMultiRowMaxSplits = 8;      // for parallelism (more only for very long histories)
constexpr int kMultiRowMaxSplitPages = 1024;  // pages of one split at most
struct MultiRowParams {
    const uint16_t* query;
    int64_t query_stride;
    const uint16_t* key;
    int64_t key_stride;
    const uint16_t* value;
    int64_t value_stride;
    uint16_t* output;
    int64_t output_stride;
    int64_t rows;
    int heads;
    int head_dim;  // 96 or 128
    const uint8_t* cache;
    int64_t plane_stride;
    int64_t num_blocks;
    int page_tokens;
    int page_width;
    const int32_t* query_start_loc;
    const int32_t* seq_lens;
    int64_t requests;
    const int32_t* block_table;
    int64_t block_table_stride;
    int64_t max_pages;
    const uint16_t* key_rotation;
    const uint16_t* value_rotation;
    const float* key_mean_loop;    // [heads, D] or null
    const float* key_mean_anchor;  // [heads, D] or null (anchor mode, residual loops only)
    RecordRegion anchor;
    RecordRegion residual;
    int has_residual;
    // Adjacent mode past loop 0: the restore chain over records 0..L
    // (chain_length = L + 1 >= 2; 0 in anchor mode) and every record's key
    // mean [records, heads, D] (or null).
    int chain_length;
    RecordRegion chain[kMaxRecords];
    const float* key_mean_all;
    int causal;
    int splits;     // history splits per (request, head, row tile)
    int compute_units;    // of the launching device
    int stream_priority;  // set by the launch: the active workgroups fit the device at once, so their
                          // waves take StreamPriority
    int row_tiles;  // 32-row tiles per request in the finish grid (the stream grid takes 16 or 32 rows a tile)
    float* partials;   // workspace [rows, heads, splits, kMultiRowEntry]
    float* row_shift;  // workspace [rows, heads]: q'.mu_L in log2 units
};
hipError_t launch_multirow(const MultiRowParams& p, hipStream_t stream);
hipError_t launch_attention_bf16(const AttentionParams& p, hipStream_t stream, hipEvent_t begin,
                                 hipEvent_t end);

}  // namespace rq
