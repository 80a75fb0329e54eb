// extern "C" entry points of librq_hip.so (declared in include/rq_hip.h).
//
// Host-side validation mirrors the reference's TORCH_CHECKs
// (plugins/residual_quantization/csrc/quantize/api.cpp:18-85,
// attention/api.cpp:23-104, dispatch/kernel_registry.h:42-72) for what a
// pointer-and-size interface can see; dtype/device/stride checks of tensors
// belong to the caller (residualquant_amd/ops.py).  Every failure returns a
// negative code and leaves its message in rq_last_error() for the thread.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/rq_hip.h"
#include "rq_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* format, ...) {
    char buffer[512];
    va_list args;
    va_start(args, format);
    std::vsnprintf(buffer, sizeof(buffer), format, args);
    va_end(args);
    g_last_error = buffer;
    return code;
}

int ok() {
    g_last_error.clear();
    return RQ_OK;
}

int check_launch(hipError_t status, const char* what) {
    if (status != hipSuccess) return fail(RQ_ELAUNCH, "%s: %s", what, hipGetErrorString(status));
    return ok();
}

// Supported geometry: the head dims and page sizes the reference registers
// (dispatch/schedules.cuh:147-148, attention/compute.cuh:279-282) and INT2/INT4
// records with groups of 16 or 32 (common/cache.cuh:31-34, :82-96).
int validate_schedule(int head_dim, int records, const int* bits, const int* groups, int page_tokens,
                      int reference_mode, int anchor_index, int heads) {
    if (records < 1 || records > 4 || bits == nullptr || groups == nullptr)
        return fail(RQ_EINVAL, "A nonempty group of at most 4 records is required");
    if (reference_mode != RQ_MODE_ANCHOR && reference_mode != RQ_MODE_ADJACENT)
        return fail(RQ_EINVAL, "Unknown packed reference mode: %d", reference_mode);
    for (int r = 0; r < records; ++r) {
        if ((bits[r] != 2 && bits[r] != 4) || (groups[r] != 16 && groups[r] != 32) ||
            head_dim % groups[r] != 0)
            return fail(RQ_ENOKERNEL,
                        "No compiled packed HIP kernel for heads=%d, head_dim=%d, record %d=(%d, %d)",
                        heads, head_dim, r, bits[r], groups[r]);
    }
    if ((head_dim != 96 && head_dim != 128) || (page_tokens != 16 && page_tokens != 32) ||
        anchor_index < 0 || anchor_index >= records ||
        (reference_mode == RQ_MODE_ADJACENT && records > 1 && anchor_index != 0))
        return fail(RQ_ENOKERNEL,
                    "No compiled packed HIP kernel for heads=%d, head_dim=%d, record count=%d, "
                    "reference_mode=%s, anchor_index=%d, page_tokens=%d",
                    heads, head_dim, records, reference_mode == RQ_MODE_ANCHOR ? "anchor" : "adjacent",
                    anchor_index, page_tokens);
    return RQ_OK;
}

void fill_regions(int head_dim, int records, const int* bits, const int* groups, int page_tokens,
                  rq::RecordRegion* regions) {
    int offset = 0;
    for (int r = 0; r < records; ++r) {
        regions[r].offset = page_tokens * offset;
        regions[r].bits = bits[r];
        regions[r].group = groups[r];
        regions[r].code_bytes = head_dim * bits[r] / 8;
        regions[r].groups = head_dim / groups[r];
        offset += rq::record_bytes(head_dim, bits[r], groups[r]);
    }
}

// ---------------------------------------------------------------- split sizing

std::mutex g_device_mutex;
std::vector<int> g_compute_units;
int g_split_target = 0;

int compute_units() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(g_device_mutex);
    if ((int)g_compute_units.size() <= device) g_compute_units.resize(device + 1, 0);
    if (g_compute_units[device] == 0) {
        int units = 0;
        if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            units <= 0)
            units = 256;
        g_compute_units[device] = units;
    }
    return g_compute_units[device];
}

// Splits per (row, head): enough workgroups for `target` (by default
// `per_cu` per compute unit: two for the streaming decode kernels, whose long
// page streams per workgroup measured best at batch 32 x 8k, one at D = 96),
// at least 16 pages per split, at most rq::kMaxSplits.  With 4 pages per
// split a one-row call's 512 workgroups spent their time in the prologue and
// the merge: 4-call step at batch 1, 16 heads, 2048 history 90.3 -> 74.1 us
// with 16 pages (4096: 93.3 -> 83.9 us; 8192 and every batch-8 shape keep
// their counts and times).
int split_count(int64_t rows, int heads, int64_t max_pages, int per_cu = 2) {
    int64_t target;
    {
        std::lock_guard<std::mutex> lock(g_device_mutex);
        target = g_split_target;
    }
    if (target <= 0) target = (int64_t)per_cu * compute_units();
    const int64_t pairs = std::max<int64_t>(1, rows * heads);
    int64_t splits = (target + pairs - 1) / pairs;
    const int64_t by_pages = std::max<int64_t>(1, (max_pages + 15) / 16);
    splits = std::min<int64_t>(splits, std::min<int64_t>(by_pages, rq::kMaxSplits));
    return (int)std::max<int64_t>(1, splits);
}

size_t align256(size_t bytes) { return (bytes + 255) & ~size_t(255); }

struct WorkspaceLayout {
    size_t row_request, arrivals, prep, partials, total;
};

constexpr int64_t kMultiRowMinRows = 3;          // anchor-loop calls
constexpr int64_t kMultiRowMinRowsResidual = 2;  // residual-loop calls

// Several rows per request (either head dim, either mode) run the multi-row
// MFMA kernels: one workgroup per (request, head, 32-row tile, history split).
// Two stream workgroups fit a compute unit.  Splits are the count at or just
// below the one that fills those slots once over `groups` = requests x heads
// x row tiles (one round, which the wave priority by stream progress levels)
// or the count just above it, whichever leaves the busiest compute unit the
// least history: ceil(groups s / CUs) / s of a group's pages, the smaller
// count on a tie.  Measured per residual call (16 rows per request): 440
// groups (C4 history) 133.3 us at 2 splits against 117.9 us at 1; 192 groups
// 135.3 us at 3 against 115.9 us at 2; 384 groups 205 us at 2 against 224 us
// at 1.  At most kMultiRowMaxSplits, no more than the history's 32-token tiles
// allow (four per split, one per wave), and at least enough that no split
// holds more than kMultiRowMaxSplitPages pages.  The count never grows with
// the groups, so the workspace is sized for the most splits any call of these
// row and head counts can take (one request).
int multirow_splits(int64_t groups, int64_t max_pages, int page_tokens) {
    const int64_t units = compute_units();
    const int64_t target = 2LL * units;
    const int64_t g = std::max<int64_t>(1, groups);
    const int64_t below = std::max<int64_t>(1, target / g), above = std::max<int64_t>(1, (target + g - 1) / g);
    // Busiest compute unit's share, compared as ceil(g s / units) / s by cross-multiplying.
    auto busiest = [&](int64_t s) { return (g * s + units - 1) / units; };
    int64_t splits = busiest(above) * below < busiest(below) * above ? above : below;
    const int64_t tiles = std::max<int64_t>(1, (max_pages * page_tokens + 31) / 32);
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, tiles / 4));
    splits = std::min<int64_t>(splits, rq::kMultiRowMaxSplits);
    const int64_t tiles_per_split_max = (int64_t)(rq::kMultiRowMaxSplitPages - 1) * page_tokens / 32;
    splits = std::max<int64_t>(splits, (tiles + tiles_per_split_max - 1) / tiles_per_split_max);
    return (int)std::max<int64_t>(1, splits);
}

// The most splits a multi-row call of `rows` rows can take.  A call runs
// requests x heads x average_tiles groups, with average_tiles =
// max(1, ceil(floor(rows / requests) / 32)) (attention_packed); over every
// request count that product is at least ceil(rows / 33) x heads, so
// heads x max(1, rows / 64) is a lower bound on the groups, and
// multirow_splits, which never grows with the groups, is bounded by its
// value there.
int multirow_workspace_splits(int64_t rows, int heads, int64_t max_pages, int page_tokens) {
    const int64_t min_groups = (int64_t)heads * std::max<int64_t>(1, rows / 64);
    return multirow_splits(min_groups, max_pages, page_tokens);
}

struct MultiRowLayout {
    size_t partials, row_shift, total;
};

MultiRowLayout multirow_layout(int64_t rows, int heads, int splits) {
    MultiRowLayout w;
    w.partials = 0;
    w.row_shift = align256(sizeof(float) * (size_t)rows * heads * splits * rq::kMultiRowEntry);
    w.total = w.row_shift + align256(sizeof(float) * (size_t)rows * heads);
    return w;
}

WorkspaceLayout workspace_layout(int64_t rows, int heads, int head_dim, int splits) {
    WorkspaceLayout w;
    w.row_request = 0;
    w.arrivals = align256(sizeof(int32_t) * (size_t)rows);
    w.prep = w.arrivals + align256(sizeof(int32_t) * (size_t)rows * heads);
    w.partials = w.prep + align256(sizeof(float) * (size_t)rows * heads * rq::kPrepFloats);
    w.total = w.partials + align256(sizeof(float) * (size_t)rows * heads * splits * (head_dim + 2));
    return w;
}

// ---------------------------------------------------------------- timing

struct TimingState {
    std::mutex mutex;
    bool enabled = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> free_pairs;
};
TimingState g_timing;

bool timing_events(hipStream_t stream, hipEvent_t* begin, hipEvent_t* end) {
    *begin = *end = nullptr;
    std::lock_guard<std::mutex> lock(g_timing.mutex);
    if (!g_timing.enabled) return false;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone)
        return false;
    std::pair<hipEvent_t, hipEvent_t> pair;
    if (!g_timing.free_pairs.empty()) {
        pair = g_timing.free_pairs.back();
        g_timing.free_pairs.pop_back();
    } else {
        if (hipEventCreate(&pair.first) != hipSuccess) return false;
        if (hipEventCreate(&pair.second) != hipSuccess) {
            (void)hipEventDestroy(pair.first);
            return false;
        }
    }
    g_timing.pending.push_back(pair);
    *begin = pair.first;
    *end = pair.second;
    return true;
}

}  // namespace

extern "C" {

int rq_version(void) { return (0 << 16) | 1; }

const char* rq_last_error(void) { return g_last_error.c_str(); }

int rq_page_width(int head_dim, int records, const int* bits, const int* groups) {
    if (records < 1 || records > rq::kMaxRecords || bits == nullptr || groups == nullptr || head_dim <= 0 ||
        head_dim % 32 != 0)
        return fail(RQ_EINVAL, "Head dimension must be a positive multiple of 32 with 1-8 records");
    int width = 0;
    for (int r = 0; r < records; ++r) {
        if ((bits[r] != 2 && bits[r] != 4) || groups[r] <= 0 || head_dim % groups[r] != 0)
            return fail(RQ_EINVAL, "Head dimension must be divisible by every quantization group size");
        width += rq::record_bytes(head_dim, bits[r], groups[r]);
    }
    ok();
    return width;
}

int rq_quantize(int records, const void* const* key_ptrs, const int64_t* key_strides,
                const void* const* value_ptrs, const int64_t* value_strides, int64_t input_rows,
                void* kv_cache, int64_t num_blocks, int heads, int page_tokens, int page_width,
                const int64_t* slot_mapping, int64_t tokens, int head_dim, const void* key_rotation,
                const void* value_rotation, const float* key_mean, const int* bits, const int* groups,
                int reference_mode, int anchor_index, int coefficient, hipStream_t stream) {
    if (records < 1 || key_ptrs == nullptr || value_ptrs == nullptr || key_strides == nullptr ||
        value_strides == nullptr)
        return fail(RQ_EINVAL, "A nonempty group with one K/V input per record required");
    if (kv_cache == nullptr || num_blocks < 0 || heads <= 0 || page_tokens <= 0)
        return fail(RQ_EINVAL,
                    "Contiguous CUDA UINT8 [2, blocks, heads, page tokens, page width] cache required");
    int status = validate_schedule(head_dim, records, bits, groups, page_tokens, reference_mode,
                                   anchor_index, heads);
    if (status != RQ_OK) return status;
    if (coefficient < RQ_COEF_UNIT || coefficient > RQ_COEF_LS) return fail(RQ_EINVAL, "Unsupported coefficient");
    if (tokens < 0 || (tokens > 0 && slot_mapping == nullptr))
        return fail(RQ_EINVAL, "Contiguous INT64 slot mapping on the cache device required");
    if (input_rows < tokens) return fail(RQ_EINVAL, "Input has fewer rows than slot mapping");
    const int width = rq_page_width(head_dim, records, bits, groups);
    if (width != page_width) return fail(RQ_EINVAL, "Packed cache width differs from records");
    for (int r = 0; r < records; ++r)
        if ((tokens > 0 && (key_ptrs[r] == nullptr || value_ptrs[r] == nullptr)) ||
            key_strides[r] < (int64_t)heads * head_dim || value_strides[r] < (int64_t)heads * head_dim)
            return fail(RQ_EINVAL, "BF16 [tokens, heads, channels] with packed trailing strides required");
    // The rotation phase reads input rows with 8-byte scalar loads and stages
    // each FP16 rotation with 16-byte loads.
    for (int r = 0; r < records; ++r)
        if (reinterpret_cast<uintptr_t>(key_ptrs[r]) % 8 || reinterpret_cast<uintptr_t>(value_ptrs[r]) % 8 ||
            key_strides[r] % 4 || value_strides[r] % 4)
            return fail(RQ_EINVAL, "K/V addresses and token strides must be 8-byte aligned");
    if (reinterpret_cast<uintptr_t>(key_rotation) % 16 || reinterpret_cast<uintptr_t>(value_rotation) % 16)
        return fail(RQ_EINVAL, "Rotation addresses must be 16-byte aligned");
    if (tokens == 0) return ok();

    rq::QuantizeParams p{};
    for (int r = 0; r < records; ++r) {
        p.key_ptrs[r] = static_cast<const uint16_t*>(key_ptrs[r]);
        p.value_ptrs[r] = static_cast<const uint16_t*>(value_ptrs[r]);
        p.key_strides[r] = key_strides[r];
        p.value_strides[r] = value_strides[r];
    }
    p.cache = static_cast<uint8_t*>(kv_cache);
    p.plane_stride = num_blocks * heads * (int64_t)page_tokens * page_width;
    p.num_blocks = num_blocks;
    p.slots = slot_mapping;
    p.tokens = tokens;
    p.key_rotation = static_cast<const uint16_t*>(key_rotation);
    p.value_rotation = static_cast<const uint16_t*>(value_rotation);
    p.key_mean = key_mean;
    p.heads = heads;
    p.page_tokens = page_tokens;
    p.page_width = page_width;
    p.records = records;
    p.anchor = anchor_index;
    // A single-record group is always its own anchor (dispatch/schedules.cuh:99-111).
    p.adjacent = records > 1 && reference_mode == RQ_MODE_ADJACENT;
    p.coefficient = coefficient;
    p.page_shift = page_tokens == 32 ? 5 : 4;
    p.compute_units = compute_units();
    fill_regions(head_dim, records, bits, groups, page_tokens, p.region);
    return check_launch(rq::launch_quantize(p, head_dim, stream), "quantize launch");
}

// One workspace serves both paths of a packed attention call (the per-row
// decode kernels and the multi-row kernels), so its size is the larger one.
static int chain_splits(int64_t rows, int heads, int64_t max_pages);

static size_t attention_workspace_total(int64_t rows, int heads, int head_dim, int64_t max_pages,
                                        int page_tokens) {
    const int splits = std::max(split_count(rows, heads, max_pages), chain_splits(rows, heads, max_pages));
    size_t total = workspace_layout(rows, heads, head_dim, splits).total;
    if ((head_dim == 96 || head_dim == 128) && (page_tokens == 16 || page_tokens == 32))
        total = std::max(total,
                         multirow_layout(rows, heads, multirow_workspace_splits(rows, heads, max_pages, page_tokens)).total);
    return total;
}

// RQ_ENOSPACE for a workspace smaller than the route of the call needs; a
// call of rq_attention_noalloc names its static scratch instead.
static int workspace_too_small(size_t needed, size_t got, bool static_scratch) {
    if (static_scratch)
        return fail(RQ_ENOSPACE,
                    "rq_attention_noalloc: this call needs %zu bytes of scratch, the static scratch holds %zu; "
                    "call rq_attention with a workspace instead",
                    needed, got);
    return fail(RQ_ENOSPACE, "Attention workspace of %zu bytes required (got %zu)", needed, got);
}

size_t rq_attention_workspace_bytes(int64_t rows, int heads, int head_dim, int64_t max_pages,
                                    int page_tokens) {
    if (rows <= 0 || heads <= 0 || head_dim <= 0) return 256;
    return attention_workspace_total(rows, heads, head_dim, max_pages, page_tokens);
}

static int attention_common(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                            const void* value, int64_t value_stride, void* output, int64_t output_stride,
                            int64_t rows, int heads, int head_dim, const int32_t* query_start_loc,
                            const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                            int64_t block_table_stride, int64_t max_pages, void* workspace,
                            size_t workspace_bytes, int splits, rq::AttentionParams* p,
                            bool static_scratch = false) {
    if (rows < 0 || heads <= 0) return fail(RQ_EINVAL, "Q/K/V/output must have matching shapes and devices");
    if (rows > 0 && (query == nullptr || key == nullptr || value == nullptr || output == nullptr))
        return fail(RQ_EINVAL, "Q/K/V/output must have matching shapes and devices");
    const int64_t min_stride = (int64_t)heads * head_dim;
    if (query_stride < min_stride || key_stride < min_stride || value_stride < min_stride ||
        output_stride < min_stride)
        return fail(RQ_EINVAL, "BF16 [tokens, heads, channels] with packed trailing strides required");
    if ((reinterpret_cast<uintptr_t>(query) % 8) != 0 || (reinterpret_cast<uintptr_t>(key) % 8) != 0 ||
        query_stride % 4 != 0 || key_stride % 4 != 0)
        return fail(RQ_EINVAL, "Q/K addresses and token strides must be 8-byte aligned");
    if (requests < 0 || (requests > 0 && (query_start_loc == nullptr || seq_lens == nullptr)))
        return fail(RQ_EINVAL, "Contiguous INT32 query starts with one final boundary required");
    if ((rows > 0 && block_table == nullptr) || max_pages < 0 || block_table_stride < max_pages)
        return fail(RQ_EINVAL, "INT32 page table with packed rows required");
    if (splits <= 0) return RQ_OK;  // validation only
    const WorkspaceLayout layout = workspace_layout(rows, heads, head_dim, splits);
    if (rows > 0 && (workspace == nullptr || workspace_bytes < layout.total))
        return workspace_too_small(layout.total, workspace_bytes, static_scratch);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    *p = rq::AttentionParams{};
    p->query = static_cast<const uint16_t*>(query);
    p->query_stride = query_stride;
    p->key = static_cast<const uint16_t*>(key);
    p->key_stride = key_stride;
    p->value = static_cast<const uint16_t*>(value);
    p->value_stride = value_stride;
    p->output = static_cast<uint16_t*>(output);
    p->output_stride = output_stride;
    p->rows = rows;
    p->heads = heads;
    p->head_dim = head_dim;
    p->query_start_loc = query_start_loc;
    p->seq_lens = seq_lens;
    p->requests = requests;
    p->block_table = block_table;
    p->block_table_stride = block_table_stride;
    p->max_pages = max_pages;
    p->row_request = reinterpret_cast<int32_t*>(ws + layout.row_request);
    p->arrivals = reinterpret_cast<int32_t*>(ws + layout.arrivals);
    p->prep = reinterpret_cast<float*>(ws + layout.prep);
    p->partials = reinterpret_cast<float*>(ws + layout.partials);
    p->splits = splits;
    return RQ_OK;
}

// Splits per (row, head) of a packed attention call.  At D = 96 a call takes
// one workgroup per (row, head) once those fill the compute units: every loop
// runs decode96_dma_kernel (one token half per lane, pages staged in LDS),
// which prepares its query inside the decode launch (one launch per call; at
// 55 heads x B8 x 4096 the residual call measured 82.1, 85.8, 92.4 and 92.3
// us at 1, 2, 3 and 4 splits).
static int packed_splits(int64_t rows, int heads, int head_dim, int64_t max_pages) {
    return split_count(rows, heads, max_pages, head_dim == 96 ? 1 : 2);
}

// Splits per (row, head) of an adjacent-mode call past loop 0
// (decode_chain_kernel).  That kernel is bound by its VALU work, not by HBM,
// and shorter page spans per workgroup let one workgroup's prologue and
// finish overlap another's chain: at batch 32 x 8k x 16 heads, loops 1 / 2 /
// 3 measured 364 / 512 / 660 us at two workgroups per compute unit and
// 320 / 498 / 628 us at eight.
static int chain_splits(int64_t rows, int heads, int64_t max_pages) {
    return split_count(rows, heads, max_pages, 8);
}

static int attention_packed(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                            const void* value, int64_t value_stride, void* output, int64_t output_stride,
                            int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                            int page_tokens, int page_width, const int32_t* query_start_loc,
                            const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                            int64_t block_table_stride, int64_t max_pages, const void* key_rotation,
                            const void* value_rotation, const float* key_mean, int records, const int* bits,
                            const int* groups, int reference_mode, int anchor_index, int loop_index,
                            void* workspace, size_t workspace_bytes, hipStream_t stream, bool timed,
                            bool causal = false, bool static_scratch = false) {
    int status = validate_schedule(head_dim, records, bits, groups, page_tokens, reference_mode,
                                   anchor_index, heads);
    if (status != RQ_OK) return status;
    if (loop_index < 0 || loop_index >= records) return fail(RQ_EINVAL, "Invalid loop index");
    if (kv_cache == nullptr || num_blocks < 0)
        return fail(RQ_EINVAL, "Contiguous UINT8 KV cache on the query device required");
    if (key_mean != nullptr && (reinterpret_cast<uintptr_t>(key_mean) % 16) != 0)
        return fail(RQ_EINVAL,
                    "16-byte aligned contiguous FP32 key mean with matching dimensions required");
    if (key_rotation != nullptr && (reinterpret_cast<uintptr_t>(key_rotation) % 16) != 0)
        return fail(RQ_EINVAL, "16-byte aligned key rotation required for asynchronous copies");
    if (value_rotation != nullptr && (reinterpret_cast<uintptr_t>(value_rotation) % 16) != 0)
        return fail(RQ_EINVAL, "16-byte aligned value rotation required");
    const int width = rq_page_width(head_dim, records, bits, groups);
    if (width != page_width) return fail(RQ_EINVAL, "Packed cache width differs from records");
    const bool adjacent = records > 1 && reference_mode == RQ_MODE_ADJACENT;
    // Several rows per request (and every prefill over packed history) take
    // the multi-row MFMA kernels, which stream each request's pages once for
    // all its rows but dequantize every page tile into LDS.  Measured at 8192
    // history tokens x 16 heads x D128 in anchor mode (4-call step, multi-row
    // against per-row decode kernel): 3 rows per request 868 against 1462 us
    // (B32), 4 rows 233 against 500 us per residual call, 16 rows 480 against
    // 3280 us (B16); at 2 rows the residual-loop call is faster (228 against
    // 284 us at B32; 129 against 145 us on the 55-head D96 history at B8) but
    // the anchor-only call is not always (D96: 102 against 90 us; adjacent
    // loop 0: 170 against 163 us), so decode calls take them from an average
    // of kMultiRowMinRowsResidual rows per request in a residual loop (and in
    // adjacent mode past loop 0, where the per-row kernel rebuilds the chain
    // once per row) and kMultiRowMinRows in the anchor-only loop.
    const bool anchor_only = adjacent ? loop_index == 0 : loop_index == anchor_index;
    const int64_t min_rows = anchor_only ? kMultiRowMinRows : kMultiRowMinRowsResidual;
    if (causal || (requests > 0 && rows >= min_rows * requests)) {
        status = attention_common(query, query_stride, key, key_stride, value, value_stride, output, output_stride,
                                  rows, heads, head_dim, query_start_loc, seq_lens, requests, block_table,
                                  block_table_stride, max_pages, nullptr, 0, 0, nullptr);
        if (status != RQ_OK) return status;
        if (rows == 0 || requests == 0) return ok();
        // The grid's row tiles cover the longest request the row count allows
        // (a request may have no new rows, so one request may hold them all);
        // the split count is sized from the average request (tiles past a
        // request's rows exit at once, so counting them would take too few
        // splits and leave compute units idle).
        const int64_t row_tiles = (rows + 31) / 32;
        const int64_t average_tiles = std::max<int64_t>(1, (rows / requests + 31) / 32);
        const int splits = multirow_splits(requests * heads * average_tiles, max_pages, page_tokens);
        const MultiRowLayout layout = multirow_layout(rows, heads, splits);
        if (workspace == nullptr || workspace_bytes < layout.total)
            return workspace_too_small(layout.total, workspace_bytes, static_scratch);
        rq::RecordRegion regions[rq::kMaxRecords];
        fill_regions(head_dim, records, bits, groups, page_tokens, regions);
        rq::MultiRowParams m{};
        m.query = static_cast<const uint16_t*>(query);
        m.query_stride = query_stride;
        m.key = static_cast<const uint16_t*>(key);
        m.key_stride = key_stride;
        m.value = static_cast<const uint16_t*>(value);
        m.value_stride = value_stride;
        m.output = static_cast<uint16_t*>(output);
        m.output_stride = output_stride;
        m.rows = rows;
        m.heads = heads;
        m.head_dim = head_dim;
        m.cache = static_cast<const uint8_t*>(kv_cache);
        m.plane_stride = num_blocks * heads * (int64_t)page_tokens * page_width;
        m.num_blocks = num_blocks;
        m.page_tokens = page_tokens;
        m.page_width = page_width;
        m.query_start_loc = query_start_loc;
        m.seq_lens = seq_lens;
        m.requests = requests;
        m.block_table = block_table;
        m.block_table_stride = block_table_stride;
        m.max_pages = max_pages;
        m.key_rotation = static_cast<const uint16_t*>(key_rotation);
        m.value_rotation = static_cast<const uint16_t*>(value_rotation);
        // Adjacent mode: loop 0 is its own anchor (record 0 alone, as the
        // per-row route decodes it); later loops decode the restore chain.
        const int anchor = adjacent ? 0 : anchor_index;
        m.anchor = regions[anchor];
        m.has_residual = !adjacent && loop_index != anchor;
        m.residual = regions[loop_index];
        m.chain_length = adjacent && loop_index > 0 ? loop_index + 1 : 0;
        for (int r = 0; r < m.chain_length; ++r) m.chain[r] = regions[r];
        m.key_mean_all = m.chain_length > 0 ? key_mean : nullptr;
        m.key_mean_loop = key_mean ? key_mean + (int64_t)loop_index * heads * head_dim : nullptr;
        m.key_mean_anchor = (key_mean && m.has_residual) ? key_mean + (int64_t)anchor * heads * head_dim : nullptr;
        m.causal = causal ? 1 : 0;
        m.splits = splits;
        m.row_tiles = (int)row_tiles;
        m.compute_units = compute_units();
        uint8_t* ws = static_cast<uint8_t*>(workspace);
        m.partials = reinterpret_cast<float*>(ws + layout.partials);
        m.row_shift = reinterpret_cast<float*>(ws + layout.row_shift);
        if ((int64_t)m.splits * m.row_tiles > 65535 || requests > (int64_t)INT32_MAX || rows > (int64_t)INT32_MAX)
            return fail(RQ_EINVAL, "Too many rows for one multi-row attention launch");
        hipEvent_t begin = nullptr, end = nullptr;
        if (timed) timing_events(stream, &begin, &end);
        if (begin) (void)hipEventRecord(begin, stream);
        const hipError_t launched = rq::launch_multirow(m, stream);
        if (end) (void)hipEventRecord(end, stream);
        return check_launch(launched, "multi-row attention launch");
    }
    rq::AttentionParams p;
    // Never more splits than rq_attention_workspace_bytes() provides for.
    const int splits = adjacent && loop_index > 0 ? chain_splits(rows, heads, max_pages)
                                                  : packed_splits(rows, heads, head_dim, max_pages);
    const int anchor_record = adjacent ? 0 : anchor_index;
    status = attention_common(query, query_stride, key, key_stride, value, value_stride, output,
                              output_stride, rows, heads, head_dim, query_start_loc, seq_lens, requests,
                              block_table, block_table_stride, max_pages, workspace, workspace_bytes, splits, &p,
                              static_scratch);
    if (status != RQ_OK) return status;
    if (rows == 0) return ok();
    rq::RecordRegion regions[rq::kMaxRecords];
    fill_regions(head_dim, records, bits, groups, page_tokens, regions);
    const int anchor = anchor_record;
    p.cache = static_cast<const uint8_t*>(kv_cache);
    p.plane_stride = num_blocks * heads * (int64_t)page_tokens * page_width;
    p.num_blocks = num_blocks;
    p.page_tokens = page_tokens;
    p.page_width = page_width;
    p.key_rotation = static_cast<const uint16_t*>(key_rotation);
    p.value_rotation = static_cast<const uint16_t*>(value_rotation);
    p.anchor = regions[anchor];
    p.has_residual = loop_index != anchor;
    p.residual = regions[loop_index];
    p.key_mean_loop = key_mean ? key_mean + (int64_t)loop_index * heads * head_dim : nullptr;
    p.key_mean_anchor = (key_mean && p.has_residual) ? key_mean + (int64_t)anchor * heads * head_dim : nullptr;
    p.fused_prepare = p.splits == 1 ? 1 : 0;
    p.compute_units = compute_units();
    // Adjacent mode past loop 0 decodes the restore chain of records 0..loop.
    p.chain_length = adjacent && loop_index > 0 ? loop_index + 1 : 0;
    for (int r = 0; r < p.chain_length; ++r) p.chain[r] = regions[r];
    p.key_mean_all = key_mean;
    hipEvent_t begin = nullptr, end = nullptr;
    if (timed) timing_events(stream, &begin, &end);
    return check_launch(rq::launch_attention(p, stream, begin, end), "attention launch");
}

// ------------------------------------------------- attention without a workspace

// Device scratch of rq_attention_noalloc: the attention workspace (request of
// each row, split arrival counters, query records, split partials) for
// callers that cannot allocate.  Each GPU holds its own copy for the life of
// the process; host code reaches it only through the address that
// hipGetSymbolAddress returns on that device (ScratchState::address), never
// through the name.  Every noalloc call on a GPU shares it; what must start
// at zero (the arrival counters) is cleared by the call's own kernels.
// Calls made eagerly are ordered by the library: a call on another stream
// than the previous one first makes its stream wait for an event recorded
// after the previous call's kernels.  Calls captured into a graph are not
// (a capture cannot wait on work outside it): replays of such a graph must
// not overlap other noalloc work on the same GPU.
constexpr size_t kAttentionScratchBytes = RQ_ATTENTION_NOALLOC_MAX_BYTES;
static __device__ __align__(256) uint8_t scratch[kAttentionScratchBytes];

// Per device: the scratch address, and the event and stream of the last
// eager call (the event holds no device memory and records no timing).
struct ScratchState {
    void* address = nullptr;
    hipEvent_t last_call = nullptr;
    hipStream_t last_stream = nullptr;
    bool has_last = false;
};
static std::mutex g_scratch_mutex;  // held across a call's whole enqueue
static std::vector<ScratchState> g_scratch;

// The current device's state, set up once per device with that device
// current (held lock: g_scratch_mutex).
static int scratch_state(ScratchState** state) {
    int device = 0;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return fail(RQ_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(status));
    if ((int)g_scratch.size() <= device) g_scratch.resize(device + 1);
    ScratchState& s = g_scratch[device];
    if (s.address == nullptr) {
        void* ptr = nullptr;
        status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (status != hipSuccess || ptr == nullptr)
            return fail(RQ_ELAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(status));
        status = hipEventCreateWithFlags(&s.last_call, hipEventDisableTiming);
        if (status != hipSuccess)
            return fail(RQ_ELAUNCH, "hipEventCreateWithFlags(noalloc order): %s", hipGetErrorString(status));
        s.address = ptr;
    }
    *state = &s;
    return RQ_OK;
}

int rq_attention(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                 const void* value, int64_t value_stride, void* output, int64_t output_stride,
                 int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                 int page_tokens, int page_width, const int32_t* query_start_loc, const int32_t* seq_lens,
                 int64_t requests, const int32_t* block_table, int64_t block_table_stride,
                 int64_t max_pages, const void* key_rotation, const void* value_rotation,
                 const float* key_mean, int records, const int* bits, const int* groups,
                 int reference_mode, int anchor_index, int loop_index, void* workspace,
                 size_t workspace_bytes, hipStream_t stream) {
    return attention_packed(query, query_stride, key, key_stride, value, value_stride, output, output_stride,
                            rows, heads, head_dim, kv_cache, num_blocks, page_tokens, page_width,
                            query_start_loc, seq_lens, requests, block_table, block_table_stride, max_pages,
                            key_rotation, value_rotation, key_mean, records, bits, groups, reference_mode,
                            anchor_index, loop_index, workspace, workspace_bytes, stream, true);
}

int rq_packed_prefill_attention(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                                const void* value, int64_t value_stride, void* output, int64_t output_stride,
                                int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                                int page_tokens, int page_width, const int32_t* query_start_loc,
                                const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                                int64_t block_table_stride, int64_t max_pages, const void* key_rotation,
                                const void* value_rotation, const float* key_mean, int records, const int* bits,
                                const int* groups, int reference_mode, int anchor_index, int loop_index,
                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return attention_packed(query, query_stride, key, key_stride, value, value_stride, output, output_stride,
                            rows, heads, head_dim, kv_cache, num_blocks, page_tokens, page_width,
                            query_start_loc, seq_lens, requests, block_table, block_table_stride, max_pages,
                            key_rotation, value_rotation, key_mean, records, bits, groups, reference_mode,
                            anchor_index, loop_index, workspace, workspace_bytes, stream, true, true);
}

int rq_attention_noalloc(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                         const void* value, int64_t value_stride, void* output, int64_t output_stride,
                         int64_t rows, int heads, int head_dim, const void* kv_cache, int64_t num_blocks,
                         int page_tokens, int page_width, const int32_t* query_start_loc,
                         const int32_t* seq_lens, int64_t requests, const int32_t* block_table,
                         int64_t block_table_stride, int64_t max_pages, const void* key_rotation,
                         const void* value_rotation, const float* key_mean, int records, const int* bits,
                         const int* groups, int reference_mode, int anchor_index, int loop_index,
                         hipStream_t stream) {
    // The route the call takes (per-row or multi-row kernels) checks its own
    // workspace size against the scratch, before any device work.
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchState* state = nullptr;
    int status = scratch_state(&state);
    if (status != RQ_OK) return status;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t error = hipStreamIsCapturing(stream, &capture);
    if (error != hipSuccess) return fail(RQ_ELAUNCH, "hipStreamIsCapturing: %s", hipGetErrorString(error));
    const bool eager = capture == hipStreamCaptureStatusNone;
    if (eager && state->has_last && state->last_stream != stream) {
        // The previous call ran on another stream: this one starts after it.
        error = hipStreamWaitEvent(stream, state->last_call, 0);
        if (error != hipSuccess) return fail(RQ_ELAUNCH, "hipStreamWaitEvent: %s", hipGetErrorString(error));
    }
    status = attention_packed(query, query_stride, key, key_stride, value, value_stride, output, output_stride,
                              rows, heads, head_dim, kv_cache, num_blocks, page_tokens, page_width,
                              query_start_loc, seq_lens, requests, block_table, block_table_stride, max_pages,
                              key_rotation, value_rotation, key_mean, records, bits, groups, reference_mode,
                              anchor_index, loop_index, state->address, kAttentionScratchBytes, stream, false,
                              false, true);
    if (status == RQ_OK && eager) {
        error = hipEventRecord(state->last_call, stream);
        if (error != hipSuccess) return fail(RQ_ELAUNCH, "hipEventRecord: %s", hipGetErrorString(error));
        state->last_stream = stream;
        state->has_last = true;
    }
    return status;
}

int rq_dequantize(const void* kv_cache, int64_t num_blocks, int heads, int page_tokens, int page_width,
                  const int64_t* slots, int64_t tokens, int head_dim, const float* key_mean, int records,
                  const int* bits, const int* groups, int reference_mode, int anchor_index, int loop_index,
                  void* key_out, void* value_out, hipStream_t stream) {
    int status = validate_schedule(head_dim, records, bits, groups, page_tokens, reference_mode,
                                   anchor_index, heads);
    if (status != RQ_OK) return status;
    if (loop_index < 0 || loop_index >= records) return fail(RQ_EINVAL, "Invalid loop index");
    if (kv_cache == nullptr || num_blocks < 0 || tokens < 0 || (tokens > 0 && (slots == nullptr ||
                                                                              key_out == nullptr ||
                                                                              value_out == nullptr)))
        return fail(RQ_EINVAL, "Packed cache, slots and BF16 outputs required");
    const int width = rq_page_width(head_dim, records, bits, groups);
    if (width != page_width) return fail(RQ_EINVAL, "Packed cache width differs from records");
    if (tokens == 0) return ok();
    rq::RestoreParams p{};
    p.cache = static_cast<const uint8_t*>(kv_cache);
    p.plane_stride = num_blocks * heads * (int64_t)page_tokens * page_width;
    p.num_blocks = num_blocks;
    p.heads = heads;
    p.page_tokens = page_tokens;
    p.page_width = page_width;
    p.head_dim = head_dim;
    p.slots = slots;
    p.tokens = tokens;
    p.key_mean = key_mean;
    const bool adjacent = records > 1 && reference_mode == RQ_MODE_ADJACENT;
    p.chain_length = 0;
    if (adjacent) {
        for (int r = 0; r <= loop_index; ++r) p.chain[p.chain_length++] = r;
    } else {
        p.chain[p.chain_length++] = anchor_index;
        if (loop_index != anchor_index) p.chain[p.chain_length++] = loop_index;
    }
    fill_regions(head_dim, records, bits, groups, page_tokens, p.region);
    p.key_out = static_cast<uint16_t*>(key_out);
    p.value_out = static_cast<uint16_t*>(value_out);
    return check_launch(rq::launch_restore(p, stream), "restore launch");
}

int rq_paged_attention_bf16(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                            const void* value, int64_t value_stride, void* output, int64_t output_stride,
                            int64_t rows, int heads, int head_dim, const void* cache, int64_t num_blocks,
                            int page_tokens, const int32_t* query_start_loc, const int32_t* seq_lens,
                            int64_t requests, const int32_t* block_table, int64_t block_table_stride,
                            int64_t max_pages, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if ((head_dim != 96 && head_dim != 128) || (page_tokens != 16 && page_tokens != 32))
        return fail(RQ_ENOKERNEL, "No compiled BF16 paged kernel for head_dim=%d, page_tokens=%d", head_dim,
                    page_tokens);
    if (cache == nullptr || num_blocks < 0) return fail(RQ_EINVAL, "BF16 paged cache required");
    rq::AttentionParams p;
    int status = attention_common(query, query_stride, key, key_stride, value, value_stride, output,
                                  output_stride, rows, heads, head_dim, query_start_loc, seq_lens, requests,
                                  block_table, block_table_stride, max_pages, workspace, workspace_bytes,
                                  split_count(rows, heads, max_pages), &p);
    if (status != RQ_OK) return status;
    if (rows == 0) return ok();
    p.cache = static_cast<const uint8_t*>(cache);
    p.plane_stride = num_blocks * heads * (int64_t)page_tokens * head_dim * 2;
    p.num_blocks = num_blocks;
    p.page_tokens = page_tokens;
    p.page_width = head_dim * 2;
    hipEvent_t begin, end;
    timing_events(stream, &begin, &end);
    return check_launch(rq::launch_attention_bf16(p, stream, begin, end), "bf16 attention launch");
}

int rq_prefill_attention(const void* query, int64_t query_stride, const void* key, int64_t key_stride,
                         const void* value, int64_t value_stride, void* output, int64_t output_stride,
                         int heads_q, int heads_k, int head_dim, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int64_t batch, int64_t max_seqlen_q,
                         int64_t max_seqlen_k, float softmax_scale, int causal, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
    if (head_dim != 96 && head_dim != 128)
        return fail(RQ_ENOKERNEL, "No compiled prefill attention kernel for head_dim=%d", head_dim);
    if (heads_q <= 0 || heads_k <= 0 || heads_q % heads_k != 0)
        return fail(RQ_EINVAL, "Query heads must be a positive multiple of key/value heads");
    if (batch < 0 || max_seqlen_q < 0 || max_seqlen_q > (int64_t)INT32_MAX || max_seqlen_k < 0 ||
        max_seqlen_k > (int64_t)INT32_MAX || batch > 65535)
        return fail(RQ_EINVAL, "Invalid batch, max_seqlen_q or max_seqlen_k");
    if (batch > 0 && (cu_seqlens_q == nullptr || cu_seqlens_k == nullptr))
        return fail(RQ_EINVAL, "cu_seqlens_q and cu_seqlens_k required");
    if (!(softmax_scale > 0.f) || !std::isfinite(softmax_scale)) return fail(RQ_EINVAL, "softmax_scale must be positive");
    const int64_t q_row = (int64_t)heads_q * head_dim, k_row = (int64_t)heads_k * head_dim;
    if (query_stride < q_row || output_stride < q_row || key_stride < k_row || value_stride < k_row)
        return fail(RQ_EINVAL, "BF16 [tokens, heads, head_dim] with packed trailing strides required");
    const void* rows[4] = {query, key, value, output};
    const int64_t strides[4] = {query_stride, key_stride, value_stride, output_stride};
    for (int i = 0; i < 4; ++i)
        if ((reinterpret_cast<uintptr_t>(rows[i]) % 8) || strides[i] % 4)
            return fail(RQ_EINVAL, "Q/K/V/output addresses and token strides must be 8-byte aligned");
    if (batch == 0 || max_seqlen_q == 0) return ok();
    if (query == nullptr || key == nullptr || value == nullptr || output == nullptr)
        return fail(RQ_EINVAL, "Q/K/V/output required");
    rq::PrefillParams p{};
    p.query = static_cast<const uint16_t*>(query);
    p.query_stride = query_stride;
    p.key = static_cast<const uint16_t*>(key);
    p.key_stride = key_stride;
    p.value = static_cast<const uint16_t*>(value);
    p.value_stride = value_stride;
    p.output = static_cast<uint16_t*>(output);
    p.output_stride = output_stride;
    p.cu_seqlens_q = cu_seqlens_q;
    p.cu_seqlens_k = cu_seqlens_k;
    p.batch = (int)batch;
    p.heads_q = heads_q;
    p.group = heads_q / heads_k;
    p.head_dim = head_dim;
    p.max_seqlen_q = (int)max_seqlen_q;
    p.causal = causal != 0;
    p.softmax_scale = softmax_scale;
    const size_t needed = rq::prefill_plan(p, max_seqlen_k);
    if (needed > 0 && (workspace == nullptr || workspace_bytes < needed))
        return fail(RQ_ENOSPACE, "Prefill workspace of %zu bytes required, %zu given", needed, workspace_bytes);
    return check_launch(rq::launch_prefill(p, stream), "prefill attention launch");
}

int rq_rms_norm(const void* x, int64_t x_stride, const void* pre_weight, const void* residual,
                int64_t residual_stride, void* residual_out, int64_t residual_out_stride, const void* weight, void* y,
                int64_t y_stride, int64_t rows, int hidden, float eps, hipStream_t stream) {
    if (rows < 0 || rows > (int64_t)INT32_MAX || hidden <= 0 || hidden % 8 != 0 || hidden > 2048)
        return fail(RQ_EINVAL, "RMSNorm needs rows >= 0 and a hidden size that is a multiple of 8 up to 2048");
    if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(RQ_EINVAL, "RMSNorm eps must be finite and non-negative");
    if ((residual == nullptr) != (residual_out == nullptr))
        return fail(RQ_EINVAL, "A residual input and a residual output go together");
    if (rows == 0) return ok();
    const void* pointers[6] = {x, weight, y, residual, residual_out, pre_weight};
    const int64_t strides[6] = {x_stride, 0, y_stride, residual_stride, residual_out_stride, 0};
    for (int i = 0; i < 6; ++i) {
        if (i < 3 && pointers[i] == nullptr) return fail(RQ_EINVAL, "RMSNorm input, weight and output required");
        if (pointers[i] == nullptr) continue;
        if ((reinterpret_cast<uintptr_t>(pointers[i]) % 16) || strides[i] % 8 ||
            (i != 1 && i != 5 && strides[i] < hidden))
            return fail(RQ_EINVAL, "RMSNorm rows must be 16-byte aligned BF16 rows of at least hidden elements");
    }
    rq::StepNormParams p{};
    p.x = static_cast<const uint16_t*>(x);
    p.x_stride = x_stride;
    p.pre_weight = static_cast<const uint16_t*>(pre_weight);
    p.residual = static_cast<const uint16_t*>(residual);
    p.residual_stride = residual_stride;
    p.residual_out = static_cast<uint16_t*>(residual_out);
    p.residual_out_stride = residual_out_stride;
    p.weight = static_cast<const uint16_t*>(weight);
    p.y = static_cast<uint16_t*>(y);
    p.y_stride = y_stride;
    p.rows = rows;
    p.hidden = hidden;
    p.eps = eps;
    return check_launch(rq::launch_rms_norm(p, stream), "RMSNorm launch");
}

int rq_rope_qkv(const void* qkv, int64_t qkv_stride, const int64_t* positions, const float* cos_table,
                const float* sin_table, int64_t table_rows, int heads, int head_dim, int64_t rows, void* query,
                int64_t query_stride, void* key, int64_t key_stride, void* key_stage, void* value_stage,
                int64_t stage_stride, hipStream_t stream) {
    if (rows < 0 || rows > (int64_t)INT32_MAX || heads <= 0 || heads > 32768 || head_dim <= 0 || head_dim % 2 != 0)
        return fail(RQ_EINVAL, "Rotary embedding needs rows >= 0, heads > 0 and an even head_dim");
    const int64_t row = (int64_t)heads * head_dim;
    if (qkv_stride < 3 * row || query_stride < row || key_stride < row ||
        ((key_stage != nullptr || value_stage != nullptr) && stage_stride < row))
        return fail(RQ_EINVAL, "Fused [q | k | v] rows and [heads, head_dim] outputs required");
    if (rows == 0) return ok();
    if (table_rows <= 0 || qkv == nullptr || positions == nullptr || cos_table == nullptr || sin_table == nullptr ||
        query == nullptr || key == nullptr)
        return fail(RQ_EINVAL, "QKV, positions, cos/sin tables and Q/K outputs required");
    rq::StepRopeParams p{};
    p.qkv = static_cast<const uint16_t*>(qkv);
    p.qkv_stride = qkv_stride;
    p.positions = positions;
    p.cos_table = cos_table;
    p.sin_table = sin_table;
    p.table_rows = table_rows;
    p.heads = heads;
    p.head_dim = head_dim;
    p.rows = rows;
    p.q = static_cast<uint16_t*>(query);
    p.q_stride = query_stride;
    p.k = static_cast<uint16_t*>(key);
    p.k_stride = key_stride;
    p.k_stage = static_cast<uint16_t*>(key_stage);
    p.v_stage = static_cast<uint16_t*>(value_stage);
    p.stage_stride = stage_stride;
    return check_launch(rq::launch_rope(p, stream), "rotary embedding launch");
}

int rq_silu_mul(const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride, int64_t rows, int width,
                hipStream_t stream) {
    if (rows < 0 || rows > 65535 || width <= 0 || width % 2 != 0)
        return fail(RQ_EINVAL, "SiLU-mul needs 0 <= rows <= 65535 and an even width");
    if (gate_up_stride < 2 * (int64_t)width || out_stride < width || gate_up_stride % 2 || out_stride % 2)
        return fail(RQ_EINVAL, "[gate | up] rows of 2 * width and output rows of width required (even strides)");
    if (rows == 0) return ok();
    if (gate_up == nullptr || out == nullptr || (reinterpret_cast<uintptr_t>(gate_up) % 4) ||
        (reinterpret_cast<uintptr_t>(out) % 4))
        return fail(RQ_EINVAL, "4-byte aligned gate/up input and output required");
    return check_launch(rq::launch_silu_mul(static_cast<const uint16_t*>(gate_up), gate_up_stride,
                                            static_cast<uint16_t*>(out), out_stride, rows, width, stream),
                        "SiLU-mul launch");
}

int rq_linear_rows(const void* x, int64_t x_stride, const void* weight, void* y, int64_t y_stride, int64_t rows,
                   int64_t out_features, int64_t in_features, hipStream_t stream) {
    if (rows < 0 || rows > rq::kLinearMaxRows)
        return fail(RQ_ENOKERNEL, "No compiled row-projection kernel for %lld rows (at most %d)", (long long)rows,
                    rq::kLinearMaxRows);
    if (out_features <= 0 || out_features > (int64_t)INT32_MAX || in_features <= 0 || in_features % 8 != 0 ||
        in_features > 6144)
        return fail(RQ_EINVAL, "Projection needs out_features > 0 and in_features a multiple of 8 up to 6144");
    if (x_stride < in_features || x_stride % 8 != 0 || y_stride < out_features)
        return fail(RQ_EINVAL, "x rows of in_features (stride a multiple of 8) and y rows of out_features required");
    if (rows == 0) return ok();
    if (x == nullptr || weight == nullptr || y == nullptr || (reinterpret_cast<uintptr_t>(x) % 16) ||
        (reinterpret_cast<uintptr_t>(weight) % 16) || (reinterpret_cast<uintptr_t>(y) % 2))
        return fail(RQ_EINVAL, "16-byte aligned x and weight and a BF16 output required");
    return check_launch(rq::launch_linear_rows(static_cast<const uint16_t*>(x), x_stride,
                                               static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(y),
                                               y_stride, (int)rows, (int)out_features, (int)in_features, stream),
                        "row projection launch");
}

size_t rq_prefill_workspace_bytes(int64_t batch, int heads_q, int head_dim, int64_t max_seqlen_q,
                                  int64_t max_seqlen_k, int causal, int same_lengths) {
    if (batch <= 0 || heads_q <= 0 || head_dim <= 0 || max_seqlen_q <= 0 || max_seqlen_k <= 0 ||
        max_seqlen_q > (int64_t)INT32_MAX || max_seqlen_k > (int64_t)INT32_MAX)
        return 0;
    rq::PrefillParams p{};
    p.batch = (int)batch;
    p.heads_q = heads_q;
    p.head_dim = head_dim;
    p.max_seqlen_q = (int)max_seqlen_q;
    p.causal = causal != 0;
    (void)same_lengths;
    return rq::prefill_plan(p, max_seqlen_k);
}

void rq_timing_enable(int enabled) {
    std::lock_guard<std::mutex> lock(g_timing.mutex);
    g_timing.enabled = enabled != 0;
}

int rq_timing_read(double* milliseconds, int64_t* launches) {
    std::lock_guard<std::mutex> lock(g_timing.mutex);
    double total = 0.0;
    int64_t count = 0;
    for (auto& pair : g_timing.pending) {
        if (hipEventSynchronize(pair.second) != hipSuccess) return fail(RQ_ELAUNCH, "timing event failed");
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, pair.first, pair.second) != hipSuccess)
            return fail(RQ_ELAUNCH, "timing event failed");
        total += ms;
        ++count;
        g_timing.free_pairs.push_back(pair);
    }
    g_timing.pending.clear();
    if (milliseconds) *milliseconds = total;
    if (launches) *launches = count;
    return ok();
}

void rq_set_split_target(int workgroups) {
    std::lock_guard<std::mutex> lock(g_device_mutex);
    g_split_target = workgroups;
}

}  // extern "C"
