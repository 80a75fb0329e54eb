// Causal varlen prefill attention over raw BF16 Q/K/V for gfx950.
//
// This is the full-prompt branch of the reference backend
// (plugins/residual_quantization/src/residual_quantization/packed_backend.py:63-77),
// which calls vLLM's flash_attn_varlen_func(q, k, v, out, cu_seqlens_q,
// cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal=True):
// out[i] = softmax(scale * q_i . K_j^T over keys j <= i + (len_k - len_q)) V.
//
// Work mapping: a workgroup is 8 waves in two groups of 4 and takes a pair of
// 128-query blocks of one (sequence, head): the heavy block H = n - 1 - i and
// the light block L = i of the sequence's n blocks (a lone middle block when
// n is odd).  Under causal attention over equal lengths the pair needs
// T(H) + T(L) = n + 1 key tiles of 64 for every i, so every workgroup has the
// same work and no query block is split across workgroups.  Group A takes H's
// first a = ceil((T(H) + T(L)) / 2) tiles; group B takes all of L, then H's
// remaining tiles; at the end B hands its partial (max, sum, output) for H to
// A through LDS and A merges and writes H.  Both groups run the same number
// of tile steps between workgroup barriers; each loads its own K and V tiles
// (row-major, chunk-swizzled) into its own double buffer with DMA loads
// straight into LDS, one tile ahead.
//
// Per wave: 32 queries.  S^T = K Q^T with v_mfma_f32_32x32x16_bf16, so lane l
// owns query l % 32: the row max is in-lane plus one exchange between the
// wave's halves, and the probabilities P^T stay in the accumulator registers
// as the B operand of O^T += V^T P^T, with the key order of each P.V step
// permuted to match the accumulator layout.  The A operand V^T comes from the
// row-major V tile through transposed LDS reads (ds_read_b64_tr_b16) at the
// same keys.  The row max moves lazily: the output is rescaled only when a
// row's max grows by more than 2^8 (P then stays below 256, exact in the
// final normalisation), and each half-wave keeps its own row sum until the
// end.
//
// Lane layouts of v_mfma_f32_32x32x16_bf16 (checked on gfx950): A row l % 32,
// k 8 (l / 32) + e; B column l % 32, k 8 (l / 32) + e; C register r holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.

#include "rq_device.h"
#include "rq_kernels.h"

namespace rq {

namespace {

typedef __bf16 Bf16x8 __attribute__((ext_vector_type(8)));
typedef float F32x16 __attribute__((ext_vector_type(16)));

constexpr int kGroupWaves = 4;
constexpr int kGroupThreads = 64 * kGroupWaves;
constexpr int kPrefillThreads = 2 * kGroupThreads;
constexpr int kBlockQueries = kPrefillBlockQueries;  // 32 per wave
constexpr int kBlockKeys = kPrefillBlockKeys;
constexpr float kLazyRescale = 8.0f;  // log2 units: rescale when a row max grows by more
constexpr int kXcds = 8;              // MI355X accelerator complex dies
static_assert(kBlockQueries == 32 * kGroupWaves, "one 32-query MFMA column block per wave");

__device__ __forceinline__ F32x16 mfma(Bf16x8 a, Bf16x8 b, F32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 8 BF16 from a row that is only 8-byte aligned.
__device__ __forceinline__ Bf16x8 load8(const uint16_t* src) {
    const uint2 a = reinterpret_cast<const uint2*>(src)[0];
    const uint2 b = reinterpret_cast<const uint2*>(src)[1];
    return __builtin_bit_cast(Bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}

// The value of lane l and of lane l ^ 32, low half first in every lane
// (v_permlane32_swap, one VALU op instead of an LDS permute round trip).
__device__ __forceinline__ float2 halves(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_max(float v) {
    const float2 h = halves(v);
    return fmaxf(h.x, h.y);
}
__device__ __forceinline__ float halves_sum(float v) {
    const float2 h = halves(v);
    return h.x + h.y;
}

// LDS of a workgroup: per group, two buffers of [K tile | V tile], each tile
// 64 rows of D BF16 with no padding, filled by DMA loads (buffer_load ... lds:
// lane l of a load writes its 16 bytes at the load's LDS base + 16 l).  The
// 16-byte chunk c of row r sits at position c ^ swizzle(r) of its row, which
// keeps the MFMA operand reads free of bank conflicts:
// - K (ds_read_b128, lane = row, one chunk): 16 consecutive rows at one
//   chunk fall on distinct banks (8 at D = 96, whose 192-byte rows already
//   spread rows 0..3);
// - V^T (ds_read_b64_tr_b16, 16 lanes read 4 consecutive rows x 2 adjacent
//   chunks): the 4 rows fall on distinct banks (by the row length at D = 96).
template <int D>
struct Lds {
    static constexpr int kChunks = D / 8;                  // 16-byte chunks per row
    static constexpr int kRowBytes = 2 * D;
    static constexpr int kTileBytes = kBlockKeys * kRowBytes;
    static constexpr int kBufferBytes = 2 * kTileBytes;    // K tile, then V tile
    static constexpr int kGroupBytes = 2 * kBufferBytes;   // double-buffered
    static constexpr int kBytes = 2 * kGroupBytes;
    static constexpr int kLoadsPerWave = kChunks / kGroupWaves;  // 1 KB DMA loads per wave, tile and plane
    static_assert(kBlockKeys * kChunks == 64 * kGroupWaves * kLoadsPerWave, "a tile is whole 1 KB loads");
    // The merge hand-off reuses the tiles: [wave][D + 2][32] floats.
    static constexpr int kMergeBytes = kGroupWaves * (D + 2) * 32 * 4;
    static_assert(kMergeBytes <= kBytes, "merge buffer fits in the tile buffers");

    __device__ static int k_swizzle(int row) { return D == 128 ? (row & 15) : ((row >> 2) & 1); }
    __device__ static int v_swizzle(int row) { return D == 128 ? 4 * (row & 3) : 0; }
};

typedef short Short4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void LdsVoid;
typedef __attribute__((address_space(3))) Short4 LdsShort4;

// ds_read_b64_tr_b16 (gfx950, checked on the device): within each 16 lanes,
// output lane o gets element o % 4 of the 8 bytes addressed by lanes
// o / 4 + 4 p, p = 0..3.  With lane 4a + b addressing row a, channels
// 4b..4b+3 of a 4-row block, lane o receives channel o of rows 0..3.
__device__ __forceinline__ Short4 read_transposed(const char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsShort4*)p);
}

// One DMA load: lane l's 16 bytes at `offset` of the resource go to
// lds + 16 l (lds wave-uniform).
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t rsrc, char* lds, uint32_t offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LdsVoid*)lds, 16, offset, 0, 0, 0);
}

// One query block's running state for a wave's 32 queries.
template <int D>
struct BlockState {
    F32x16 out[D / 32];
    float running_max, running_sum;  // log2 units; the sum of this half-wave's keys
};

template <int D>
__global__ __launch_bounds__(kPrefillThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(PrefillParams p) {
    using L = Lds<D>;
    __shared__ __attribute__((aligned(1024))) char lds[L::kBytes];

    // XCD-aware order: workgroups are dispatched round-robin over the 8
    // XCDs, so the linear id is remapped to give each XCD a run of
    // consecutive (item, head, sequence) work, i.e. whole heads whose K/V
    // tiles stay in that XCD's L2 (when the grid divides by 8).
    int linear = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int grid_total = gridDim.x * gridDim.y * gridDim.z;
    if (grid_total % kXcds == 0) linear = (linear % kXcds) * (grid_total / kXcds) + linear / kXcds;
    const int item = linear % gridDim.x;
    const int head = (linear / gridDim.x) % gridDim.y;
    const int sequence = linear / (gridDim.x * gridDim.y);
    const int q_begin = p.cu_seqlens_q[sequence];
    const int q_len = p.cu_seqlens_q[sequence + 1] - q_begin;
    const int k_begin = p.cu_seqlens_k[sequence];
    const int k_len = p.cu_seqlens_k[sequence + 1] - k_begin;
    const int n_blocks = (q_len + kBlockQueries - 1) / kBlockQueries;
    if (item >= (n_blocks + 1) / 2) return;  // uniform over the workgroup, before any barrier
    const int shift = k_len - q_len;         // query i sees keys j <= i + shift (causal)
    const int kv_head = head / p.group;

    // Keys a block's queries may see and the key tiles that covers.
    auto block_keys = [&](int block) __attribute__((always_inline)) {
        if (!p.causal) return k_len;
        const int limit = (block + 1) * kBlockQueries + shift;
        return limit < k_len ? (limit > 0 ? limit : 0) : k_len;
    };
    auto block_tiles = [&](int block) __attribute__((always_inline)) { return (block_keys(block) + kBlockKeys - 1) / kBlockKeys; };

    const int heavy = n_blocks - 1 - item;
    const int light = item < heavy ? item : -1;
    const int heavy_tiles = block_tiles(heavy);
    const int light_tiles = light >= 0 ? block_tiles(light) : 0;
    const int total = heavy_tiles + light_tiles;
    const int split = heavy_tiles < (total + 1) / 2 ? heavy_tiles : (total + 1) / 2;  // A: heavy [0, split)
    const int steps = split > total - split ? split : total - split;

    // Wave-uniform by construction; readfirstlane tells the compiler, so the
    // tile resources stay in SGPRs (no waterfall loop around each load).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int group = wave >> 2;  // 0: A, 1: B
    const int group_wave = wave & 3;
    const int lane = threadIdx.x & 63;
    const int column = lane & 31;
    const int half = lane >> 5;

    // (block, tile) of this group at a step, or block -1 when idle.
    auto step_block = [&](int step) __attribute__((always_inline)) {
        if (group == 0) return step < split ? heavy : -1;
        if (step < light_tiles) return light;
        return step - light_tiles < heavy_tiles - split ? heavy : -1;
    };
    auto step_tile = [&](int step) __attribute__((always_inline)) {
        if (group == 0) return step;
        return step < light_tiles ? step : split + step - light_tiles;
    };

    char* group_lds = lds + group * L::kGroupBytes;

    // Tile loads: DMA from a wave-uniform buffer resource rebased at each
    // tile straight into LDS (no registers, no staging pass); rows past the
    // sequence lie outside the resource and arrive as zeros.  Wave w of a
    // group fills the 1 KB slices w * kLoadsPerWave + j of both planes:
    // slice slot s = 64 (w kLoadsPerWave + j) + lane holds chunk
    // (s % kChunks) ^ swizzle(row) of row s / kChunks.
    constexpr int kLoads = L::kLoadsPerWave;
    const uint32_t key_row_bytes = (uint32_t)p.key_stride * 2, value_row_bytes = (uint32_t)p.value_stride * 2;
    uint32_t k_offset[kLoads], v_offset[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int slot = 64 * (group_wave * kLoads + j) + lane;
        const int row = slot / L::kChunks, position = slot % L::kChunks;
        k_offset[j] = (uint32_t)row * key_row_bytes + 16 * (position ^ L::k_swizzle(row));
        v_offset[j] = (uint32_t)row * value_row_bytes + 16 * (position ^ L::v_swizzle(row));
    }
    const uint16_t* k_base = p.key + (int64_t)k_begin * p.key_stride + kv_head * D;
    const uint16_t* v_base = p.value + (int64_t)k_begin * p.value_stride + kv_head * D;
    auto tile_resource = [&](const uint16_t* base, int64_t row_elements, int kt) __attribute__((always_inline)) {
        // Bytes from row kt to the end of the tile's last valid row (its D
        // channels); at most one tile of rows, so the count stays small.
        const int64_t remaining = k_len - kt < kBlockKeys ? k_len - kt : kBlockKeys;
        const uint32_t bytes = remaining > 0 ? (uint32_t)((remaining - 1) * row_elements * 2 + D * 2) : 0u;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + (int64_t)kt * row_elements), (short)0,
                                                 (int)bytes, 0x00020000);
    };
    // Loads of the tile starting at key kt into buffer `buffer` of this
    // group; kt < 0 (no tile of this group's own) issues nothing.
    auto fetch = [&](int kt, int buffer) __attribute__((always_inline)) {
        if (kt < 0) return;
        const auto k_rsrc = tile_resource(k_base, p.key_stride, kt);
        const auto v_rsrc = tile_resource(v_base, p.value_stride, kt);
        char* slices = group_lds + buffer * L::kBufferBytes + group_wave * kLoads * 1024;
#pragma unroll
        for (int j = 0; j < kLoads; ++j)
            load_to_lds(k_rsrc, slices + j * 1024, k_offset[j]);
#pragma unroll
        for (int j = 0; j < kLoads; ++j) load_to_lds(v_rsrc, slices + L::kTileBytes + j * 1024, v_offset[j]);
    };
    // This wave's DMA writes have landed (vmcnt counts them); a barrier
    // after it publishes them to the workgroup.
    auto wait_loads = [&]() __attribute__((always_inline)) { __builtin_amdgcn_s_waitcnt(0x0F70); };

    // Per-lane byte offsets of the operand reads within a tile.
    // K (A of S^T = K Q^T): row 32 sub + column, chunk 2 m + half.
    const int k_lane = L::kRowBytes * column + 16 * (half ^ L::k_swizzle(column));
    auto k_read = [&](int m) __attribute__((always_inline)) { return D == 128 ? (k_lane ^ (32 * m)) : (k_lane + 32 * m); };
    // V^T (A of O^T += V^T P^T) by transposed reads: lane 16 g + 4 a + b
    // (g = 2 h + g') addresses row 4 h + a of an 8-row block, channels
    // 32 t + 16 g' + 4 b..+3, and receives channel 32 t + 16 g' + lane % 16 of
    // rows 4 h..4 h + 3.
    const int tr_a = (lane >> 2) & 3, tr_b = lane & 3, tr_g = (lane >> 4) & 1;
    const int v_lane = L::kRowBytes * (4 * half + tr_a) + 16 * L::v_swizzle(tr_a) + 32 * tr_g + 8 * tr_b;
    auto v_read = [&](int t) __attribute__((always_inline)) { return D == 128 ? (v_lane ^ (64 * t)) : (v_lane + 64 * t); };

    const float c = p.softmax_scale * 1.4426950408889634f;  // scores in log2 units

    // The running block of this wave and its queries.
    BlockState<D> st;
    Bf16x8 q_operand[D / 16];
    int cur_block = -1, wave_q0 = 0, wave_keys = 0, my_q = 0, my_limit = 0;
    auto begin_block = [&](int block) __attribute__((always_inline)) {
        cur_block = block;
        wave_q0 = block * kBlockQueries + 32 * group_wave;
        my_q = wave_q0 + column;
        wave_keys = k_len;
        if (p.causal) {
            const int limit = wave_q0 + 32 + shift;
            wave_keys = limit < k_len ? limit : k_len;
        }
        my_limit = p.causal ? my_q + shift : k_len - 1;  // last key this query sees
        // Q^T operand (B of S^T = K Q^T): chunk m holds d = 16m + 8 half + e.
        const int row = my_q < q_len ? my_q : q_len - 1;
        const uint16_t* src = p.query + (int64_t)(q_begin + row) * p.query_stride + head * D + 8 * half;
#pragma unroll
        for (int m = 0; m < D / 16; ++m) q_operand[m] = load8(src + 16 * m);
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) st.out[t][r] = 0.f;
        st.running_max = -__builtin_inff();
        st.running_sum = 0.f;
    };
    // Normalised BF16 output rows of the running block.
    auto write_block = [&](const BlockState<D>& s, float total_sum) __attribute__((always_inline)) {
        if (my_q >= q_len) return;
        const float inverse = total_sum > 0.f ? 1.0f / total_sum : 0.f;
        uint16_t* dst = p.output + (int64_t)(q_begin + my_q) * p.output_stride + head * D + 4 * half;
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t b0 = bf16_rn(s.out[t][4 * g] * inverse), b1 = bf16_rn(s.out[t][4 * g + 1] * inverse);
                const uint32_t b2 = bf16_rn(s.out[t][4 * g + 2] * inverse), b3 = bf16_rn(s.out[t][4 * g + 3] * inverse);
                *reinterpret_cast<uint2*>(dst + 32 * t + 8 * g) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
            }
    };

    // One key tile of the running block.
    auto compute_tile = [&](int kt, const char* k_tile, const char* v_tile) __attribute__((always_inline)) {
        // S^T for two sub-tiles of 32 keys: register r of lane l holds key
        // kt + 32 sub + 8 (r / 4) + 4 half + r % 4 against query my_q.
        F32x16 s[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[sub][r] = 0.f;
            const char* k_rows = k_tile + 32 * sub * L::kRowBytes;
#pragma unroll
            for (int m = 0; m < D / 16; ++m)
                s[sub] = mfma(*reinterpret_cast<const Bf16x8*>(k_rows + k_read(m)), q_operand[m], s[sub]);
        }
        // Raw scores: the scale is positive, so the row max of the scaled
        // scores is the scaled row max and is folded into the exp2 argument.
        float tile_max = -__builtin_inff();
        // Only tiles that cross the sequence end or this wave's causal
        // diagonal need the per-key mask (wave-uniform branch).
        const bool masked = kt + kBlockKeys > k_len || (p.causal && kt + kBlockKeys - 1 > wave_q0 + shift);
        if (masked) {
#pragma unroll
            for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt + 32 * sub + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (!(key < k_len && key <= my_limit)) s[sub][r] = -__builtin_inff();
                    tile_max = fmaxf(tile_max, s[sub][r]);
                }
        } else {
#pragma unroll
            for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s[sub][r]);
        }
        tile_max = halves_max(tile_max) * c;
        // Lazy max: keep the running max unless the tile exceeds it by more
        // than 2^8; the weights then stay below 256 and cancel in the final
        // normalisation.
        const bool grow = tile_max > st.running_max + kLazyRescale;
        const float new_max = grow ? tile_max : st.running_max;
        // A query with no visible key yet keeps zero weights (no -inf - -inf).
        const float base = new_max == -__builtin_inff() ? 0.f : new_max;
        const float rescale = grow ? __builtin_amdgcn_exp2f(st.running_max - base) : 1.0f;
        st.running_max = new_max;
        if (!__all(!grow)) {
#pragma unroll
            for (int t = 0; t < D / 32; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) st.out[t][r] *= rescale;
        }

        // P^T in BF16 as the B operand of O^T += V^T P^T: step j of sub-tile
        // `sub` takes registers 8j..8j+7, i.e. k-slot (half, e) is key
        // 32 sub + 16 j + 4 half + e + (e >= 4 ? 4 : 0).
        float tile_sum = 0.f;
        Bf16x8 p_operand[2][2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float w = __builtin_amdgcn_exp2f(fmaf(s[sub][8 * j + e], c, -base));
                    p_operand[sub][j][e] = (__bf16)w;
                    tile_sum += w;
                }
        st.running_sum = st.running_sum * rescale + tile_sum;

#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const char* v_rows = v_tile + (32 * sub + 16 * j) * L::kRowBytes;
#pragma unroll
                for (int t = 0; t < D / 32; ++t) {
                    // Keys 4 half + 0..3 and 4 half + 8..11 of the 16, as P^T's k-slots.
                    const Short4 lo = read_transposed(v_rows + v_read(t));
                    const Short4 hi = read_transposed(v_rows + 8 * L::kRowBytes + v_read(t));
                    const Bf16x8 a = __builtin_bit_cast(
                        Bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    st.out[t] = mfma(a, p_operand[sub][j], st.out[t]);
                }
            }
    };

    // A owns H from the start, B owns L (when the pair has one): a block with
    // no visible key still writes its (zero) rows.
    if (group == 0)
        begin_block(heavy);
    else if (light >= 0)
        begin_block(light);
    // While group B works on L its tile at each step is A's (both start at
    // key tile 0): A loads that tile once and both groups read A's buffer.
    // Under full (non-causal) attention every step is shared this way.
    const int shared_steps = light >= 0 ? (light_tiles < split ? light_tiles : split) : 0;
    auto own_tile = [&](int step) __attribute__((always_inline)) { return group == 0 || step >= shared_steps; };
    // The key of a group's own tile at a step, or -1 (idle, or a shared step of B).
    auto tile_key = [&](int step) __attribute__((always_inline)) {
        return step < steps && step_block(step) >= 0 && own_tile(step) ? step_tile(step) * kBlockKeys : -1;
    };
    // Step s computes tile s from buffer s & 1 while the DMA loads of tile
    // s + 1 fill buffer (s + 1) & 1, which every wave finished reading
    // before the barrier that ended step s - 1.
    fetch(tile_key(0), 0);
    wait_loads();
    __syncthreads();
    for (int step = 0; step < steps; ++step) {
        const int block = step_block(step);
        if (block >= 0 && block != cur_block) {
            // Group B moves to H's tail: its L (if any) is complete.
            if (cur_block >= 0) write_block(st, halves_sum(st.running_sum));
            begin_block(block);
        }
        fetch(tile_key(step + 1), (step + 1) & 1);
        if (block >= 0) {
            const int kt = step_tile(step) * kBlockKeys;
            const char* buffer = (own_tile(step) ? group_lds : lds) + (step & 1) * L::kBufferBytes;
            if (kt < wave_keys) compute_tile(kt, buffer, buffer + L::kTileBytes);
        }
        wait_loads();
        __syncthreads();
    }

    const bool handoff = split < heavy_tiles;  // group B holds part of H
    if (!handoff) {
        // A's H and B's L (if any) are complete.
        if (cur_block >= 0) write_block(st, halves_sum(st.running_sum));
        return;
    }
    // B's partial for H to LDS as [wave][row][query]: rows 0..D-1 the output,
    // D the running max (log2 units), D + 1 the running sum (both halves).
    float* merge = reinterpret_cast<float*>(lds) + group_wave * (D + 2) * 32;
    const float sum_both = halves_sum(st.running_sum);
    if (group == 1) {
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) merge[(32 * t + 8 * (r >> 2) + 4 * half + (r & 3)) * 32 + column] = st.out[t][r];
        if (half == 0) {
            merge[D * 32 + column] = st.running_max;
            merge[(D + 1) * 32 + column] = sum_both;
        }
    }
    __syncthreads();
    if (group == 0) {
        const float other_max = merge[D * 32 + column];
        const float other_sum = merge[(D + 1) * 32 + column];
        const float m = fmaxf(st.running_max, other_max);
        const float base = m == -__builtin_inff() ? 0.f : m;
        const float mine = st.running_max == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(st.running_max - base);
        const float theirs = other_max == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(other_max - base);
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st.out[t][r] = st.out[t][r] * mine +
                               merge[(32 * t + 8 * (r >> 2) + 4 * half + (r & 3)) * 32 + column] * theirs;
        write_block(st, sum_both * mine + other_sum * theirs);
    }
}

}  // namespace

size_t prefill_plan(PrefillParams& p, int64_t max_seqlen_k) {
    (void)max_seqlen_k;
    p.query_blocks = (int)((p.max_seqlen_q + kBlockQueries - 1) / kBlockQueries);
    p.items = (p.query_blocks + 1) / 2;  // block pairs per (sequence, head)
    return 0;                            // no workspace: blocks merge within their workgroup
}

hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream) {
    if (p.batch == 0 || p.max_seqlen_q == 0 || p.items == 0) return hipSuccess;
    const dim3 grid((unsigned)p.items, (unsigned)p.heads_q, (unsigned)p.batch);
    if (p.head_dim == 128)
        hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kPrefillThreads), 0, stream, p);
    else if (p.head_dim == 96)
        hipLaunchKernelGGL(prefill_kernel<96>, grid, dim3(kPrefillThreads), 0, stream, p);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace rq
