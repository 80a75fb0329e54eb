// Causal varlen prefill attention over raw BF16 Q/K/V for gfx950.
//
// This is the full-prompt branch of the reference backend
// (plugins/residual_quantization/src/residual_quantization/packed_backend.py:63-77),
// which calls vLLM's flash_attn_varlen_func(q, k, v, out, cu_seqlens_q,
// cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal=True):
// out[i] = softmax(scale * q_i . K_j^T over keys j <= i + (len_k - len_q)) V.
//
// Work mapping: one workgroup = 128 queries of one (sequence, head), four
// waves of 32 queries; key tiles of 64 are staged in LDS (K row-major, V
// transposed) and shared by the waves.  Each wave computes S^T = K Q^T with
// v_mfma_f32_32x32x16_bf16, so lane l owns query l % 32: the softmax row max
// and sum are in-lane plus one exchange between the wave's halves, and the
// probabilities P^T stay in the accumulator registers as the B operand of
// O^T += V^T P^T.  The key order inside each P.V step is permuted to match
// the accumulator layout (the A operand reads V^T at the same keys), so P
// never moves between lanes.  Query blocks launch latest-first, since later
// blocks see more keys.
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

constexpr int kPrefillWaves = 4;
constexpr int kPrefillThreads = 64 * kPrefillWaves;
constexpr int kBlockQueries = kPrefillBlockQueries;  // 32 per wave
constexpr int kBlockKeys = kPrefillBlockKeys;
constexpr int kSplitTiles = 16;  // key tiles per work item at most (1024 keys)
static_assert(kBlockQueries == 32 * kPrefillWaves, "one 32-query MFMA column block per wave");

// ---------------------------------------------------------------- plan

// Key tiles query block qb may need: all of them, or 2 (qb + 1) when the
// attention is causal over equal query and key lengths.
__host__ __device__ inline int planned_tiles(const PrefillParams& p, int block) {
    const int need = 2 * (block + 1);
    return (p.causal_same && need < p.max_tiles) ? need : p.max_tiles;
}

__host__ __device__ inline int block_splits(const PrefillParams& p, int block) {
    if (p.split_tiles <= 0) return 1;
    const int n = (planned_tiles(p, block) + p.split_tiles - 1) / p.split_tiles;
    return n < 1 ? 1 : (n > kMaxSplits ? kMaxSplits : n);
}

struct PrefillItem {
    int block, split, splits, slot;  // slot: first partial slot of the block (split blocks only)
};

// Work items run heaviest first: query blocks from the last, their splits in order.
__device__ inline PrefillItem decode_item(const PrefillParams& p, int item) {
    int slot = 0;
    for (int block = p.query_blocks - 1; block >= 0; --block) {
        const int n = block_splits(p, block);
        if (item < n) return {block, item, n, slot};
        item -= n;
        if (n > 1) slot += n;
    }
    return {-1, 0, 1, 0};
}

__device__ __forceinline__ F32x16 mfma(Bf16x8 a, Bf16x8 b, F32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 8 BF16 from a row that is only 8-byte aligned.
__device__ __forceinline__ Bf16x8 load8(const uint16_t* src) {
    const uint2 a = reinterpret_cast<const uint2*>(src)[0];
    const uint2 b = reinterpret_cast<const uint2*>(src)[1];
    const uint4 v = make_uint4(a.x, a.y, b.x, b.y);
    return __builtin_bit_cast(Bf16x8, v);
}

__device__ __forceinline__ uint4 load16(const uint16_t* src) {
    const uint2 a = reinterpret_cast<const uint2*>(src)[0];
    const uint2 b = reinterpret_cast<const uint2*>(src)[1];
    return make_uint4(a.x, a.y, b.x, b.y);
}

template <int D>
__global__ __launch_bounds__(kPrefillThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(PrefillParams p) {
    // Double-buffered K tile [key][KS] and V^T tile [d][VS]; the pads put the
    // 32 rows a wave reads at once on distinct banks.
    constexpr int KS = D + 8;
    constexpr int VS = kBlockKeys + 4;
    __shared__ __attribute__((aligned(16))) uint16_t k_tiles[2][kBlockKeys * KS];
    __shared__ __attribute__((aligned(16))) uint16_t v_tiles[2][D * VS];

    const int sequence = blockIdx.z;
    const int head = blockIdx.y;
    const PrefillItem work = decode_item(p, blockIdx.x);
    if (work.block < 0) return;
    const int q_block = work.block;
    const int q_begin = p.cu_seqlens_q[sequence];
    const int q_len = p.cu_seqlens_q[sequence + 1] - q_begin;
    const int k_begin = p.cu_seqlens_k[sequence];
    const int k_len = p.cu_seqlens_k[sequence + 1] - k_begin;
    const int q0 = q_block * kBlockQueries;
    if (q0 >= q_len) return;  // uniform over the workgroup, before any barrier
    const int shift = k_len - q_len;  // query i sees keys j <= i + shift (causal)
    const int kv_head = head / p.group;

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int column = lane & 31;
    const int half = lane >> 5;
    const int wave_q0 = q0 + 32 * wave;
    const int my_q = wave_q0 + column;

    int block_keys = k_len;
    int wave_keys = k_len;
    if (p.causal) {
        const int block_limit = q0 + kBlockQueries + shift;
        const int wave_limit = wave_q0 + 32 + shift;
        block_keys = block_limit < k_len ? block_limit : k_len;
        wave_keys = wave_limit < k_len ? wave_limit : k_len;
    }
    const int my_limit = p.causal ? my_q + shift : k_len - 1;  // last key this query sees

    // Q^T operand (B of S^T = K Q^T): chunk m holds d = 16m + 8 half + e.
    Bf16x8 q_operand[D / 16];
    {
        const int row = my_q < q_len ? my_q : q_len - 1;
        const uint16_t* src = p.query + (int64_t)(q_begin + row) * p.query_stride + head * D + 8 * half;
#pragma unroll
        for (int m = 0; m < D / 16; ++m) q_operand[m] = load8(src + 16 * m);
    }

    F32x16 out[D / 32];
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) out[t][r] = 0.f;
    float running_max = -__builtin_inff();
    float running_sum = 0.f;
    const float c = p.softmax_scale * 1.4426950408889634f;  // scores in log2 units

    const uint16_t* k_base = p.key + (int64_t)k_begin * p.key_stride + kv_head * D;
    const uint16_t* v_base = p.value + (int64_t)k_begin * p.value_stride + kv_head * D;

    // Tile loads: each thread fetches K chunks (row, 8 channels) and V units
    // (key pair, 8 channels) of the next tile into registers while the current
    // tile computes, then stages them (V transposed) into the other buffer.
    // The loads are raw buffer loads from a wave-uniform resource rebased at
    // each tile, so rows past the sequence read as zero without a branch and
    // every per-thread offset is a loop-invariant 32-bit value.
    constexpr int kKChunks = (kBlockKeys * (D / 8) + kPrefillThreads - 1) / kPrefillThreads;
    constexpr int kVUnits = ((kBlockKeys / 2) * (D / 8) + kPrefillThreads - 1) / kPrefillThreads;
    constexpr uint32_t kOutOfRange = 0x80000000u;  // beyond any tile's record count: loads zero
    const uint32_t key_row_bytes = (uint32_t)p.key_stride * 2, value_row_bytes = (uint32_t)p.value_stride * 2;
    uint32_t k_offset[kKChunks], v_offset[kVUnits];
#pragma unroll
    for (int i = 0; i < kKChunks; ++i) {
        const int chunk = threadIdx.x + i * kPrefillThreads;
        k_offset[i] = chunk < kBlockKeys * (D / 8) ? (uint32_t)(chunk / (D / 8)) * key_row_bytes + 16 * (chunk % (D / 8))
                                                   : kOutOfRange;
    }
#pragma unroll
    for (int i = 0; i < kVUnits; ++i) {
        const int unit = threadIdx.x + i * kPrefillThreads;
        v_offset[i] = unit < (kBlockKeys / 2) * (D / 8)
                          ? (uint32_t)(2 * (unit % (kBlockKeys / 2))) * value_row_bytes + 16 * (unit / (kBlockKeys / 2))
                          : kOutOfRange;
    }
    auto tile_resource = [&](const uint16_t* base, int64_t row_elements, int kt) {
        // Bytes from row kt to the end of the tile's last valid row (its D
        // channels); at most one tile of rows, so the count stays small.
        const int64_t remaining = k_len - kt < kBlockKeys ? k_len - kt : kBlockKeys;
        const uint32_t bytes = remaining > 0 ? (uint32_t)((remaining - 1) * row_elements * 2 + D * 2) : 0u;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + (int64_t)kt * row_elements), (short)0,
                                                 (int)bytes, 0x00020000);
    };
    uint4 k_next[kKChunks], v_next[kVUnits][2];
    auto fetch = [&](int kt) {
        const auto k_rsrc = tile_resource(k_base, p.key_stride, kt);
        const auto v_rsrc = tile_resource(v_base, p.value_stride, kt);
#pragma unroll
        for (int i = 0; i < kKChunks; ++i)
            k_next[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, k_offset[i], 0, 0));
#pragma unroll
        for (int i = 0; i < kVUnits; ++i) {
            v_next[i][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(v_rsrc, v_offset[i], 0, 0));
            v_next[i][1] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(v_rsrc, v_offset[i] + value_row_bytes, 0, 0));
        }
    };
    auto stage = [&](int buffer) {
#pragma unroll
        for (int i = 0; i < kKChunks; ++i) {
            const int chunk = threadIdx.x + i * kPrefillThreads;
            if (chunk < kBlockKeys * (D / 8))
                *reinterpret_cast<uint4*>(&k_tiles[buffer][(chunk / (D / 8)) * KS + 8 * (chunk % (D / 8))]) = k_next[i];
        }
#pragma unroll
        for (int i = 0; i < kVUnits; ++i) {
            const int unit = threadIdx.x + i * kPrefillThreads;
            const int pair = unit % (kBlockKeys / 2), group = unit / (kBlockKeys / 2);
            if (unit < (kBlockKeys / 2) * (D / 8)) {
                const uint4 a = v_next[i][0], b = v_next[i][1];
                const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
                uint16_t* column = &v_tiles[buffer][(8 * group) * VS + 2 * pair];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // (key, key + 1) pairs of channels 2e and 2e + 1.
                    *reinterpret_cast<uint32_t*>(column + (2 * e) * VS) = __builtin_amdgcn_perm(bv[e], av[e], 0x05040100u);
                    *reinterpret_cast<uint32_t*>(column + (2 * e + 1) * VS) =
                        __builtin_amdgcn_perm(bv[e], av[e], 0x07060302u);
                }
            }
        }
    };

    // This item's share of the block's key tiles.
    const int block_tiles = block_keys > 0 ? (block_keys + kBlockKeys - 1) / kBlockKeys : 0;
    const int per_split = (block_tiles + work.splits - 1) / work.splits;
    const int first_tile = work.split * per_split;
    const int end_tile = first_tile + per_split < block_tiles ? first_tile + per_split : block_tiles;
    const int key_end = end_tile * kBlockKeys < block_keys ? end_tile * kBlockKeys : block_keys;

    if (first_tile * kBlockKeys < key_end) {
        fetch(first_tile * kBlockKeys);
        stage(0);
    }
    __syncthreads();
    int buffer = 0;
    for (int kt = first_tile * kBlockKeys; kt < key_end; kt += kBlockKeys, buffer ^= 1) {
        // Buffer `buffer` holds this tile; every wave finished reading the
        // other one before the barrier that ended the previous iteration.
        const bool more = kt + kBlockKeys < key_end;
        if (more) fetch(kt + kBlockKeys);
        const uint16_t* k_tile = k_tiles[buffer];
        const uint16_t* v_tile = v_tiles[buffer];
        if (kt < wave_keys) {  // wave-uniform: this wave's queries see some of these keys

        // S^T for two sub-tiles of 32 keys: register r of lane l holds key
        // kt + 32 sub + 8 (r / 4) + 4 half + r % 4 against query my_q.
        F32x16 s[2];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[sub][r] = 0.f;
            const uint16_t* k_row = &k_tile[(32 * sub + column) * KS + 8 * half];
#pragma unroll
            for (int m = 0; m < D / 16; ++m)
                s[sub] = mfma(*reinterpret_cast<const Bf16x8*>(k_row + 16 * m), q_operand[m], s[sub]);
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
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32)) * c;
        const float new_max = fmaxf(running_max, tile_max);
        // A query with no visible key yet keeps zero weights (no -inf - -inf).
        const float base = new_max == -__builtin_inff() ? 0.f : new_max;
        const float rescale = __builtin_amdgcn_exp2f(running_max - base);
        running_max = new_max;

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
        tile_sum += __shfl_xor(tile_sum, 32);
        running_sum = running_sum * rescale + tile_sum;
        // Once the row maxima settle, most tiles leave every query's max in place.
        if (!__all(rescale == 1.0f)) {
#pragma unroll
            for (int t = 0; t < D / 32; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) out[t][r] *= rescale;
        }

#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int key_offset = 32 * sub + 16 * j + 4 * half;
#pragma unroll
                for (int t = 0; t < D / 32; ++t) {
                    const uint16_t* v_row = &v_tile[(32 * t + column) * VS + key_offset];
                    const uint2 lo = *reinterpret_cast<const uint2*>(v_row);
                    const uint2 hi = *reinterpret_cast<const uint2*>(v_row + 8);
                    const Bf16x8 a = __builtin_bit_cast(Bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    out[t] = mfma(a, p_operand[sub][j], out[t]);
                }
            }
        }
        if (more) stage(buffer ^ 1);
        __syncthreads();
    }

    if (work.splits > 1) {
        // Unnormalised partial [slot][row][query]: rows 0..D-1 the output,
        // D the running max (log2 units), D + 1 the running sum.
        if (my_q < q_len) {
            const int query = 32 * wave + column;
            float* partial = p.partials +
                             ((((int64_t)sequence * p.heads_q + head) * p.partial_slots + work.slot + work.split) *
                              (D + 2)) * kBlockQueries + query;
#pragma unroll
            for (int t = 0; t < D / 32; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    partial[(32 * t + 8 * (r >> 2) + 4 * half + (r & 3)) * kBlockQueries] = out[t][r];
            if (half == 0) {
                partial[D * kBlockQueries] = running_max;
                partial[(D + 1) * kBlockQueries] = running_sum;
            }
        }
        return;
    }
    if (my_q < q_len) {
        const float inverse = running_sum > 0.f ? 1.0f / running_sum : 0.f;
        uint16_t* dst = p.output + (int64_t)(q_begin + my_q) * p.output_stride + head * D + 4 * half;
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t b0 = bf16_rn(out[t][4 * g] * inverse), b1 = bf16_rn(out[t][4 * g + 1] * inverse);
                const uint32_t b2 = bf16_rn(out[t][4 * g + 2] * inverse), b3 = bf16_rn(out[t][4 * g + 3] * inverse);
                *reinterpret_cast<uint2*>(dst + 32 * t + 8 * g) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
            }
    }
}

// Combines the partials of split query blocks: the LSE merge of (max, sum,
// output) triples in log2 units, then the BF16 row.  Thread = (query, 8
// channels): grid.x = query_blocks * D / 8 chunk groups of 128 queries.
template <int D>
__global__ __launch_bounds__(kBlockQueries) void prefill_merge_kernel(PrefillParams p) {
    const int block = blockIdx.x / (D / 8), chunk = blockIdx.x % (D / 8);
    const int head = blockIdx.y, sequence = blockIdx.z;
    const int splits = block_splits(p, block);
    if (splits <= 1) return;
    int slot = 0;
    for (int b = p.query_blocks - 1; b > block; --b) {
        const int n = block_splits(p, b);
        if (n > 1) slot += n;
    }
    const int q_begin = p.cu_seqlens_q[sequence];
    const int q_len = p.cu_seqlens_q[sequence + 1] - q_begin;
    const int query = threadIdx.x;
    const int q = block * kBlockQueries + query;
    if (q >= q_len) return;
    const float* base = p.partials + ((((int64_t)sequence * p.heads_q + head) * p.partial_slots + slot) * (D + 2)) *
                                         kBlockQueries + query;
    const int64_t stride = (int64_t)(D + 2) * kBlockQueries;
    float maximum = -__builtin_inff();
    for (int s = 0; s < splits; ++s) maximum = fmaxf(maximum, base[s * stride + D * kBlockQueries]);
    float total = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < splits; ++s) {
        const float* part = base + s * stride;
        const float m = part[D * kBlockQueries];
        const float w = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - maximum);
        total += w * part[(D + 1) * kBlockQueries];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += w * part[(8 * chunk + e) * kBlockQueries];
    }
    const float inverse = total > 0.f ? 1.0f / total : 0.f;
    uint32_t packed[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) packed[e] = bf16_rn(acc[2 * e] * inverse) | (bf16_rn(acc[2 * e + 1] * inverse) << 16);
    uint16_t* dst = p.output + (int64_t)(q_begin + q) * p.output_stride + head * D + 8 * chunk;
    reinterpret_cast<uint2*>(dst)[0] = make_uint2(packed[0], packed[1]);
    reinterpret_cast<uint2*>(dst)[1] = make_uint2(packed[2], packed[3]);
}

}  // namespace

size_t prefill_plan(PrefillParams& p, int64_t max_seqlen_k) {
    p.query_blocks = (int)((p.max_seqlen_q + kBlockQueries - 1) / kBlockQueries);
    p.max_tiles = (int)((max_seqlen_k + kBlockKeys - 1) / kBlockKeys);
    p.split_tiles = kSplitTiles;
    p.items = 0;
    p.partial_slots = 0;
    for (int block = 0; block < p.query_blocks; ++block) {
        const int n = block_splits(p, block);
        p.items += n;
        if (n > 1) p.partial_slots += n;
    }
    return sizeof(float) * (size_t)p.batch * p.heads_q * p.partial_slots * (p.head_dim + 2) * kBlockQueries;
}

hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream) {
    if (p.batch == 0 || p.max_seqlen_q == 0 || p.items == 0) return hipSuccess;
    const dim3 grid((unsigned)p.items, (unsigned)p.heads_q, (unsigned)p.batch);
    const dim3 merge_grid((unsigned)(p.query_blocks * (p.head_dim / 8)), (unsigned)p.heads_q, (unsigned)p.batch);
    if (p.head_dim == 128) {
        hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kPrefillThreads), 0, stream, p);
        if (p.partial_slots > 0)
            hipLaunchKernelGGL(prefill_merge_kernel<128>, merge_grid, dim3(kBlockQueries), 0, stream, p);
    } else if (p.head_dim == 96) {
        hipLaunchKernelGGL(prefill_kernel<96>, grid, dim3(kPrefillThreads), 0, stream, p);
        if (p.partial_slots > 0)
            hipLaunchKernelGGL(prefill_merge_kernel<96>, merge_grid, dim3(kBlockQueries), 0, stream, p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rq
