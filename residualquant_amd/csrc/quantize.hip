// Fused quantize-on-write for gfx950.
//
// Semantics follow the reference's quantize_kernel
// (plugins/residual_quantization/csrc/quantize/kernel.cuh:14-355): per token,
// head and plane, rotate every record of the loop group by the shared
// rotation, commit the anchor record, then every residual in loop order with
// its LS/Norm/Unit coefficient, FP8 E4M3 group scale/offset and INT2/INT4
// codes, scattered by slot_mapping into the paged cache.
//
// Arithmetic is the canonical order the CPU oracle defines (bit-exact):
// k-ascending FP32 rotation, per-lane fmaf chains over the 4 channels of
// each of 32 "canonical lanes" plus the 16,8,4,2,1 xor butterfly for the LS
// sums, IEEE division/sqrt, RNE satfinite FP8, single rounded BF16 restores.
// Contraction is disabled for this file.
//
// One kernel, quantize_mfma_kernel, does every call: the rotation on the
// matrix cores, then the commit on the VALU.  On gfx950 the FP32 MFMAs and
// the VALU do not execute concurrently (a wave interleaving 8 MFMAs with 64
// independent FMAs takes the sum of the two times, at one and at two waves
// per SIMD), so a call costs its rotation plus its commit.
//
// Commit lanes: a wave commits 4 tokens at a time, 16 lanes per token.  Lane
// j of a token owns canonical lanes j and j + 16, i.e. channels 4j..4j+3 and
// 64+4j..64+4j+3 of every record; the xor-16 level of the butterfly is the
// in-lane sum of the two canonical lanes, the other levels and the group
// min/max run across the 16 lanes of the token with DPP.
#include "rq_device.h"
#include "rq_kernels.h"

#pragma clang fp contract(off)

namespace rq {

namespace {

// ---------------------------------------------------------------- lanes

// Lane exchange within DPP rows.  Every control used here reads a lane of
// the same 16-lane row, so all sources are valid and bound_ctrl never
// applies; with it set the compiler folds the exchange into a consuming VOP2
// add (v_add_f32_dpp) instead of a separate v_mov_b32_dpp.
template <int Control>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Control, 0xf, 0xf, true));
}

constexpr int kXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kRor4 = 0x124;       // row_ror:4 inside 16 lanes
constexpr int kXor8 = 0x128;       // row_ror:8 inside 16 lanes
constexpr int kHalfMirror = 0x141;  // row_half_mirror: lane 7 - i inside each 8 lanes

// The xor butterfly of kernel.cuh:15-20 over the 32 canonical partials, given
// this lane's two (canonical lanes j and j + 16): the distance-16 level is
// their in-lane sum, distances 8, 4, 2, 1 pair lanes j ^ d of the token.
// After the distance-8 level lane j and j ^ 8 hold the same sum (a + b is
// b + a), so the 16 lanes repeat with period 8 and row_ror:4 brings lane
// j ^ 4's value: the same operands in the same order as an xor-4 exchange,
// without an LDS round trip.
__device__ __forceinline__ float butterfly_sum(float low, float high) {
    float v = low + high;
    v += dpp<kXor8>(v);
    v += dpp<kRor4>(v);
    v += dpp<kXor2>(v);
    v += dpp<kXor1>(v);
    return v;
}

// IEEE-754 minimum/maximum: -0 orders below +0 (the min_z/max_z order).
__device__ __forceinline__ float fmin_z(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float fmax_z(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Both E4M3 codes of a group with one v_cvt_pk_fp8_f32 (RNE; the med3 clamp
// to +-448 gives the satfinite behaviour of __nv_fp8_e4m3).
__device__ __forceinline__ uint32_t e4m3_pair(float low_value, float high_value) {
    const float a = __builtin_amdgcn_fmed3f(low_value, -448.0f, 448.0f);
    const float b = __builtin_amdgcn_fmed3f(high_value, -448.0f, 448.0f);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// floor(-q + 0.5) as an integer in one instruction (v_cvt_rpi_i32_f32 with
// a negated source), i.e. -ceil(q - 0.5): checked on gfx950 against the
// clamped ceil(q - 0.5) of every finite FP32 q, for both code widths.
__device__ __forceinline__ int round_half_up_negated(float q) {
    int r;
    asm("v_cvt_rpi_i32_f32_e64 %0, -%1" : "=v"(r) : "v"(q));
    return r;
}

__device__ __forceinline__ float e4m3_value(uint32_t code) {
    return __builtin_amdgcn_cvt_f32_fp8((int)code, 0);
}

// ---------------------------------------------------------------- commit

// Commit one record of one token (kernel.cuh:33-228) for the lane's two
// canonical lanes (h = 0: channels 4j.., h = 1: channels 64+4j..).  All 16
// lanes of the token call this together; `store` masks the global writes.
//
// The division (x - offset) / scale uses the exact reciprocal y = RN(1/scale)
// and one correction step, q = RN(q0 + RN(a - q0 * scale) * y) with
// q0 = RN(a * y): for every E4M3 scale this equals the IEEE quotient (checked
// exhaustively over all FP32 mantissas).  code * scale + offset is exact in
// FP32 (E4M3 operands, 4-bit codes), and a BF16 + BF16 sum rounded once from
// FP32 equals its single-rounded value, so the anchor restore needs no
// TwoSum; the residual chain of adjacent mode keeps it.
__device__ __forceinline__ void commit_record(float (&x)[2][4], const bool (&active)[2], bool is_anchor,
                                              bool restore, int coefficient, const float (&mean)[2][4],
                                              bool has_mean, float (&reference)[2][4],
                                              const RecordRegion& region, uint8_t* page, int token,
                                              int page_tokens, int j, bool store, const float* inverse_scale) {
    float previous[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) previous[h][i] = (!is_anchor && active[h]) ? reference[h][i] : 0.f;

    float alpha = 1.0f;
    if (!is_anchor && coefficient != RQ_COEF_UNIT_) {
        float numerator[2] = {0.f, 0.f}, denominator[2] = {0.f, 0.f};
        // Norm: sum x^2; LS: sum x * previous.  The empty asm keeps this a
        // uniform branch: speculated, both chains would run plus a select.
        if (coefficient == RQ_COEF_NORM_) {
            __asm__ volatile("");
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    numerator[h] = fmaf(x[h][i], x[h][i], numerator[h]);
                    denominator[h] = fmaf(previous[h][i], previous[h][i], denominator[h]);
                }
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    numerator[h] = fmaf(x[h][i], previous[h][i], numerator[h]);
                    denominator[h] = fmaf(previous[h][i], previous[h][i], denominator[h]);
                }
        }
        const float num = butterfly_sum(numerator[0], numerator[1]);
        const float den = butterfly_sum(denominator[0], denominator[1]);
        if (coefficient == RQ_COEF_NORM_)
            alpha = den > 0.f ? sqrtf(num) / fmaxf(sqrtf(den), 1e-6f) : 0.f;
        else
            alpha = num / fmaxf(den, 1e-12f);
    }
    const uint32_t stored_alpha = bf16_rn(alpha);
    alpha = bf16_f32(stored_alpha);

    const int bits = region.bits;
    const float levels = bits == 2 ? 3.0f : 15.0f;
    const float inverse_levels = bits == 2 ? 1.0f / 3.0f : 1.0f / 15.0f;  // RN(1/levels)
    const float clip = bits == 2 ? 0.9f : 1.0f;
    uint32_t packed[2];
    uint32_t parameters[2];
    if (!is_anchor)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[h][i] = fmaf(-previous[h][i], alpha, x[h][i]);
    if (has_mean) {
        __asm__ volatile("");  // a uniform branch, not a speculated select
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[h][i] = x[h][i] - mean[h][i];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float low = fmin_z(fmin_z(x[h][0], x[h][1]), fmin_z(x[h][2], x[h][3]));
        float high = fmax_z(fmax_z(x[h][0], x[h][1]), fmax_z(x[h][2], x[h][3]));
        // A group spans 4 canonical lanes (G16) or 8 (G32), all with the same h;
        // idle canonical lanes (head_dim 96) form groups of their own.
        // min_z/max_z are exact, commutative and associative, so any exchange
        // that covers the group's lanes gives the same result: the mirror
        // pairs lanes i and 7 - i of the 8, the quad levels finish it.
        if (region.group == 32) {
            low = fmin_z(low, dpp<kHalfMirror>(low));
            high = fmax_z(high, dpp<kHalfMirror>(high));
        }
        low = fmin_z(low, dpp<kXor2>(low));
        high = fmax_z(high, dpp<kXor2>(high));
        low = fmin_z(low, dpp<kXor1>(low));
        high = fmax_z(high, dpp<kXor1>(high));

        const float center = (low + high) * 0.5f;
        // (high - low) * 0.9 * 0.5 for INT2, (high - low) * 0.5 for INT4 (x * 1 is exact).
        const float radius = ((high - low) * clip) * 0.5f;
        // (2 radius) / levels through y = RN(1/levels): q = RN(q0 + RN(v - q0 levels) y),
        // q0 = RN(v y), equals the IEEE quotient (checked exhaustively over every
        // binade with subnormal parts, three scale-invariant binades and the top five).
        const float width = 2.0f * radius;
        const float q0 = width * inverse_levels;
        const float step = fmaf(fmaf(-q0, levels, width), inverse_levels, q0);
        parameters[h] = e4m3_pair(center - radius, step);
        const float offset = __builtin_amdgcn_cvt_f32_fp8((int)parameters[h], 0);
        const float scale = __builtin_amdgcn_cvt_f32_fp8((int)parameters[h], 1);
        // RN(1/scale); 0 for a zero (or NaN) scale, which yields code 0.
        const float reciprocal = inverse_scale[(parameters[h] >> 8) & 0x7fu];

        // The codes are packed negated: sum of (-code_i) << (i bits), mod 2^32,
        // then one negation (the fields do not overlap).
        uint32_t negated = 0;
        int neg_code[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // |a| <= 2^100 keeps q0 finite; beyond it the code saturates anyway.
            const float a = __builtin_amdgcn_fmed3f(x[h][i] - offset, -0x1p100f, 0x1p100f);
            const float q0 = a * reciprocal;
            const float r = fmaf(-q0, scale, a);
            const float q = fmaf(r, reciprocal, q0);
            // floor(q) + (frac(q) > 0.5) == ceil(q - 0.5), clamped to [0, levels],
            // which equals ceil(q' - 0.5) for q' = q clamped to [0, levels]; its
            // negation is floor(-q' + 0.5).
            neg_code[i] = round_half_up_negated(__builtin_amdgcn_fmed3f(q, 0.0f, levels));
            negated += (uint32_t)neg_code[i] << (i * bits);
        }
        packed[h] = 0u - negated;
        if (restore) {
            // The restored record, two channels per rounding: bf16(c s + o),
            // then bf16(that + bf16(mu)) on the K plane with key means.
            float value[4];
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const uint32_t pair = bf16x2_rn(fmaf(-(float)neg_code[i], scale, offset),
                                                fmaf(-(float)neg_code[i + 1], scale, offset));
                value[i] = bf16_f32(pair & 0xffffu);
                value[i + 1] = bf16_f32(pair >> 16);
            }
            if (has_mean) {
#pragma unroll
                for (int i = 0; i < 4; i += 2) {
                    const uint32_t mu = bf16x2_rn(mean[h][i], mean[h][i + 1]);
                    const uint32_t pair = bf16x2_rn(value[i] + bf16_f32(mu & 0xffffu),
                                                    value[i + 1] + bf16_f32(mu >> 16));
                    value[i] = bf16_f32(pair & 0xffffu);
                    value[i + 1] = bf16_f32(pair >> 16);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                reference[h][i] = is_anchor ? value[i] : bf16_f32(bf16_fma_rn(reference[h][i], alpha, value[i]));
        }
    }

    if (store) {
        // 32-bit offsets from the page base (a page is far below 4 GiB), so
        // the per-record terms stay single registers.
        const uint32_t codes = (uint32_t)region.offset;
        const uint32_t scales = codes + (uint32_t)(page_tokens * region.code_bytes);
        const uint32_t offsets = scales + (uint32_t)(page_tokens * region.groups);
        const uint32_t alphas = offsets + (uint32_t)(page_tokens * region.groups);
        const int group_shift = region.group == 32 ? 3 : 2;  // log2(canonical lanes per group)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (!active[h]) continue;
            const int lane = j + 16 * h;
            if (bits == 2) {
                page[codes + (uint32_t)(token * region.code_bytes + lane)] = (uint8_t)packed[h];
            } else {
                *reinterpret_cast<uint16_t*>(page + codes + (uint32_t)(token * region.code_bytes + 2 * lane)) =
                    (uint16_t)packed[h];
            }
            if ((lane & ((1 << group_shift) - 1)) == 0) {
                const uint32_t index = (uint32_t)(token * region.groups + (lane >> group_shift));
                page[scales + index] = (uint8_t)(parameters[h] >> 8);
                page[offsets + index] = (uint8_t)(parameters[h] & 0xffu);
            }
        }
        if (j == 0) *reinterpret_cast<uint16_t*>(page + alphas + (uint32_t)(2 * token)) = (uint16_t)stored_alpha;
    }
}

// ---------------------------------------------------------------- kernel
//
// The rotation on the matrix cores: a chain of K = 1
// FP32 MFMAs (v_mfma_f32_16x16x1_4b_f32) accumulates each output with one
// rounding per step in k order, i.e. exactly the k-ascending fmaf chain
// (checked on gfx950 including subnormals, signed zeros and cancellation).
//
// One wave rotates 4 tokens per pass.  The 16 rows of the MFMA are the
// (token, record slot) pairs of those tokens, row 4 token + slot, so a pass
// keeps 32 accumulator registers and 16 waves (4 per SIMD) fit a CU: while
// some waves run their k loop on the matrix core, others commit on the VALU.
// MFMA (half h) takes A = x[row l % 16][k] (the same value in all 4 blocks)
// and B = R[k][64 h + l]; accumulator register i of lane l then holds token
// l / 16, record slot i % 4, channel 64 h + 16 (i / 4) + l % 16.  The commit
// lanes of token l / 16 are the same 16 lanes, so each record passes through
// a 4-token transpose in LDS to the canonical layout right before its commit.
// Slots at or beyond R rotate a copy of record 0 and are never committed.
//
// Inputs are staged per wave through LDS as FP32 in chunks of kInputChunk k,
// double-buffered: each lane converts four BF16 inputs per chunk and the
// MFMAs read their A operands four k at a time (converting in the k loop
// instead cost two VALU per two k steps in every lane, 7% more C1 time).  The
// rotation sits in LDS as FP32
// [k / 2][lane][R[k][l], R[k][64 + l], R[k + 1][l], R[k + 1][64 + l]], one
// 16-byte read per two k steps.
constexpr int kMfmaWaves = 16;
constexpr int kMfmaThreads = 64 * kMfmaWaves;
constexpr int kMfmaTokens = 4;        // tokens per wave per pass
constexpr int kTransposeStride = 144;  // floats per token row of the transpose: 16 q + j spreads the banks

typedef float F32x16 __attribute__((ext_vector_type(16)));

template <int D>
constexpr int kInputChunk = 16;  // an even number of chunks per row at D = 96 and 128
constexpr int kAStride4 = 5;     // float4s per staged A row: 16 k + 4 floats of padding

template <int D, int R, int A, bool Rotated>
__global__ __launch_bounds__(kMfmaThreads) void quantize_mfma_kernel(QuantizeParams p, int block_tokens,
                                                                     int plane_first) {
    static_assert(R <= 4, "four record slots per token");
    constexpr int C = kInputChunk<D>;
    constexpr int kChunks = D / C;
    __shared__ float inverse_scale[128];
    __shared__ __attribute__((aligned(16))) float mean_lds[R * D];
    __shared__ __attribute__((aligned(16))) float transpose_lds[kMfmaWaves][kMfmaTokens * kTransposeStride];
    __shared__ __attribute__((aligned(16))) float rotation_lds[D * 128];
    __shared__ float4 a_lds[Rotated ? kMfmaWaves : 1][2][16][kAStride4];

    const int plane = plane_first + (int)blockIdx.z;
    const int head = blockIdx.y;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane64 = threadIdx.x & 63;
    const int q = lane64 >> 4;  // token of the pass (commit and accumulator role)
    const int j = lane64 & 15;
    const bool active[2] = {4 * j < D, 4 * (j + 16) < D};
    const int column[2] = {4 * j, active[1] ? 64 + 4 * j : 64};

    // Prologue loads all go out before any of them is waited for: the
    // rotation as 16-byte chunks (8 consecutive columns of one row; the
    // addresses are 16-byte aligned, checked on the host) and the key means.
    // Staged one 2-byte load per iteration, each waiting for the last, the
    // rotation took 16 memory round trips per workgroup.
    constexpr int kRowChunks = D / 8;
    constexpr int kRotationChunks = D * kRowChunks;
    constexpr int kChunksPerThread = (kRotationChunks + kMfmaThreads - 1) / kMfmaThreads;
    uint4 chunk_words[kChunksPerThread];
    if constexpr (Rotated) {
        const uint16_t* rotation = plane == 0 ? p.key_rotation : p.value_rotation;
        const uint4* source = reinterpret_cast<const uint4*>(rotation + (int64_t)head * D * D);
#pragma unroll
        for (int u = 0; u < kChunksPerThread; ++u) {
            const int i = (int)threadIdx.x + u * kMfmaThreads;
            chunk_words[u] = i < kRotationChunks ? source[i] : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    const bool has_mean = plane == 0 && p.key_mean != nullptr;
    float mean_value = 0.f;
    static_assert(R * D <= kMfmaThreads, "one key mean per thread");
    if (has_mean && (int)threadIdx.x < R * D)
        mean_value = p.key_mean[((int64_t)(threadIdx.x / D) * p.heads + head) * D + threadIdx.x % D];
    if constexpr (Rotated) {
        // Element (k, c) sits at [k / 2][c % 64][2 (k % 2) + c / 64]; columns
        // from D to 127 (D = 96) are zeros.
#pragma unroll
        for (int u = 0; u < kChunksPerThread; ++u) {
            const int i = (int)threadIdx.x + u * kMfmaThreads;
            if (i < kRotationChunks) {
                const int k = i / kRowChunks, c0 = 8 * (i % kRowChunks);
                const uint32_t w[4] = {chunk_words[u].x, chunk_words[u].y, chunk_words[u].z, chunk_words[u].w};
                float* dst = rotation_lds + ((k >> 1) * 64 + (c0 & 63)) * 4 + 2 * (k & 1) + (c0 >> 6);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    dst[4 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
            }
        }
        if constexpr (D < 128) {
            for (int i = threadIdx.x; i < D * (128 - D); i += kMfmaThreads) {
                const int k = i / (128 - D), c = D + i % (128 - D);
                rotation_lds[((k >> 1) * 64 + (c & 63)) * 4 + 2 * (k & 1) + (c >> 6)] = 0.f;
            }
        }
    }
    if (has_mean && (int)threadIdx.x < R * D) mean_lds[threadIdx.x] = mean_value;
    if (threadIdx.x < 128) {
        const uint32_t code = threadIdx.x;
        inverse_scale[code] = (code == 0 || code == 0x7f) ? 0.0f : 1.0f / e4m3_value(code);
    }
    __syncthreads();

    const int64_t block_first = (int64_t)blockIdx.x * block_tokens;
    const int64_t block_end = block_first + block_tokens < p.tokens ? block_first + block_tokens : p.tokens;
    constexpr int64_t kStride = (int64_t)kMfmaWaves * kMfmaTokens;
    float* transpose = transpose_lds[wave];

    // Loader role: lane l stages row l / 4 = (token, record slot), k quad l % 4
    // of each chunk: one 8-byte load, four exact BF16 -> FP32 conversions and
    // one 16-byte LDS write; the MFMAs then read their FP32 A operands, four
    // k at a time.  Each element is converted once instead of once per k step
    // in every lane (the A operand repeats in all 4 blocks).
    const int ld_row = lane64 >> 2, ld_quad = lane64 & 3;
    const int ld_token = ld_row >> 2, ld_slot = ld_row & 3;
    const int ld_record = ld_slot < R ? ld_slot : 0;
    const uint16_t* ld_base = nullptr;
    int64_t ld_stride = 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (ld_record == r) {
            ld_base = (plane == 0 ? p.key_ptrs[r] : p.value_ptrs[r]) + head * D + 4 * ld_quad;
            ld_stride = plane == 0 ? p.key_strides[r] : p.value_strides[r];
        }
    auto ld_row_of = [&](int64_t f) {
        const int64_t n = f + ld_token < block_end ? f + ld_token : block_end - 1;
        return ld_base + n * ld_stride;
    };
    // Rows are only guaranteed 8-byte aligned: one 8-byte load per chunk.
    auto load_chunk = [&](const uint16_t* row, int chunk) {
        return *reinterpret_cast<const uint2*>(row + chunk * C);
    };
    float4 (*stage)[16][kAStride4] = a_lds[wave];
    auto stage_chunk = [&](uint2 w, int buffer) {
        stage[buffer][ld_row][ld_quad] = make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                                                     __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
    };
    const float4* rotation4 = reinterpret_cast<const float4*>(rotation_lds) + lane64;

    // The slot of this lane's token of the pass starting at `f` (-1 past the block).
    auto load_slot = [&](int64_t f) {
        const bool inside = f + q < block_end;
        const int64_t slot = p.slots[inside ? f + q : block_end - 1];
        return inside ? slot : (int64_t)-1;
    };

    // Pipeline: at the start of chunk c the data of chunk c + 1 (loaded one
    // chunk earlier) goes to LDS and chunk c + 2 is loaded; chunks run on
    // into the next pass's rows (a_row clamps past the block, so the last
    // pass loads too and no branch joins the load counters).
    int64_t first = block_first + wave * kMfmaTokens;
    const uint16_t* row = nullptr;
    uint2 pending = make_uint2(0, 0);
    int64_t next_slot = -1;
    if (Rotated && first < block_end) {
        row = ld_row_of(first);
        stage_chunk(load_chunk(row, 0), 0);
        pending = load_chunk(row, 1);
        next_slot = load_slot(first);
    }
    const int passes = first < block_end ? (int)((block_end - first + kStride - 1) / kStride) : 0;
    // One round of workgroups (launch_quantize_mfma): every one takes it.
    const StreamPriority priority(passes, true);
    int pass = 0;
    for (; first < block_end; first += kStride, ++pass) {
        priority.set(pass);
        const int64_t n = first + q;
        // Rotated passes take the slot prefetched with their first chunk.
        const int64_t slot = Rotated ? next_slot : load_slot(first);
        F32x16 acc[2];
        if constexpr (Rotated) {
            acc[0] = acc[1] = F32x16{};
            float4 a, b0, b1;  // the operands of the next group of k
#pragma unroll
            for (int chunk = 0; chunk < kChunks; ++chunk) {
                // kChunks is even: chunk c of every pass sits in buffer c & 1.
                stage_chunk(pending, (chunk + 1) & 1);
                if (chunk + 2 < kChunks) {
                    pending = load_chunk(row, chunk + 2);
                } else {
                    if (chunk + 2 == kChunks) {
                        row = ld_row_of(first + kStride);
                        next_slot = load_slot(first + kStride);
                    }
                    pending = load_chunk(row, chunk + 2 - kChunks);
                }
                // Keeps the load here: left alone, the compiler sinks it to
                // its first use and every chunk waits a full round trip.
                __asm__ volatile("" ::: "memory");
                const float4* a_read = &stage[chunk & 1][lane64 & 15][0];
                // Operands one group ahead: group g + 1's reads are issued
                // before group g's MFMAs, and the next chunk's first group
                // before this chunk's last (its A was staged at this chunk's
                // start); a pass's first group is read here.
                if (chunk == 0) {
                    a = a_read[0];
                    b0 = rotation4[0];
                    b1 = rotation4[64];
                }
#pragma unroll
                for (int g = 0; g < C / 4; ++g) {
                    const float4 ca = a, cb0 = b0, cb1 = b1;
                    if (g + 1 < C / 4) {
                        a = a_read[g + 1];
                        b0 = rotation4[((chunk * C) / 2 + 2 * g + 2) * 64];
                        b1 = rotation4[((chunk * C) / 2 + 2 * g + 3) * 64];
                    } else if (chunk + 1 < kChunks) {
                        a = stage[(chunk + 1) & 1][lane64 & 15][0];
                        b0 = rotation4[(((chunk + 1) * C) / 2) * 64];
                        b1 = rotation4[(((chunk + 1) * C) / 2 + 1) * 64];
                    }
                    {
                    const float4 a = ca, b0 = cb0, b1 = cb1;
                    acc[0] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.x, b0.x, acc[0], 0, 0, 0);
                    acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.x, b0.y, acc[1], 0, 0, 0);
                    acc[0] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.y, b0.z, acc[0], 0, 0, 0);
                    acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.y, b0.w, acc[1], 0, 0, 0);
                    acc[0] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.z, b1.x, acc[0], 0, 0, 0);
                    acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.z, b1.y, acc[1], 0, 0, 0);
                    acc[0] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.w, b1.z, acc[0], 0, 0, 0);
                    acc[1] = __builtin_amdgcn_mfma_f32_16x16x1f32(a.w, b1.w, acc[1], 0, 0, 0);
                    }
                    // The next group's reads go out ahead of these MFMAs.
                    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
                }
                // Nothing of the next chunk moves above this chunk's MFMAs,
                // so the load issued at its start has the chunk to land.
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        const bool valid = n < block_end && slot >= 0 && (slot >> p.page_shift) < p.num_blocks;
        uint8_t* page = nullptr;
        int token = 0;
        if (valid) {
            const int64_t block = slot >> p.page_shift;
            token = (int)(slot & (p.page_tokens - 1));
            page = p.cache + plane * p.plane_stride + (block * p.heads + head) * (int64_t)p.page_tokens * p.page_width;
        }
        float reference[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // restored BF16 values
        // Anchor first, then every other record ascending (kernel.cuh:321-329).
#pragma unroll
        for (int step = 0; step < R; ++step) {
            const int r = step == 0 ? A : (step - 1 < A ? step - 1 : step);
            const bool is_anchor = r == A;
            float x[2][4];
            if constexpr (Rotated) {
                // The transpose is private to this wave and its LDS operations
                // complete in order; the compiler barriers keep this record's
                // writes after the previous record's reads.
                __asm__ volatile("" ::: "memory");
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        if (64 * h + 16 * b < D) transpose[q * kTransposeStride + 64 * h + 16 * b + j] = acc[h][4 * b + r];
                __asm__ volatile("" ::: "memory");
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (active[h]) v = *reinterpret_cast<const float4*>(transpose + q * kTransposeStride + column[h]);
                    x[h][0] = v.x; x[h][1] = v.y; x[h][2] = v.z; x[h][3] = v.w;
                }
                __asm__ volatile("" ::: "memory");
            } else {
                const int64_t nn = n < block_end ? n : block_end - 1;
                const uint16_t* src = (plane == 0 ? p.key_ptrs[r] + nn * p.key_strides[r]
                                                  : p.value_ptrs[r] + nn * p.value_strides[r]) + head * D;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint2 v = make_uint2(0, 0);
                    if (active[h]) v = *reinterpret_cast<const uint2*>(src + column[h]);
                    x[h][0] = bf16_f32(v.x & 0xffffu);
                    x[h][1] = bf16_f32(v.x >> 16);
                    x[h][2] = bf16_f32(v.y & 0xffffu);
                    x[h][3] = bf16_f32(v.y >> 16);
                }
            }
            float mean[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
                if (has_mean && active[h]) m = *reinterpret_cast<const float4*>(&mean_lds[r * D + column[h]]);
                mean[h][0] = m.x; mean[h][1] = m.y; mean[h][2] = m.z; mean[h][3] = m.w;
            }
            commit_record(x, active, is_anchor, is_anchor || p.adjacent, p.coefficient, mean, has_mean, reference,
                          p.region[r], page, token, p.page_tokens, j, valid, inverse_scale);
        }
    }
}

template <int D, int R, int A>
hipError_t launch_quantize_mfma(const QuantizeParams& p, hipStream_t stream) {
    // One workgroup per CU fits the LDS: split each (head, plane)'s tokens
    // over as many workgroups as make one round on the CUs, in whole passes
    // of kMfmaTokens per wave.  A plane without a rotation takes the
    // unrotated instantiation; planes that differ are two launches.
    const bool key_rotated = p.key_rotation != nullptr, value_rotated = p.value_rotation != nullptr;
    const int planes = key_rotated == value_rotated ? 2 : 1;
    const int64_t pairs = (int64_t)p.heads * planes;
    int64_t per_pair = p.compute_units > 0 ? p.compute_units / pairs : 1;
    per_pair = per_pair < 1 ? 1 : per_pair;
    int64_t block_tokens = (p.tokens + per_pair - 1) / per_pair;
    block_tokens = (block_tokens + kMfmaTokens - 1) / kMfmaTokens * kMfmaTokens;
    block_tokens = block_tokens < (1 << 24) ? block_tokens : (1 << 24);
    const dim3 grid((unsigned)((p.tokens + block_tokens - 1) / block_tokens), (unsigned)p.heads, (unsigned)planes);
    for (int plane = 0; plane < 2; plane += planes) {
        if (plane == 0 ? key_rotated : value_rotated)
            hipLaunchKernelGGL((quantize_mfma_kernel<D, R, A, true>), grid, dim3(kMfmaThreads), 0, stream, p,
                               (int)block_tokens, plane);
        else
            hipLaunchKernelGGL((quantize_mfma_kernel<D, R, A, false>), grid, dim3(kMfmaThreads), 0, stream, p,
                               (int)block_tokens, plane);
        const hipError_t status = hipGetLastError();
        if (status != hipSuccess) return status;
    }
    return hipSuccess;
}

template <int D, int R>
hipError_t dispatch_anchor(const QuantizeParams& p, int anchor, hipStream_t stream) {
    switch (anchor) {
        case 0: return launch_quantize_mfma<D, R, 0>(p, stream);
        case 1: if constexpr (R > 1) return launch_quantize_mfma<D, R, 1>(p, stream); break;
        case 2: if constexpr (R > 2) return launch_quantize_mfma<D, R, 2>(p, stream); break;
        case 3: if constexpr (R > 3) return launch_quantize_mfma<D, R, 3>(p, stream); break;
        default: break;
    }
    return hipErrorInvalidValue;
}

template <int D>
hipError_t dispatch_records(const QuantizeParams& p, hipStream_t stream) {
    switch (p.records) {
        case 1: return dispatch_anchor<D, 1>(p, p.anchor, stream);
        case 2: return dispatch_anchor<D, 2>(p, p.anchor, stream);
        case 3: return dispatch_anchor<D, 3>(p, p.anchor, stream);
        case 4: return dispatch_anchor<D, 4>(p, p.anchor, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_quantize(const QuantizeParams& p, int head_dim, hipStream_t stream) {
    if (p.tokens == 0) return hipSuccess;
    if (head_dim == 128) return dispatch_records<128>(p, stream);
    if (head_dim == 96) return dispatch_records<96>(p, stream);
    return hipErrorInvalidValue;
}

}  // namespace rq
