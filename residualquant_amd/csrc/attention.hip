// Split-K paged decode attention over packed INT2/INT4 pages (gfx950).
//
// Semantics: the reference's attention() path
// (plugins/residual_quantization/csrc/attention/prepare.cuh:13-430,
// compute.cuh:226-727, merge.cuh:8-84, output.cuh:9-31).  Anchor mode, loop L:
// the history key of token t is K_L = alpha_L * K_A + deq_L (+ means), scored
// against q' = (q . R_k) / sqrt(D); the live token is folded in at the merge;
// the history value sum is inverse-rotated by R_v when given.
//
// Three launches per call, all with grids fixed by host shapes:
//   prepare  (rows x heads)          q' in log2 units, live score, group sums
//                                    of q', q' as 16-bit integers split into
//                                    four nibble planes for v_dot8_u32_u4;
//   decode   (rows x heads x splits) one workgroup = 4 waves streaming the
//                                    pages of one split; each wave owns one
//                                    16-token unit at a time, lane = token x
//                                    32-channel quarter; QK on integer dot8
//                                    units, PV in FP32 registers, online
//                                    softmax per wave, LDS merge of the waves;
//   merge    (rows x heads)          log-sum-exp merge of the splits and the
//                                    live token, V inverse rotation, BF16 out.
#include "rq_device.h"
#include "rq_kernels.h"

namespace rq {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDecodeThreads = 256;
constexpr int kWaves = kDecodeThreads / 64;
constexpr int kUnitTokens = 16;

__device__ __forceinline__ float quad_xor1(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_xor2(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_sum(float x) {
    x += quad_xor1(x);
    return x + quad_xor2(x);
}

// Max / sum over the 16 tokens of a unit (lane bits 2..5).
__device__ __forceinline__ float token_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 4));
    x = fmaxf(x, __shfl_xor(x, 8));
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float token_sum(float x) {
    x += __shfl_xor(x, 4);
    x += __shfl_xor(x, 8);
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

__device__ __forceinline__ float f16_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// FP8 E4M3 byte `sel` of v to FP32.  gfx950 converts OCP E4M3 in hardware.
template <int Sel>
__device__ __forceinline__ float fp8_f32(uint32_t v) {
    return __builtin_amdgcn_cvt_f32_fp8((int)v, Sel);
}

__device__ __forceinline__ int find_request(const int32_t* qsl, int64_t requests, int64_t row) {
    if (requests <= 0 || row < qsl[0] || row >= qsl[requests]) return -1;
    int64_t lo = 0, hi = requests;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (qsl[mid] <= row) lo = mid; else hi = mid;
    }
    return (int)lo;
}

// ------------------------------------------------------------------ prepare

template <int D>
__global__ __launch_bounds__(128) void prepare_kernel(AttentionParams p) {
    const int64_t row = blockIdx.x;
    const int head = blockIdx.y;
    const int c = threadIdx.x;
    const int lane = c & 63;
    const int wave = c >> 6;
    __shared__ float q_lds[128];
    __shared__ float totals[4][2];

    const int request = find_request(p.query_start_loc, p.requests, row);
    if (head == 0 && c == 0) p.row_request[row] = request;
    if (request < 0) return;

    const bool active = c < D;
    const float q = active ? bf16_f32(p.query[row * p.query_stride + head * D + c]) : 0.f;
    q_lds[c] = q;
    __syncthreads();

    float qr = q;
    if (p.key_rotation != nullptr) {
        float acc = 0.f;
        if (active) {
            const uint16_t* m = p.key_rotation + (int64_t)head * D * D + c;
            for (int k = 0; k < D; ++k) acc = fmaf(q_lds[k], f16_f32(m[(int64_t)k * D]), acc);
        }
        qr = acc;
    }
    const float scale = kLog2e / sqrtf((float)D);
    qr *= scale;

    const float k_live = active ? bf16_f32(p.key[row * p.key_stride + head * D + c]) : 0.f;
    float parts[4];
    parts[0] = q * k_live;
    parts[1] = (active && p.key_mean_loop) ? qr * p.key_mean_loop[head * D + c] : 0.f;
    parts[2] = (active && p.key_mean_anchor) ? qr * p.key_mean_anchor[head * D + c] : 0.f;
    parts[3] = fabsf(qr);
#pragma unroll
    for (int d = 32; d; d >>= 1) {
        parts[0] += __shfl_xor(parts[0], d);
        parts[1] += __shfl_xor(parts[1], d);
        parts[2] += __shfl_xor(parts[2], d);
        parts[3] = fmaxf(parts[3], __shfl_xor(parts[3], d));
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) totals[i][wave] = parts[i];
    }

    // Group sums of q' over 16 and 32 channels.
    float q16 = qr;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) q16 += __shfl_xor(q16, d);
    const float q32 = q16 + __shfl_xor(q16, 16);
    __syncthreads();

    const float amax = fmaxf(totals[3][0], totals[3][1]);
    const float delta = amax > 0.f ? amax / 32767.0f : 1.0f;
    float* prep = p.prep + (row * p.heads + head) * (int64_t)kPrepFloats;
    if (c == 0) {
        prep[0] = delta;
        prep[1] = scale * (totals[0][0] + totals[0][1]) - (totals[1][0] + totals[1][1]);
        prep[2] = totals[2][0] + totals[2][1];
    }
    if (active && (c & 15) == 0) prep[3 + c / 16] = q16;
    if (active && (c & 31) == 0) prep[11 + c / 32] = q32;
    prep[kPrepScalars + c] = active ? qr : 0.f;

    // 16-bit offset-binary integer of q', four nibble planes.
    const float scaled = fminf(fmaxf(rintf(qr / delta), -32767.f), 32767.f);
    const uint32_t qu = active ? (uint32_t)((int)scaled + 32768) : 32768u;
    uint32_t* planes4 = reinterpret_cast<uint32_t*>(prep + kPrepScalars + kPrepQuery);
    uint32_t* planes2 = planes4 + kPrepPlanes;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t nibble = (qu >> (4 * j)) & 15u;
        // INT4 order: word c/8, nibble c%8.
        uint32_t w4 = nibble << (4 * (c & 7));
        w4 |= __shfl_xor(w4, 1);
        w4 |= __shfl_xor(w4, 2);
        w4 |= __shfl_xor(w4, 4);
        // INT2 order: 16-channel word c/16 split into even/odd channels,
        // nibble (c%16)/2 of nibble-word 2*(c/16) + c%2.
        uint32_t w2 = nibble << (4 * ((c & 15) >> 1));
        w2 |= __shfl_xor(w2, 2);
        w2 |= __shfl_xor(w2, 4);
        w2 |= __shfl_xor(w2, 8);
        if (active && (c & 7) == 0) planes4[j * 16 + c / 8] = w4;
        if (active && (c & 14) == 0) planes2[j * 16 + 2 * (c / 16) + (c & 1)] = w2;
    }
}

// ------------------------------------------------------------------ packed decode

template <int Bits>
struct Codes;
template <>
struct Codes<4> {
    uint32_t w[4];
    __device__ __forceinline__ void load(const uint8_t* p) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
};
template <>
struct Codes<2> {
    uint32_t w[2];
    __device__ __forceinline__ void load(const uint8_t* p) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        w[0] = v.x; w[1] = v.y;
    }
};

// Scale/offset of the lane's group(s): one byte each for G32, two for G16.
template <int G>
struct GroupParams {
    float scale[2], offset[2];
    __device__ __forceinline__ void load(const uint8_t* scales, const uint8_t* offsets) {
        if constexpr (G == 32) {
            const uint32_t s = *scales, o = *offsets;
            scale[0] = scale[1] = fp8_f32<0>(s);
            offset[0] = offset[1] = fp8_f32<0>(o);
        } else {
            const uint32_t s = *reinterpret_cast<const uint16_t*>(scales);
            const uint32_t o = *reinterpret_cast<const uint16_t*>(offsets);
            scale[0] = fp8_f32<0>(s);
            scale[1] = fp8_f32<1>(s);
            offset[0] = fp8_f32<0>(o);
            offset[1] = fp8_f32<1>(o);
        }
    }
};

// Integer q'.codes over the lane's 32 channels, per 16-channel half.
// planes[j][i]: nibble plane j of the lane's i-th code word (4 words).
template <int Bits>
__device__ __forceinline__ void code_dots(const Codes<Bits>& codes, const uint32_t (&planes)[4][4],
                                          int (&dot)[2]) {
    uint32_t d[2][4] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    uint32_t count[2] = {0u, 0u};
    constexpr uint32_t kOnes = 0x11111111u;
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = i >> 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) d[h][j] = __builtin_amdgcn_udot8(planes[j][i], codes.w[i], d[h][j], false);
            count[h] = __builtin_amdgcn_udot8(kOnes, codes.w[i], count[h], false);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t even = codes.w[i] & 0x33333333u;
            const uint32_t odd = (codes.w[i] >> 2) & 0x33333333u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                d[i][j] = __builtin_amdgcn_udot8(planes[j][2 * i], even, d[i][j], false);
                d[i][j] = __builtin_amdgcn_udot8(planes[j][2 * i + 1], odd, d[i][j], false);
            }
            count[i] = __builtin_amdgcn_udot8(kOnes, even, count[i], false);
            count[i] = __builtin_amdgcn_udot8(kOnes, odd, count[i], false);
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
        dot[h] = (int)(d[h][0] + 16u * d[h][1] + 256u * d[h][2] + 4096u * d[h][3]) -
                 32768 * (int)count[h];
}

// acc[c] += weight[half(c)] * code[c] over the lane's 32 channels.
template <int Bits>
__device__ __forceinline__ void accumulate_codes(const Codes<Bits>& codes, const float (&weight)[2],
                                                 float (&acc)[32]) {
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float w = weight[i >> 1];
            const uint32_t lo = codes.w[i] & 0x0f0f0f0fu;
            const uint32_t hi = (codes.w[i] >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc[8 * i + 2 * b] = fmaf(w, (float)((lo >> (8 * b)) & 0xffu), acc[8 * i + 2 * b]);
                acc[8 * i + 2 * b + 1] = fmaf(w, (float)((hi >> (8 * b)) & 0xffu), acc[8 * i + 2 * b + 1]);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float w = weight[i];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t part = (codes.w[i] >> (2 * k)) & 0x03030303u;
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[16 * i + 4 * b + k] = fmaf(w, (float)((part >> (8 * b)) & 0xffu), acc[16 * i + 4 * b + k]);
            }
        }
    }
}

template <int Bits>
__device__ __forceinline__ void load_planes(const float* prep, int qd, uint32_t (&planes)[4][4]) {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(prep + kPrepScalars + kPrepQuery) +
                           (Bits == 2 ? kPrepPlanes : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 v = *reinterpret_cast<const uint4*>(base + j * 16 + 4 * qd);
        planes[j][0] = v.x; planes[j][1] = v.y; planes[j][2] = v.z; planes[j][3] = v.w;
    }
}

// Record region addresses for one (page, token, quarter).
template <int Bits, int G>
struct RecordView {
    const uint8_t* codes;
    const uint8_t* scales;
    const uint8_t* offsets;
    const uint8_t* alpha;
    __device__ __forceinline__ RecordView(const uint8_t* page, const RecordRegion& r, int page_tokens,
                                          int token, int qd) {
        const uint8_t* base = page + r.offset;
        codes = base + token * r.code_bytes + qd * (32 * Bits / 8);
        scales = base + page_tokens * r.code_bytes + token * r.groups + qd * (32 / G);
        offsets = scales + page_tokens * r.groups;
        alpha = base + page_tokens * (r.code_bytes + 2 * r.groups) + 2 * token;
    }
};

// Lane part of one record's score: sum over the lane's group(s) of
// scale * delta * (q_int . codes) + offset * sum(q').
template <int G>
__device__ __forceinline__ float record_score(const GroupParams<G>& gp, const int (&dot)[2],
                                              float delta, const float (&q_sum)[2]) {
    if constexpr (G == 32)
        return gp.scale[0] * (delta * (float)(dot[0] + dot[1])) + gp.offset[0] * q_sum[0];
    else
        return gp.scale[0] * (delta * (float)dot[0]) + gp.offset[0] * q_sum[0] +
               gp.scale[1] * (delta * (float)dot[1]) + gp.offset[1] * q_sum[1];
}

template <int G>
__device__ __forceinline__ void group_sums(const float* prep, int qd, float (&q_sum)[2]) {
    if constexpr (G == 32) {
        q_sum[0] = q_sum[1] = prep[11 + qd];
    } else {
        q_sum[0] = prep[3 + 2 * qd];
        q_sum[1] = prep[3 + 2 * qd + 1];
    }
}

// Writes (m, l, acc[D]) of this split after merging the four waves in LDS.
template <int D>
__device__ __forceinline__ void write_partial(float (&acc)[32], float m, float l_lane, int lane,
                                              int wave, bool lane_active, float* partial) {
    __shared__ float red_acc[kWaves][16][128];
    __shared__ float red_m[kWaves], red_l[kWaves];
    const int t = lane >> 2, qd = lane & 3;
    const float l_wave = token_sum((lane_active && qd == 0) ? l_lane : 0.f);
    if (lane == 0) {
        red_m[wave] = m;
        red_l[wave] = l_wave;
    }
    __syncthreads();
    float m_all = red_m[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m_all = fmaxf(m_all, red_m[w]);
    const float wave_scale = m == -INFINITY ? 0.f : exp2f(m - m_all);
    float* dst = &red_acc[wave][t][qd * 32];
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        float4 v;
        v.x = acc[i] * wave_scale;
        v.y = acc[i + 1] * wave_scale;
        v.z = acc[i + 2] * wave_scale;
        v.w = acc[i + 3] * wave_scale;
        *reinterpret_cast<float4*>(dst + i) = v;
    }
    __syncthreads();
    const int c = threadIdx.x;
    if (c < D) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int tt = 0; tt < 16; ++tt) sum += red_acc[w][tt][c];
        partial[2 + c] = sum;
    }
    if (c == 0) {
        float l_all = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            l_all += red_m[w] == -INFINITY ? 0.f : red_l[w] * exp2f(red_m[w] - m_all);
        partial[0] = m_all;
        partial[1] = l_all;
    }
}

// Page range of one split (in 16-token units) for the request of `row`.
struct SplitRange {
    int request;
    int64_t history, unit_begin, unit_end;
};

__device__ __forceinline__ SplitRange split_range(const AttentionParams& p, int64_t row, int split) {
    SplitRange r;
    r.request = p.row_request[row];
    r.history = 0;
    r.unit_begin = r.unit_end = 0;
    if (r.request < 0) return r;
    int64_t history = p.seq_lens[r.request] - 1;
    if (history < 0) history = 0;
    int64_t pages = (history + p.page_tokens - 1) / p.page_tokens;
    if (pages > p.max_pages) pages = p.max_pages;
    if (history > pages * p.page_tokens) history = pages * p.page_tokens;
    const int units_per_page = p.page_tokens / kUnitTokens;
    r.history = history;
    r.unit_begin = (split * pages / p.splits) * units_per_page;
    r.unit_end = ((split + 1) * pages / p.splits) * units_per_page;
    return r;
}

template <int D, int BA, int GA, int BL, int GL, bool HasL>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(AttentionParams p) {
    constexpr int Quarters = D / 32;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = lane >> 2;
    const int qd = lane & 3;
    const bool lane_active = qd < Quarters;
    const int lq = lane_active ? qd : 0;
    const int split = blockIdx.x % p.splits;
    const int64_t rh = blockIdx.x / p.splits;
    const int head = (int)(rh % p.heads);
    const int64_t row = rh / p.heads;

    const SplitRange range = split_range(p, row, split);
    if (range.request < 0) return;
    float* partial = p.partials + (rh * p.splits + split) * (int64_t)(D + 2);

    const float* prep = p.prep + rh * (int64_t)kPrepFloats;
    const float delta = prep[0];
    const float q_mean_anchor = prep[2];
    float q_sum_a[2], q_sum_l[2];
    group_sums<GA>(prep, lq, q_sum_a);
    group_sums<GL>(prep, lq, q_sum_l);
    uint32_t planes_a[4][4], planes_l[4][4];
    load_planes<BA>(prep, lq, planes_a);
    if constexpr (HasL) load_planes<BL>(prep, lq, planes_l);

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
    float cst[2] = {0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    const int32_t* table = p.block_table + (int64_t)range.request * p.block_table_stride;
    const int64_t page_bytes = (int64_t)p.page_tokens * p.page_width;
    const int units_per_page = p.page_tokens / kUnitTokens;

    for (int64_t u = range.unit_begin + wave; u < range.unit_end; u += kWaves) {
        const int64_t page_index = u / units_per_page;
        const int token = (int)(u % units_per_page) * kUnitTokens + t;
        const int64_t block = table[page_index];
        if (block < 0 || block >= p.num_blocks) continue;
        const bool valid = lane_active && page_index * p.page_tokens + token < range.history;
        const uint8_t* kpage = p.cache + (block * p.heads + head) * page_bytes;
        const uint8_t* vpage = kpage + p.plane_stride;

        const RecordView<BA, GA> ka(kpage, p.anchor, p.page_tokens, token, lq);
        const RecordView<BA, GA> va(vpage, p.anchor, p.page_tokens, token, lq);
        Codes<BA> kcodes_a, vcodes_a;
        GroupParams<GA> kpar_a, vpar_a;
        kcodes_a.load(ka.codes);
        kpar_a.load(ka.scales, ka.offsets);
        vcodes_a.load(va.codes);
        vpar_a.load(va.scales, va.offsets);

        Codes<BL> kcodes_l, vcodes_l;
        GroupParams<GL> kpar_l, vpar_l;
        float alpha_k = 1.f, alpha_v = 1.f;
        if constexpr (HasL) {
            const RecordView<BL, GL> kl(kpage, p.residual, p.page_tokens, token, lq);
            const RecordView<BL, GL> vl(vpage, p.residual, p.page_tokens, token, lq);
            kcodes_l.load(kl.codes);
            kpar_l.load(kl.scales, kl.offsets);
            vcodes_l.load(vl.codes);
            vpar_l.load(vl.scales, vl.offsets);
            alpha_k = bf16_f32(*reinterpret_cast<const uint16_t*>(kl.alpha));
            alpha_v = bf16_f32(*reinterpret_cast<const uint16_t*>(vl.alpha));
        }

        // ---- scores
        int dots_a[2];
        code_dots<BA>(kcodes_a, planes_a, dots_a);
        float lane_score = record_score<GA>(kpar_a, dots_a, delta, q_sum_a);
        if constexpr (HasL) {
            int dots_l[2];
            code_dots<BL>(kcodes_l, planes_l, dots_l);
            lane_score = alpha_k * lane_score + record_score<GL>(kpar_l, dots_l, delta, q_sum_l);
        }
        float score = quad_sum(lane_active ? lane_score : 0.f);
        if constexpr (HasL) score += alpha_k * q_mean_anchor;
        score = valid ? score : -INFINITY;

        // ---- online softmax (wave-uniform running maximum)
        const float unit_max = token_max(score);
        if (unit_max > m) {
            const float factor = m == -INFINITY ? 0.f : exp2f(m - unit_max);
#pragma unroll
            for (int i = 0; i < 32; ++i) acc[i] *= factor;
            cst[0] *= factor;
            cst[1] *= factor;
            l *= factor;
            m = unit_max;
        }
        const float prob = valid ? exp2f(score - m) : 0.f;
        l += prob;

        // ---- values: acc += p * (alpha_v * deq_A + deq_L), offsets folded into cst
        float w_a[2], w_l[2];
        if constexpr (HasL) {
            const float pa = prob * alpha_v;
            w_a[0] = pa * vpar_a.scale[0];
            w_a[1] = pa * vpar_a.scale[1];
            w_l[0] = prob * vpar_l.scale[0];
            w_l[1] = prob * vpar_l.scale[1];
            if (valid) {
                cst[0] = fmaf(pa, vpar_a.offset[0], fmaf(prob, vpar_l.offset[0], cst[0]));
                cst[1] = fmaf(pa, vpar_a.offset[1], fmaf(prob, vpar_l.offset[1], cst[1]));
            }
        } else {
            w_a[0] = prob * vpar_a.scale[0];
            w_a[1] = prob * vpar_a.scale[1];
            if (valid) {
                cst[0] = fmaf(prob, vpar_a.offset[0], cst[0]);
                cst[1] = fmaf(prob, vpar_a.offset[1], cst[1]);
            }
        }
        if (!valid) {
            w_a[0] = w_a[1] = 0.f;
            w_l[0] = w_l[1] = 0.f;
        }
        accumulate_codes<BA>(vcodes_a, w_a, acc);
        if constexpr (HasL) accumulate_codes<BL>(vcodes_l, w_l, acc);
    }

#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] += cst[i >> 4];
    write_partial<D>(acc, m, l, lane, wave, lane_active, partial);
}

// ------------------------------------------------------------------ BF16 baseline decode

template <int D>
__global__ __launch_bounds__(kDecodeThreads) void decode_bf16_kernel(AttentionParams p) {
    constexpr int Quarters = D / 32;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = lane >> 2;
    const int qd = lane & 3;
    const bool lane_active = qd < Quarters;
    const int lq = lane_active ? qd : 0;
    const int split = blockIdx.x % p.splits;
    const int64_t rh = blockIdx.x / p.splits;
    const int head = (int)(rh % p.heads);
    const int64_t row = rh / p.heads;

    const SplitRange range = split_range(p, row, split);
    if (range.request < 0) return;
    float* partial = p.partials + (rh * p.splits + split) * (int64_t)(D + 2);
    const float* prep = p.prep + rh * (int64_t)kPrepFloats;
    float q[32];
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(prep + kPrepScalars + lq * 32 + i);
        q[i] = v.x; q[i + 1] = v.y; q[i + 2] = v.z; q[i + 3] = v.w;
    }

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
    float m = -INFINITY, l = 0.f;
    const int32_t* table = p.block_table + (int64_t)range.request * p.block_table_stride;
    const int64_t page_elems = (int64_t)p.page_tokens * D;
    const int units_per_page = p.page_tokens / kUnitTokens;
    const uint16_t* cache = reinterpret_cast<const uint16_t*>(p.cache);
    const int64_t plane_elems = p.plane_stride / 2;

    for (int64_t u = range.unit_begin + wave; u < range.unit_end; u += kWaves) {
        const int64_t page_index = u / units_per_page;
        const int token = (int)(u % units_per_page) * kUnitTokens + t;
        const int64_t block = table[page_index];
        if (block < 0 || block >= p.num_blocks) continue;
        const bool valid = lane_active && page_index * p.page_tokens + token < range.history;
        const uint16_t* kp = cache + (block * p.heads + head) * page_elems + (int64_t)token * D + lq * 32;
        const uint16_t* vp = kp + plane_elems;
        uint4 kv[4], vv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kv[i] = reinterpret_cast<const uint4*>(kp)[i];
            vv[i] = reinterpret_cast<const uint4*>(vp)[i];
        }
        float lane_score = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lane_score = fmaf(q[8 * i + 2 * j], __uint_as_float(w[j] << 16), lane_score);
                lane_score = fmaf(q[8 * i + 2 * j + 1], __uint_as_float(w[j] & 0xffff0000u), lane_score);
            }
        }
        float score = quad_sum(lane_active ? lane_score : 0.f);
        score = valid ? score : -INFINITY;
        const float unit_max = token_max(score);
        if (unit_max > m) {
            const float factor = m == -INFINITY ? 0.f : exp2f(m - unit_max);
#pragma unroll
            for (int i = 0; i < 32; ++i) acc[i] *= factor;
            l *= factor;
            m = unit_max;
        }
        const float prob = valid ? exp2f(score - m) : 0.f;
        l += prob;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[8 * i + 2 * j] = fmaf(prob, __uint_as_float(w[j] << 16), acc[8 * i + 2 * j]);
                acc[8 * i + 2 * j + 1] = fmaf(prob, __uint_as_float(w[j] & 0xffff0000u), acc[8 * i + 2 * j + 1]);
            }
        }
    }
    write_partial<D>(acc, m, l, lane, wave, lane_active, partial);
}

// ------------------------------------------------------------------ merge

template <int D>
__global__ __launch_bounds__(128) void merge_kernel(AttentionParams p) {
    const int64_t row = blockIdx.x;
    const int head = blockIdx.y;
    const int c = threadIdx.x;
    __shared__ float weights[kMaxSplits];
    __shared__ float totals[2];
    __shared__ float history[128];
    const int request = p.row_request[row];
    if (request < 0) return;
    const int64_t rh = row * p.heads + head;
    const float live = p.prep[rh * kPrepFloats + 1];
    const float* parts = p.partials + rh * p.splits * (int64_t)(D + 2);
    if (c == 0) {
        float m = live;
        for (int s = 0; s < p.splits; ++s) m = fmaxf(m, parts[s * (D + 2)]);
        const float live_weight = exp2f(live - m);
        float denominator = live_weight;
        for (int s = 0; s < p.splits; ++s) {
            const float ms = parts[s * (D + 2)];
            const float w = ms == -INFINITY ? 0.f : exp2f(ms - m);
            weights[s] = w;
            denominator = fmaf(w, parts[s * (D + 2) + 1], denominator);
        }
        totals[0] = live_weight / denominator;
        totals[1] = 1.0f / denominator;
    }
    __syncthreads();
    float h = 0.f;
    if (c < D) {
        for (int s = 0; s < p.splits; ++s) h = fmaf(weights[s], parts[s * (D + 2) + 2 + c], h);
        h *= totals[1];
    }
    if (p.value_rotation != nullptr) {
        history[c] = h;
        __syncthreads();
        if (c < D) {
            const uint16_t* r = p.value_rotation + (int64_t)head * D * D + (int64_t)c * D;
            float acc = 0.f;
            for (int k = 0; k < D; ++k) acc = fmaf(history[k], f16_f32(r[k]), acc);
            h = acc;
        }
    }
    if (c < D) {
        const float v = bf16_f32(p.value[row * p.value_stride + head * D + c]);
        p.output[row * p.output_stride + head * D + c] = (uint16_t)bf16_rn(fmaf(totals[0], v, h));
    }
}

// ------------------------------------------------------------------ launch

template <int D, int BA, int GA, int BL, int GL, bool HasL>
void launch_decode(const AttentionParams& p, hipStream_t stream) {
    const unsigned blocks = (unsigned)(p.rows * p.heads * p.splits);
    hipLaunchKernelGGL((decode_kernel<D, BA, GA, BL, GL, HasL>), dim3(blocks), dim3(kDecodeThreads), 0,
                       stream, p);
}

template <int D, int BA, int GA>
bool dispatch_residual(const AttentionParams& p, hipStream_t stream) {
    if (!p.has_residual) {
        launch_decode<D, BA, GA, 2, 32, false>(p, stream);
        return true;
    }
    const int bits = p.residual.bits, group = p.residual.group;
    if (bits == 2 && group == 32) launch_decode<D, BA, GA, 2, 32, true>(p, stream);
    else if (bits == 2 && group == 16) launch_decode<D, BA, GA, 2, 16, true>(p, stream);
    else if (bits == 4 && group == 32) launch_decode<D, BA, GA, 4, 32, true>(p, stream);
    else if (bits == 4 && group == 16) launch_decode<D, BA, GA, 4, 16, true>(p, stream);
    else return false;
    return true;
}

template <int D>
bool dispatch_anchor(const AttentionParams& p, hipStream_t stream) {
    const int bits = p.anchor.bits, group = p.anchor.group;
    if (bits == 4 && group == 32) return dispatch_residual<D, 4, 32>(p, stream);
    if (bits == 4 && group == 16) return dispatch_residual<D, 4, 16>(p, stream);
    if (bits == 2 && group == 32) return dispatch_residual<D, 2, 32>(p, stream);
    if (bits == 2 && group == 16) return dispatch_residual<D, 2, 16>(p, stream);
    return false;
}

template <int D>
hipError_t launch_all(const AttentionParams& p, hipStream_t stream, hipEvent_t begin, hipEvent_t end,
                      bool bf16) {
    hipLaunchKernelGGL((prepare_kernel<D>), dim3((unsigned)p.rows, (unsigned)p.heads), dim3(128), 0,
                       stream, p);
    if (begin) hipEventRecord(begin, stream);
    if (bf16) {
        const unsigned blocks = (unsigned)(p.rows * p.heads * p.splits);
        hipLaunchKernelGGL((decode_bf16_kernel<D>), dim3(blocks), dim3(kDecodeThreads), 0, stream, p);
    } else if (!dispatch_anchor<D>(p, stream)) {
        return hipErrorInvalidValue;
    }
    if (end) hipEventRecord(end, stream);
    hipLaunchKernelGGL((merge_kernel<D>), dim3((unsigned)p.rows, (unsigned)p.heads), dim3(128), 0,
                       stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention(const AttentionParams& p, hipStream_t stream, hipEvent_t begin,
                            hipEvent_t end) {
    if (p.rows == 0) return hipSuccess;
    if (p.head_dim == 128) return launch_all<128>(p, stream, begin, end, false);
    if (p.head_dim == 96) return launch_all<96>(p, stream, begin, end, false);
    return hipErrorInvalidValue;
}

hipError_t launch_attention_bf16(const AttentionParams& p, hipStream_t stream, hipEvent_t begin,
                                 hipEvent_t end) {
    if (p.rows == 0) return hipSuccess;
    if (p.head_dim == 128) return launch_all<128>(p, stream, begin, end, true);
    if (p.head_dim == 96) return launch_all<96>(p, stream, begin, end, true);
    return hipErrorInvalidValue;
}

}  // namespace rq
