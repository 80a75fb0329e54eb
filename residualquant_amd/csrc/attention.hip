// Split-K paged decode attention over packed INT2/INT4 pages (gfx950).
//
// Semantics: the reference's attention() path
// (plugins/residual_quantization/csrc/attention/prepare.cuh:13-430,
// compute.cuh:226-727, merge.cuh:8-84, output.cuh:9-31).  Anchor mode, loop L:
// the history key of token t is K_L = alpha_L * K_A + deq_L (+ means), scored
// against q' = (q . R_k) / sqrt(D); the live token is folded in at the merge;
// the history value sum is inverse-rotated by R_v when given.
//
// Launches, with grids fixed by host shapes:
//   prepare  (rows x heads)          q' in log2 units, live score, group sums
//                                    of q', q' as 16-bit integers split into
//                                    four nibble planes for v_dot8_u32_u4
//                                    (with one split per (row, head) the
//                                    decode workgroup does this itself and
//                                    the call is one launch);
//   decode   (rows x heads x splits) one workgroup = 4 waves streaming the
//                                    pages of one split, two 16-token units
//                                    per wave iteration; lane = token x
//                                    32-channel quarter (decode_kernel), or
//                                    token x 48-channel half for D = 96
//                                    (decode96_dma_kernel); QK on
//                                    integer dot8 units, PV in FP32 registers,
//                                    online softmax per wave, LDS merge of the
//                                    waves; the split that finishes last for
//                                    its (row, head) does the log-sum-exp
//                                    merge of the splits and the live token,
//                                    the V inverse rotation and the BF16
//                                    output.
// The BF16 baseline keeps a separate merge launch.
#include "rq_chain.h"
#include "rq_device.h"
#include "rq_kernels.h"

namespace rq {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
#ifndef RQ_DECODE_WAVES
#define RQ_DECODE_WAVES 4
#endif
constexpr int kWaves = RQ_DECODE_WAVES;
constexpr int kDecodeThreads = 64 * kWaves;
static_assert(kWaves >= 4, "the finish and merge use at least 256 threads");
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

// Max over the 16 tokens of a unit (lane bits 2..5).
__device__ __forceinline__ float token_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 4));
    x = fmaxf(x, __shfl_xor(x, 8));
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float f16_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Reductions over the 16 lanes of a DPP row (lanes 16r..16r+15), the result
// in every lane of the row: quad exchanges, then rotations by 4 and 8 (each
// step a VALU operation, where a lane shuffle is an LDS round trip).
template <int Ctrl>
__device__ __forceinline__ int dpp_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, Ctrl, 0xF, 0xF, true);
}
__device__ __forceinline__ float row_sum16(float x) {
    x += __int_as_float(dpp_i<0xB1>(__float_as_int(x)));   // quad_perm [1,0,3,2]
    x += __int_as_float(dpp_i<0x4E>(__float_as_int(x)));   // quad_perm [2,3,0,1]
    x += __int_as_float(dpp_i<0x124>(__float_as_int(x)));  // row_ror:4
    return x + __int_as_float(dpp_i<0x128>(__float_as_int(x)));  // row_ror:8
}
__device__ __forceinline__ float row_max16(float x) {
    x = fmaxf(x, __int_as_float(dpp_i<0xB1>(__float_as_int(x))));
    x = fmaxf(x, __int_as_float(dpp_i<0x4E>(__float_as_int(x))));
    x = fmaxf(x, __int_as_float(dpp_i<0x124>(__float_as_int(x))));
    return fmaxf(x, __int_as_float(dpp_i<0x128>(__float_as_int(x))));
}
// OR over the aligned 8 lanes of x's lane (quad exchanges, then the
// half-row mirror pairs quad 0 with quad 1).
__device__ __forceinline__ uint32_t or8(uint32_t x) {
    x |= (uint32_t)dpp_i<0xB1>((int)x);
    x |= (uint32_t)dpp_i<0x4E>((int)x);
    return x | (uint32_t)dpp_i<0x141>((int)x);  // row_half_mirror
}
// OR over the 8 lanes of x's DPP row with the same lane parity.
__device__ __forceinline__ uint32_t or_parity16(uint32_t x) {
    x |= (uint32_t)dpp_i<0x4E>((int)x);
    x |= (uint32_t)dpp_i<0x124>((int)x);
    return x | (uint32_t)dpp_i<0x128>((int)x);
}
// Sum / max over the wave of row results (one readlane per row).
__device__ __forceinline__ float rows_sum(float x) {
    return (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16))) +
           (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32)) +
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48)));
}
__device__ __forceinline__ float rows_max(float x) {
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48))));
}

// A workgroup barrier for data exchanged through LDS by ordinary LDS
// accesses: this wave's LDS operations complete (s_waitcnt lgkmcnt(0)), then
// s_barrier; the empty asm statements keep the compiler from moving memory
// accesses across it.  __syncthreads (and an LDS release fence, which also
// covers LDS writes of DMA loads) waits for every load in flight
// (vmcnt(0)): in the decode prologues that would hold the query preparation
// until the first page loads, issued before it, have landed.  Not for data
// written to LDS by DMA loads or read from global memory.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ------------------------------------------------------------------ prepare


// Loads of the prepare that do not depend on the request: q, the live key and
// the two key means of (row, head), and R_k, all into registers.  Issued
// before the request lookup so their round trips overlap.  R_k stays in
// registers: thread t holds rows t % S, t % S + S, ... of the 8-channel
// column block t / S (S = 16 threads per block, or 8 in a 128-thread
// workgroup), so prepare_record multiplies q by its rows and the S threads of
// a block (adjacent lanes) add their sums with DPP.  prepare_record reads no
// global memory, so page loads issued after prepare_load and before
// prepare_record stay in flight (the waits for R_k count only the loads
// issued before them).
template <int D, int Threads>
struct PrepareInputs {
    static constexpr int kBlocks = D / 8;                          // 8-channel column blocks of R_k
    static constexpr int kSpan = Threads / kBlocks >= 16 ? 16 : 8;  // threads per block
    static constexpr int kRows = D / kSpan;                         // rows of R_k per thread
    static_assert(kBlocks * kSpan <= Threads && D % kSpan == 0, "every block has its threads");
    Chunk16 chunk[kRows];          // R_k[kSpan i + t % kSpan][8 (t / kSpan) .. + 7], FP16
    float mean_loop, mean_anchor;  // FP32 key means of channel min(c, D - 1) (0 without)
    uint32_t q_bits, k_bits;       // BF16 q and live key of that channel
};

template <int D, int Threads>
__device__ __forceinline__ void prepare_load(const AttentionParams& p, int64_t row, int head,
                                             PrepareInputs<D, Threads>& in) {
    using In = PrepareInputs<D, Threads>;
    // Unconditional loads (threads past D read channel D - 1; prepare_record
    // masks them), converted where they are used so nothing waits here.
    const int c = threadIdx.x;
    const int channel = c < D ? c : D - 1;
    in.q_bits = p.query[row * p.query_stride + head * D + channel];
    in.k_bits = p.key[row * p.key_stride + head * D + channel];
    in.mean_loop = p.key_mean_loop ? p.key_mean_loop[head * D + channel] : 0.f;
    in.mean_anchor = p.key_mean_anchor ? p.key_mean_anchor[head * D + channel] : 0.f;
    if (p.key_rotation != nullptr) {
        // Threads past the blocks read block 0 (prepare_record drops them).
        const int block = c < In::kBlocks * In::kSpan ? c / In::kSpan : 0;
        const Chunk16* src =
            reinterpret_cast<const Chunk16*>(p.key_rotation + (int64_t)head * D * D) + block + (c % In::kSpan) * (D / 8);
#pragma unroll
        for (int i = 0; i < In::kRows; ++i) in.chunk[i] = src[i * In::kSpan * (D / 8)];
    }
}

// Sum over the aligned 8 lanes of x's lane, in every one of them.
__device__ __forceinline__ float lanes8_sum(float x) {
    x += __int_as_float(dpp_i<0xB1>(__float_as_int(x)));   // quad_perm [1,0,3,2]
    x += __int_as_float(dpp_i<0x4E>(__float_as_int(x)));   // quad_perm [2,3,0,1]
    return x + __int_as_float(dpp_i<0x141>(__float_as_int(x)));  // row_half_mirror
}

// The prepared query record of one (row, head), written to `record`
// (kPrepFloats floats, global or LDS): [0] delta, [1] live score, [2] q'.mu_A,
// [3..10] 16-channel and [11..14] 32-channel group sums of q', then q'
// (FP32, log2 units) and its four nibble planes in the INT4 and INT2 word
// orders (prepare.cuh:13-229).  Called by every thread of a workgroup of 128
// or 256 threads (threads c >= D contribute nothing) after prepare_load.  It
// reads no global memory, and its barriers order LDS only, so page loads
// issued before it stay in flight.  Returns after a barrier with `record`
// complete when `record` is in LDS (a record in global memory is read by a
// later launch).
template <int D, int Threads>
__device__ __forceinline__ void prepare_record(const AttentionParams& p, int head,
                                               const PrepareInputs<D, Threads>& in, float* record) {
    using In = PrepareInputs<D, Threads>;
    __shared__ __attribute__((aligned(16))) float q_lds[128];
    __shared__ __attribute__((aligned(16))) float rotated_lds[128];
    __shared__ float totals[4][kDecodeThreads / 64];
    const int c = threadIdx.x;
    const int lane = c & 63;
    const int wave = c >> 6;
    const int waves = blockDim.x >> 6;
    const bool active = c < D;
    const float q = active ? bf16_f32(in.q_bits) : 0.f;
    const float k_live = active ? bf16_f32(in.k_bits) : 0.f;
    if (c < 128) q_lds[c] = q;
    lds_barrier();

    float qr = q;
    if (p.key_rotation != nullptr) {
        // q.R_k: the thread's rows of its column block, then the block's
        // kSpan threads added; the block's first thread publishes its 8
        // channels.
        const int r = c % In::kSpan;
        float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < In::kRows; ++i) {
            const float qk = q_lds[In::kSpan * i + r];
            const auto h = __builtin_bit_cast(_Float16 __attribute__((ext_vector_type(8))), in.chunk[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = fmaf(qk, (float)h[e], a[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = In::kSpan == 16 ? row_sum16(a[e]) : lanes8_sum(a[e]);
        if (r == 0 && c < In::kBlocks * In::kSpan) {
            float4* dst = reinterpret_cast<float4*>(rotated_lds + 8 * (c / In::kSpan));
            dst[0] = make_float4(a[0], a[1], a[2], a[3]);
            dst[1] = make_float4(a[4], a[5], a[6], a[7]);
        }
        lds_barrier();
        qr = active ? rotated_lds[c] : 0.f;
    }
    const float scale = kLog2e / sqrtf((float)D);
    qr *= scale;

    float parts[4];
    parts[0] = q * k_live;
    parts[1] = (active && p.key_mean_loop) ? qr * in.mean_loop : 0.f;
    // The anchor term of residual loops uses the BF16 mean (compute.cuh:327-336).
    parts[2] = (active && p.key_mean_anchor) ? qr * bf16_f32(bf16_rn(in.mean_anchor)) : 0.f;
    parts[3] = fabsf(qr);
    // Wave totals (row reductions, then one readlane per row).
    const float wave_parts[4] = {rows_sum(row_sum16(parts[0])), rows_sum(row_sum16(parts[1])),
                                 rows_sum(row_sum16(parts[2])), rows_max(row_max16(parts[3]))};
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) totals[i][wave] = wave_parts[i];
    }

    // Group sums of q' over 16 channels (a DPP row) and 32 (two rows).
    const float q16 = row_sum16(qr);
    const float q32 = lane < 32 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q16), 0)) +
                                      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q16), 16))
                                : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q16), 32)) +
                                      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q16), 48));
    lds_barrier();

    float sums[4] = {0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < waves; ++w) {
        sums[0] += totals[0][w];
        sums[1] += totals[1][w];
        sums[2] += totals[2][w];
        sums[3] = fmaxf(sums[3], totals[3][w]);
    }
    const float delta = sums[3] > 0.f ? sums[3] / 32767.0f : 1.0f;
    if (c == 0) {
        record[0] = delta;
        record[1] = scale * sums[0] - sums[1];
        record[2] = sums[2];
    }
    if (active && (c & 15) == 0) record[3 + c / 16] = q16;
    if (active && (c & 31) == 0) record[11 + c / 32] = q32;
    if (c < kPrepQuery) record[kPrepScalars + c] = active ? qr : 0.f;

    // 16-bit offset-binary integer of q', four nibble planes.
    const float scaled = fminf(fmaxf(rintf(qr / delta), -32767.f), 32767.f);
    const uint32_t qu = active ? (uint32_t)((int)scaled + 32768) : 32768u;
    uint32_t* planes4 = reinterpret_cast<uint32_t*>(record + kPrepScalars + kPrepQuery);
    uint32_t* planes2 = planes4 + kPrepPlanes;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t nibble = (qu >> (4 * j)) & 15u;
        // INT4 order: word c/8, nibble c%8.
        const uint32_t w4 = or8(nibble << (4 * (c & 7)));
        // INT2 order: 16-channel word c/16 split into even/odd channels,
        // nibble (c%16)/2 of nibble-word 2*(c/16) + c%2.
        const uint32_t w2 = or_parity16(nibble << (4 * ((c & 15) >> 1)));
        if (active && (c & 7) == 0) planes4[j * 16 + c / 8] = w4;
        if (active && (c & 14) == 0) planes2[j * 16 + 2 * (c / 16) + (c & 1)] = w2;
    }
    lds_barrier();
}

// Separate prepare pass (used when a (row, head) is split over several
// workgroups, and by the BF16 baseline): one 128-thread workgroup per (row, head).
template <int D>
__global__ __launch_bounds__(128) void prepare_kernel(AttentionParams p) {
    __shared__ int request_counts[2];
    const int64_t row = blockIdx.x;
    const int head = blockIdx.y;
    const int64_t rh = row * p.heads + head;
    if (threadIdx.x == 0) p.arrivals[rh] = 0;
    PrepareInputs<D, 128> in;
    prepare_load<D, 128>(p, row, head, in);
    const int request = find_request_parallel(p.query_start_loc, p.requests, row, request_counts);
    if (head == 0 && threadIdx.x == 0) p.row_request[row] = request;
    if (request < 0) return;
    prepare_record<D, 128>(p, head, in, p.prep + rh * (int64_t)kPrepFloats);
}

// ------------------------------------------------------------------ packed decode

template <int Bits>
struct Codes;
template <>
struct Codes<4> {
    uint32_t w[4];
};
template <>
struct Codes<2> {
    uint32_t w[2];
};

// Raw buffer resource over one page (wave-uniform, SGPRs): loads take a
// 32-bit lane offset plus a uniform offset, and reads past the page return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_resource(const uint8_t* page, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(page), (short)0, (int)bytes, 0x00020000);
}

// Cache policy of the page loads by head dimension: non-temporal (nt) or the
// default, for the code words and for the FP8 scale/offset and alpha bytes.
// Chosen by measurement (A/B on one box, eager calls timed by HIP events):
//   D = 128 (16 query heads, B32 x 8192): nt codes with default parameters
//     173 us per residual-loop call; nt everywhere 184 us; nt parameters with
//     default codes 192 us; default everywhere 203 us;
//   D = 96 (55 heads, B8 x 4096): default codes with nt parameters 88 us per
//     residual-loop call (the D96 kernel reads each token's codes with two
//     loads that interleave within every line, so a line streamed past L2
//     after the first is fetched again by the second); default everywhere
//     91 us; nt everywhere 97 us.
template <int D>
struct PagePolicy {
    static constexpr int kCodes = D == 128 ? kStreamPolicy : 0;
    static constexpr int kParams = D == 128 ? 0 : kStreamPolicy;
};

template <int Bits, int Policy>
__device__ __forceinline__ void load_codes(__amdgpu_buffer_rsrc_t page, uint32_t offset, uint32_t uniform,
                                           Codes<Bits>& c) {
    if constexpr (Bits == 4) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(page, offset, uniform, Policy);
        c.w[0] = v[0]; c.w[1] = v[1]; c.w[2] = v[2]; c.w[3] = v[3];
    } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(page, offset, uniform, Policy);
        c.w[0] = v[0]; c.w[1] = v[1];
    }
}

// Raw FP8 scale/offset bytes of the lane's group(s): one byte each for G32,
// two for G16; decoded (exactly, in hardware) where they are used.
template <int G>
struct GroupParams {
    uint32_t scales, offsets;
    template <int Policy>
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t page, uint32_t scale_offset,
                                         uint32_t offset_offset, uint32_t uniform) {
        if constexpr (G == 32) {
            scales = __builtin_amdgcn_raw_buffer_load_b8(page, scale_offset, uniform, Policy);
            offsets = __builtin_amdgcn_raw_buffer_load_b8(page, offset_offset, uniform, Policy);
        } else {
            scales = __builtin_amdgcn_raw_buffer_load_b16(page, scale_offset, uniform, Policy);
            offsets = __builtin_amdgcn_raw_buffer_load_b16(page, offset_offset, uniform, Policy);
        }
    }
    // Scale / offset of the lane's 16-channel half H.
    template <int H>
    __device__ __forceinline__ float scale() const { return fp8_f32<G == 32 ? 0 : H>(scales); }
    template <int H>
    __device__ __forceinline__ float offset() const { return fp8_f32<G == 32 ? 0 : H>(offsets); }
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
        dot[h] = (int)(d[h][0] + 16u * d[h][1] + 256u * d[h][2] + 4096u * d[h][3]) - 32768 * (int)count[h];
}

// acc[c] += weight[half(c)] * code[c] over the lane's 32 channels.  A code c
// held in a byte is the FP8 E4M3 value c * 2^-9, so v_cvt_pk_f32_fp8 turns two
// codes into FP32 per instruction; `weight` carries the 2^9 back.
template <int Bits>
__device__ __forceinline__ void accumulate_codes(const Codes<Bits>& codes, const float (&weight)[2],
                                                 float (&acc)[32]) {
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float w = weight[i >> 1];
            const int lo = (int)(codes.w[i] & 0x0f0f0f0fu);         // channels 0, 2, 4, 6
            const int hi = (int)((codes.w[i] >> 4) & 0x0f0f0f0fu);  // channels 1, 3, 5, 7
            const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
            const auto l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            float* a = acc + 8 * i;
            a[0] = fmaf(w, l01[0], a[0]);
            a[2] = fmaf(w, l01[1], a[2]);
            a[4] = fmaf(w, l23[0], a[4]);
            a[6] = fmaf(w, l23[1], a[6]);
            a[1] = fmaf(w, h01[0], a[1]);
            a[3] = fmaf(w, h01[1], a[3]);
            a[5] = fmaf(w, h23[0], a[5]);
            a[7] = fmaf(w, h23[1], a[7]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float w = weight[i];
            float* a = acc + 16 * i;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // byte j of part holds channel 4j + k
                const int part = (int)((codes.w[i] >> (2 * k)) & 0x03030303u);
                const auto c01 = __builtin_amdgcn_cvt_pk_f32_fp8(part, false);
                const auto c23 = __builtin_amdgcn_cvt_pk_f32_fp8(part, true);
                a[k] = fmaf(w, c01[0], a[k]);
                a[4 + k] = fmaf(w, c01[1], a[4 + k]);
                a[8 + k] = fmaf(w, c23[0], a[8 + k]);
                a[12 + k] = fmaf(w, c23[1], a[12 + k]);
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

// Lane part of one record's score: sum over the lane's group(s) of
// scale * delta * (q_int . codes) + offset * sum(q').
template <int G>
__device__ __forceinline__ float record_score(const GroupParams<G>& gp, const int (&dot)[2],
                                              float delta, const float (&q_sum)[2]) {
    if constexpr (G == 32)
        return gp.template scale<0>() * (delta * (float)(dot[0] + dot[1])) + gp.template offset<0>() * q_sum[0];
    else
        return gp.template scale<0>() * (delta * (float)dot[0]) + gp.template offset<0>() * q_sum[0] +
               gp.template scale<1>() * (delta * (float)dot[1]) + gp.template offset<1>() * q_sum[1];
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

constexpr int kReduceBytes = kWaves * 16 * 128 * (int)sizeof(float);

// The four waves' (m, l, acc) of one split merged in LDS: thread c < D gets
// channel c of the unnormalized output; every thread gets m and l.
struct SplitResult {
    float sum, m, l;
};

template <int D>
__device__ __forceinline__ SplitResult merge_waves(float (&acc)[32], float m, float l_lane, int lane, int wave,
                                                   bool lane_active, float* lds) {
    // lds: kWaves * 16 * 128 floats, [wave][token][channel].
    float (*red_acc)[16][128] = reinterpret_cast<float (*)[16][128]>(lds);
    __shared__ float red_m[kWaves], red_l[kWaves];
    const int t = lane >> 2, qd = lane & 3;
    // Sum over the quarter-0 lanes: rotations within each row, then rows.
    float l_rows = (lane_active && qd == 0) ? l_lane : 0.f;
    l_rows += __int_as_float(dpp_i<0x124>(__float_as_int(l_rows)));
    l_rows += __int_as_float(dpp_i<0x128>(__float_as_int(l_rows)));
    const float l_wave = rows_sum(l_rows);
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
    SplitResult r;
    r.m = m_all;
    r.l = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) r.l += red_m[w] == -INFINITY ? 0.f : red_l[w] * exp2f(red_m[w] - m_all);
    r.sum = 0.f;
    const int c = threadIdx.x;
    if (c < D) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int tt = 0; tt < 16; ++tt) r.sum += red_acc[w][tt][c];
    }
    return r;
}

// Writes (m, l, acc[D]) of this split for the merge.
template <int D>
__device__ __forceinline__ void write_partial(const SplitResult& r, float* partial) {
    const int c = threadIdx.x;
    const __amdgpu_buffer_rsrc_t out = handoff_resource(partial, (D + 2) * 4);
    if (c < D) handoff_store(out, 8 + 4 * c, r.sum);
    if (c == 0) {
        handoff_store(out, 0, r.m);
        handoff_store(out, 4, r.l);
    }
}

// One split covers the whole history of this (row, head): merge the waves
// (`merge_waves()` returns this split's SplitResult), fold in the live token,
// inverse-rotate V and write the BF16 output without a round trip through the
// partials.  R_v row c and the live value are loaded before the wave merge so
// their latency overlaps it.
template <int D, typename MergeWaves>
__device__ __forceinline__ void finish_single(const AttentionParams& p, int64_t row, int head, float live,
                                              MergeWaves merge_waves) {
    __shared__ float hist[128];
    __shared__ float halves[2][128];
    const int tid = threadIdx.x;
    const int c = tid & 127, part = tid >> 7;
    const bool in_halves = tid < 256;  // two threads per channel, half of k each
    const bool rotate = p.value_rotation != nullptr;
    uint4 rv[D / 16];
    if (rotate && c < D && in_halves) {
        const uint4* r = reinterpret_cast<const uint4*>(p.value_rotation + ((int64_t)head * D + c) * D + part * (D / 2));
#pragma unroll
        for (int i = 0; i < D / 16; ++i) rv[i] = r[i];
    }
    const float v_live = tid < D ? bf16_f32(p.value[row * p.value_stride + head * D + tid]) : 0.f;

    const SplitResult r = merge_waves();
    const float mx = fmaxf(r.m, live);
    const float w_hist = r.m == -INFINITY ? 0.f : exp2f(r.m - mx);
    const float w_live = exp2f(live - mx);
    const float inv = 1.0f / fmaf(w_hist, r.l, w_live);
    if (tid < 128) hist[c] = c < D ? r.sum * (w_hist * inv) : 0.f;
    __syncthreads();
    float o = 0.f;
    if (c < D && in_halves) {
        if (rotate) {
            float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < D / 16; ++i) {
                const float* hk = hist + part * (D / 2) + 8 * i;
                const uint32_t w[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[j] = fmaf(hk[2 * j], f16_f32((uint16_t)(w[j] & 0xffffu)), a[j]);
                    a[j] = fmaf(hk[2 * j + 1], f16_f32((uint16_t)(w[j] >> 16)), a[j]);
                }
            }
            o = (a[0] + a[1]) + (a[2] + a[3]);
        } else if (part == 0) {
            o = hist[c];
        }
    }
    if (in_halves) halves[part][c] = o;
    __syncthreads();
    if (tid < D)
        p.output[row * p.output_stride + head * D + tid] =
            (uint16_t)bf16_rn(fmaf(w_live * inv, v_live, halves[0][tid] + halves[1][tid]));
}

// Page range of one split (in 16-token units) for the request of `row`.
struct SplitRange {
    int request;
    int64_t history, unit_begin, unit_end;
};

// The split's units of `request` whose sequence holds `seq_len` tokens (the
// live one included).
__device__ __forceinline__ SplitRange split_range_of(const AttentionParams& p, int request, int seq_len, int split) {
    SplitRange r;
    r.request = request;
    r.history = 0;
    r.unit_begin = r.unit_end = 0;
    if (r.request < 0) return r;
    int64_t history = (int64_t)seq_len - 1;
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

__device__ __forceinline__ SplitRange split_range(const AttentionParams& p, int request, int split) {
    return split_range_of(p, request, request < 0 ? 0 : p.seq_lens[request], split);
}

// Request and split range of `row` for a workgroup that looks them up itself
// (the fused prepare).  Decode batches map rows one-to-one to requests
// (query_start_loc = 0, 1, 2, ...), so request `row` is tried first: its two
// query_start_loc bounds and its sequence length are read with scalar loads
// issued together, one round trip, where the lookup and then the length read
// would take two or more.  Any other mapping takes the parallel lookup.
// Workgroup-uniform; the lookup's barrier is taken by every thread or none.
__device__ __forceinline__ SplitRange fused_range(const AttentionParams& p, int64_t row, int split, int* lds_counts) {
    SplitRange none;
    none.request = -1;
    none.history = none.unit_begin = none.unit_end = 0;
    if (p.requests <= 0) return none;
    const ConstantInt32* qsl = (const ConstantInt32*)p.query_start_loc;
    const ConstantInt32* lens = (const ConstantInt32*)p.seq_lens;
    const int64_t guess = row < p.requests ? row : p.requests - 1;
    const int lo = qsl[guess], hi = qsl[guess + 1], len = lens[guess];
    // Everything below uses all three values before any branch, so the three
    // loads are issued together (with a short-circuit test the compiler
    // branches after each one and serialises the round trips).
    const bool own = (lo <= row) & (row < hi);
    const SplitRange guessed = split_range_of(p, (int)guess, len, split);
    if (own) return guessed;
    const int request = find_request_parallel(p.query_start_loc, p.requests, row, lds_counts);
    return split_range_of(p, request, request < 0 ? 0 : lens[request], split);
}

// Wave max of one value per token, broadcast to every lane (quad lanes agree).
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xF, 0xF, true)));  // row_ror:4
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, true)));  // row_ror:8
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ float quad_sum_fast(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));
    return x + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));
}

// Integer q'.codes of two units at once, with the nibble planes read from LDS
// one code word at a time (planes[word][plane], shared by both units).
template <int Bits>
__device__ __forceinline__ void code_dots2(const Codes<Bits>& c0, const Codes<Bits>& c1,
                                           const uint32_t* planes, int (&dot0)[2], int (&dot1)[2]) {
    uint32_t d0[2][4] = {}, d1[2][4] = {};
    uint32_t n0[2] = {0u, 0u}, n1[2] = {0u, 0u};
    constexpr uint32_t kOnes = 0x11111111u;
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = i >> 1;
            const uint4 q = *reinterpret_cast<const uint4*>(planes + 4 * i);
            const uint32_t qj[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                d0[h][j] = __builtin_amdgcn_udot8(qj[j], c0.w[i], d0[h][j], false);
                d1[h][j] = __builtin_amdgcn_udot8(qj[j], c1.w[i], d1[h][j], false);
            }
            n0[h] = __builtin_amdgcn_udot8(kOnes, c0.w[i], n0[h], false);
            n1[h] = __builtin_amdgcn_udot8(kOnes, c1.w[i], n1[h], false);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t e0 = c0.w[i] & 0x33333333u, o0 = (c0.w[i] >> 2) & 0x33333333u;
            const uint32_t e1 = c1.w[i] & 0x33333333u, o1 = (c1.w[i] >> 2) & 0x33333333u;
            const uint4 qe = *reinterpret_cast<const uint4*>(planes + 4 * (2 * i));
            const uint4 qo = *reinterpret_cast<const uint4*>(planes + 4 * (2 * i + 1));
            const uint32_t ej[4] = {qe.x, qe.y, qe.z, qe.w};
            const uint32_t oj[4] = {qo.x, qo.y, qo.z, qo.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                d0[i][j] = __builtin_amdgcn_udot8(ej[j], e0, d0[i][j], false);
                d0[i][j] = __builtin_amdgcn_udot8(oj[j], o0, d0[i][j], false);
                d1[i][j] = __builtin_amdgcn_udot8(ej[j], e1, d1[i][j], false);
                d1[i][j] = __builtin_amdgcn_udot8(oj[j], o1, d1[i][j], false);
            }
            n0[i] = __builtin_amdgcn_udot8(kOnes, e0, __builtin_amdgcn_udot8(kOnes, o0, n0[i], false), false);
            n1[i] = __builtin_amdgcn_udot8(kOnes, e1, __builtin_amdgcn_udot8(kOnes, o1, n1[i], false), false);
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        dot0[h] = (int)(d0[h][0] + 16u * d0[h][1] + 256u * d0[h][2] + 4096u * d0[h][3]) - 32768 * (int)n0[h];
        dot1[h] = (int)(d1[h][0] + 16u * d1[h][1] + 256u * d1[h][2] + 4096u * d1[h][3]) - 32768 * (int)n1[h];
    }
}

// Registers of one 16-token unit: K/V codes, raw FP8 parameters, alphas.
template <int BA, int GA, int BL, int GL, bool HasL>
struct Unit {
    Codes<BA> kca, vca;
    GroupParams<GA> kpa, vpa;
    Codes<BL> kcl, vcl;
    GroupParams<GL> kpl, vpl;
    uint32_t alpha_k_bits, alpha_v_bits;
};

// ------------------------------------------------------------------ merge

constexpr int kMergeThreads = 256;

// Log-sum-exp merge of the splits of one (row, head) and the live token, the
// inverse V rotation, and the BF16 output, by a 256-thread workgroup
// (merge.cuh:8-84, output.cuh:9-31, rotation.cuh:10-84).  `lds` holds at
// least kMergeLdsFloats floats; the caller has made every split's partial
// visible to this workgroup.
constexpr int kMergeLdsFloats = kMaxSplits + 4 + 128 + kWaves * 128;

template <int D>
__device__ __forceinline__ void merge_output(const AttentionParams& p, int64_t row, int head, float* lds) {
    const int tid = threadIdx.x;
    const int64_t rh = row * p.heads + head;
    float* weights = lds;                    // [kMaxSplits]
    float* totals = lds + kMaxSplits;        // [2]: live weight, 1 / denominator
    float* hist = totals + 4;                // [128]
    float* halves = hist + 128;              // [waves][128]
    // Partials [split][D + 2] of this (row, head), read with coherent loads.
    constexpr uint32_t kSplitBytes = (D + 2) * 4;
    const __amdgpu_buffer_rsrc_t parts =
        handoff_resource(p.partials + rh * p.splits * (int64_t)(D + 2), (uint32_t)(p.splits * kSplitBytes));
    if (tid < 64) {
        // One lane per split (splits <= 64): (m, l) of split tid.
        const float live = p.prep[rh * kPrepFloats + 1];
        const bool has = tid < p.splits;
        const float2 ml = has ? handoff_load2(parts, tid * kSplitBytes) : make_float2(-INFINITY, 0.f);
        float m = fmaxf(ml.x, live);
#pragma unroll
        for (int d = 32; d; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
        const float w = ml.x == -INFINITY ? 0.f : exp2f(ml.x - m);
        float denominator = w * ml.y;
#pragma unroll
        for (int d = 32; d; d >>= 1) denominator += __shfl_xor(denominator, d);
        const float live_weight = exp2f(live - m);
        denominator += live_weight;
        if (has) weights[tid] = w;
        if (tid == 0) {
            totals[0] = live_weight / denominator;
            totals[1] = 1.0f / denominator;
        }
    }
    __syncthreads();
    // History sum: thread = (channel pair, split group); every load of a
    // thread is independent, so they are all in flight together.
    const int groups = blockDim.x >> 6;
    {
        const int pair = tid & 63, group = tid >> 6;
        float2 h = make_float2(0.f, 0.f);
        if (2 * pair < D) {
#pragma unroll 8
            for (int s = group; s < p.splits; s += groups) {
                const float2 v = handoff_load2(parts, s * kSplitBytes + 8 + 8 * pair);
                h.x = fmaf(weights[s], v.x, h.x);
                h.y = fmaf(weights[s], v.y, h.y);
            }
        }
        halves[group * 128 + 2 * pair] = h.x;
        halves[group * 128 + 2 * pair + 1] = h.y;
    }
    __syncthreads();
    const int c = tid & 127, part = tid >> 7;
    if (tid < 128) {
        float sum = 0.f;
        for (int g = 0; g < groups; ++g) sum += halves[g * 128 + c];
        hist[c] = c < D ? sum * totals[1] : 0.f;
    }
    __syncthreads();
    // out[c] = sum_k hist[k] R_v[c][k]: half `part` of the k range per thread
    // (the first 256 threads), R_v row c read straight from global memory (L2)
    // as 16-byte vectors.
    const bool in_halves = tid < 256;
    float o = 0.f;
    if (c < D && in_halves) {
        if (p.value_rotation != nullptr) {
            const uint4* r = reinterpret_cast<const uint4*>(p.value_rotation + ((int64_t)head * D + c) * D +
                                                            part * (D / 2));
            float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < D / 16; ++i) {
                const uint4 v = r[i];
                const float* hk = hist + part * (D / 2) + 8 * i;
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[j] = fmaf(hk[2 * j], f16_f32((uint16_t)(w[j] & 0xffffu)), a[j]);
                    a[j] = fmaf(hk[2 * j + 1], f16_f32((uint16_t)(w[j] >> 16)), a[j]);
                }
            }
            o = (a[0] + a[1]) + (a[2] + a[3]);
        } else if (part == 0) {
            o = hist[c];
        }
    }
    __syncthreads();
    if (in_halves) halves[part * 128 + c] = o;
    __syncthreads();
    if (tid < D) {
        const float v = bf16_f32(p.value[row * p.value_stride + head * D + tid]);
        p.output[row * p.output_stride + head * D + tid] =
            (uint16_t)bf16_rn(fmaf(totals[0], v, halves[tid] + halves[128 + tid]));
    }
}

// Separate merge pass (used by the BF16 baseline): one workgroup per (row, head).
template <int D>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(AttentionParams p) {
    __shared__ float lds[kMergeLdsFloats];
    const int64_t row = blockIdx.x;
    if (p.row_request[row] < 0) return;
    merge_output<D>(p, row, blockIdx.y, lds);
}

// The split that finishes last for its (row, head) merges: every split
// publishes its partial, then counts itself in `arrivals` (zeroed by prepare);
// the one that sees splits - 1 earlier arrivals reads them all.  Nothing
// waits, so no workgroup depends on another being scheduled.
template <int D>
__device__ __forceinline__ void finish_split(const AttentionParams& p, int64_t row, int head) {
    __shared__ float lds[kMergeLdsFloats];
    __shared__ int last;
    if (!arrive_last(&p.arrivals[row * p.heads + head], p.splits, &last)) return;
    merge_output<D>(p, row, head, lds);
}

#ifndef RQ_DECODE_MIN_WAVES
#define RQ_DECODE_MIN_WAVES 1
#endif

template <int D, int PT, int BA, int GA, int BL, int GL, bool HasL>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(RQ_DECODE_MIN_WAVES)))
void decode_kernel(AttentionParams p) {
    constexpr int Quarters = D / 32;
    constexpr int UnitsPerPage = PT / kUnitTokens;
    constexpr int CodeA = D * BA / 8, GroupsA = D / GA;
    constexpr int CodeL = D * BL / 8, GroupsL = D / GL;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = lane >> 2;
    const int qd = lane & 3;
    const bool lane_active = qd < Quarters;
    const int lq = lane_active ? qd : 0;
    const int split = blockIdx.x % p.splits;
    const int64_t rh = blockIdx.x / p.splits;
    const int head = (int)(rh % p.heads);
    const int64_t row = rh / p.heads;
    // Nibble planes of q' per quarter: [quarter][anchor words 0..3 | loop words 0..3][plane]
    __shared__ __attribute__((aligned(16))) uint32_t planes_lds[4][8][4];
    __shared__ __attribute__((aligned(16))) float prep_lds[kPrepFloats];
    // The wave merge at the end.
    __shared__ __attribute__((aligned(16))) float scratch_lds[kWaves * 16 * 128];
    __shared__ int request_counts[kWaves];

    // With one split per (row, head) this workgroup prepares its own query;
    // otherwise prepare_kernel has written the record.  The request lookup
    // comes first either way, so the first units' page loads are in flight
    // while the query record is computed (the loop's first iteration uses them).
    SplitRange range;
    PrepareInputs<D, kDecodeThreads> in;
    if (p.fused_prepare) {
        prepare_load<D, kDecodeThreads>(p, row, head, in);
        range = fused_range(p, row, split, request_counts);
    } else {
        range = split_range(p, p.row_request[row], split);
    }
    if (range.request < 0) return;
    // The range is the same in every lane; kept in scalar registers so the
    // block table below is read with scalar loads.
    range.request = __builtin_amdgcn_readfirstlane(range.request);
    range.history = uniform64(range.history);
    range.unit_begin = uniform64(range.unit_begin);
    range.unit_end = uniform64(range.unit_end);
    float* partial = p.partials + (rh * p.splits + split) * (int64_t)(D + 2);

    // Per-lane byte offsets inside a page (first 16-token half); the second
    // half of a 32-token page adds a wave-uniform step per region.
    const uint32_t off_codes_a = p.anchor.offset + t * CodeA + lq * (32 * BA / 8);
    const uint32_t off_scale_a = p.anchor.offset + PT * CodeA + t * GroupsA + lq * (32 / GA);
    const uint32_t off_offs_a = off_scale_a + PT * GroupsA;
    const uint32_t off_codes_l = p.residual.offset + t * CodeL + lq * (32 * BL / 8);
    const uint32_t off_scale_l = p.residual.offset + PT * CodeL + t * GroupsL + lq * (32 / GL);
    const uint32_t off_offs_l = off_scale_l + PT * GroupsL;
    const uint32_t off_alpha = p.residual.offset + PT * (CodeL + 2 * GroupsL) + 2 * t;

    // Block table entries are read through the scalar cache: their waits
    // (lgkmcnt) are not ordered behind the page loads in flight (vmcnt counts
    // vector loads in issue order, so a vector read of the next entry would
    // wait for every page load issued before it).
    const ConstantInt32* table =
        (const ConstantInt32*)(p.block_table + (int64_t)range.request * p.block_table_stride);
    const int64_t page_bytes = (int64_t)PT * p.page_width;
    const int64_t history = range.history;
    // Units u (even) and u + 1 share a page when a page holds an even number of units.
    constexpr bool kPairSharesPage = UnitsPerPage % 2 == 0;
    struct PairBlocks {
        int first, second;
    };
    auto pair_blocks = [&](int64_t u) -> PairBlocks {
        PairBlocks b{-1, -1};
        if (u < range.unit_end) {
            b.first = table[u / UnitsPerPage];
            if (kPairSharesPage)
                b.second = b.first;
            else if (u + 1 < range.unit_end)
                b.second = table[(u + 1) / UnitsPerPage];
        }
        return b;
    };

    // Issues the loads of unit u of `block` whether or not the block is valid
    // (a missing block, or -1 past the range, gets an empty buffer: its loads
    // read zeros and touch no memory), so no branch sits between the loads of
    // consecutive units and the compiler can count them (vmcnt) exactly.
    auto load_unit = [&](int block, int64_t u, Unit<BA, GA, BL, GL, HasL>& d) -> bool {
        const int half = (int)(u % UnitsPerPage);
        const bool valid = block >= 0 && block < p.num_blocks;
        const uint8_t* kbase = p.cache + (valid ? ((int64_t)block * p.heads + head) * page_bytes : 0);
        const uint32_t bytes = valid ? (uint32_t)page_bytes : 0u;
        const __amdgpu_buffer_rsrc_t kpage = page_resource(kbase, bytes);
        const __amdgpu_buffer_rsrc_t vpage = page_resource(kbase + (valid ? p.plane_stride : 0), bytes);
        const uint32_t step_codes_a = half * (kUnitTokens * CodeA);
        const uint32_t step_par_a = half * (kUnitTokens * GroupsA);
        using Policy = PagePolicy<D>;
        load_codes<BA, Policy::kCodes>(kpage, off_codes_a, step_codes_a, d.kca);
        d.kpa.template load<Policy::kParams>(kpage, off_scale_a, off_offs_a, step_par_a);
        load_codes<BA, Policy::kCodes>(vpage, off_codes_a, step_codes_a, d.vca);
        d.vpa.template load<Policy::kParams>(vpage, off_scale_a, off_offs_a, step_par_a);
        if constexpr (HasL) {
            const uint32_t step_codes_l = half * (kUnitTokens * CodeL);
            const uint32_t step_par_l = half * (kUnitTokens * GroupsL);
            const uint32_t step_alpha = half * (2 * kUnitTokens);
            load_codes<BL, Policy::kCodes>(kpage, off_codes_l, step_codes_l, d.kcl);
            d.kpl.template load<Policy::kParams>(kpage, off_scale_l, off_offs_l, step_par_l);
            load_codes<BL, Policy::kCodes>(vpage, off_codes_l, step_codes_l, d.vcl);
            d.vpl.template load<Policy::kParams>(vpage, off_scale_l, off_offs_l, step_par_l);
            d.alpha_k_bits = __builtin_amdgcn_raw_buffer_load_b16(kpage, off_alpha, step_alpha, Policy::kParams);
            d.alpha_v_bits = __builtin_amdgcn_raw_buffer_load_b16(vpage, off_alpha, step_alpha, Policy::kParams);
        }
        return valid;
    };

    const int64_t first = range.unit_begin + 2 * wave;
    Unit<BA, GA, BL, GL, HasL> d0, d1;
    bool ok0 = false, ok1 = false;
    // Issued while the prologue's own loads (R_k, q) may still be in flight:
    // those are older, so the record's arithmetic below waits for them and
    // for none of the page loads.
    PairBlocks blocks = pair_blocks(first);
    ok0 = load_unit(blocks.first, first, d0);
    ok1 = load_unit(blocks.second, first + 1, d1);
    // Table entries of the next iteration, read while this one computes.
    blocks = pair_blocks(first + 2 * kWaves);

    if (p.fused_prepare) {
        prepare_record<D, kDecodeThreads>(p, head, in, prep_lds);
    } else {
        const float* src = p.prep + rh * (int64_t)kPrepFloats;
        for (int i = threadIdx.x; i < kPrepFloats; i += kDecodeThreads) prep_lds[i] = src[i];
        __syncthreads();
    }
    const float* prep = prep_lds;
    if (threadIdx.x < 128) {
        // thread -> (quarter, record, word, plane); prep stores [plane][word] per order
        const int quarter = threadIdx.x >> 5, record = (threadIdx.x >> 4) & 1;
        const int word = (threadIdx.x >> 2) & 3, plane = threadIdx.x & 3;
        const int bits = record == 0 ? BA : BL;
        const uint32_t* base = reinterpret_cast<const uint32_t*>(prep + kPrepScalars + kPrepQuery) +
                               (bits == 2 ? kPrepPlanes : 0);
        planes_lds[quarter][record * 4 + word][plane] =
            quarter < Quarters ? base[plane * 16 + 4 * quarter + word] : 0u;
    }
    const float delta = prep[0];
    const float q_mean_anchor = prep[2];
    float q_sum_a[2], q_sum_l[2];
    group_sums<GA>(prep, lq, q_sum_a);
    group_sums<GL>(prep, lq, q_sum_l);
    lds_barrier();
    const uint32_t* planes_a = &planes_lds[lq][0][0];
    const uint32_t* planes_l = &planes_lds[lq][4][0];

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
    float cst0 = 0.f, cst1 = 0.f;
    float m = -INFINITY, l = 0.f;

    // Values of one unit: acc += p * (alpha_v * deq_A + deq_L); offsets go to cst.
    // A token past the history has p = 0, but its slot may hold any bytes
    // (0 x NaN is NaN), so its raw scale, offset and alpha bits are selected
    // to 0 before they are converted (its codes are integers and harmless).
    auto accumulate = [&](const Unit<BA, GA, BL, GL, HasL>& d, float prob, bool valid) {
        const float p512 = prob * 512.0f;
        GroupParams<GA> vpa = d.vpa;
        vpa.scales = valid ? vpa.scales : 0u;
        vpa.offsets = valid ? vpa.offsets : 0u;
        float w_a[2];
        if constexpr (HasL) {
            GroupParams<GL> vpl = d.vpl;
            vpl.scales = valid ? vpl.scales : 0u;
            vpl.offsets = valid ? vpl.offsets : 0u;
            const float alpha_v = __uint_as_float((valid ? d.alpha_v_bits : 0u) << 16);
            const float pa = prob * alpha_v;
            const float pa512 = p512 * alpha_v;
            w_a[0] = pa512 * vpa.template scale<0>();
            w_a[1] = GA == 32 ? w_a[0] : pa512 * vpa.template scale<1>();
            float w_l[2];
            w_l[0] = p512 * vpl.template scale<0>();
            w_l[1] = GL == 32 ? w_l[0] : p512 * vpl.template scale<1>();
            cst0 += fmaf(pa, vpa.template offset<0>(), prob * vpl.template offset<0>());
            cst1 += fmaf(pa, vpa.template offset<1>(), prob * vpl.template offset<1>());
            accumulate_codes<BL>(d.vcl, w_l, acc);
        } else {
            w_a[0] = p512 * vpa.template scale<0>();
            w_a[1] = GA == 32 ? w_a[0] : p512 * vpa.template scale<1>();
            cst0 += prob * vpa.template offset<0>();
            cst1 += prob * vpa.template offset<1>();
        }
        accumulate_codes<BA>(d.vca, w_a, acc);
    };

    // Scores, softmax and values of the unit pair (u, u + 1) held in (d0, d1).
    auto process = [&](Unit<BA, GA, BL, GL, HasL>& d0, Unit<BA, GA, BL, GL, HasL>& d1, bool ok0, bool ok1,
                       int64_t u) {
        const int64_t pos0 = (u / UnitsPerPage) * PT + (u % UnitsPerPage) * kUnitTokens + t;
        const int64_t pos1 = ((u + 1) / UnitsPerPage) * PT + ((u + 1) % UnitsPerPage) * kUnitTokens + t;
        const bool valid0 = ok0 && lane_active && pos0 < history;
        const bool valid1 = ok1 && lane_active && pos1 < history;

        int da0[2], da1[2];
        code_dots2<BA>(d0.kca, d1.kca, planes_a, da0, da1);
        float s0 = record_score<GA>(d0.kpa, da0, delta, q_sum_a);
        float s1 = record_score<GA>(d1.kpa, da1, delta, q_sum_a);
        if constexpr (HasL) {
            int dl0[2], dl1[2];
            code_dots2<BL>(d0.kcl, d1.kcl, planes_l, dl0, dl1);
            const float mean_part = qd == 0 ? q_mean_anchor : 0.f;
            s0 = __uint_as_float(d0.alpha_k_bits << 16) * (s0 + mean_part) +
                 record_score<GL>(d0.kpl, dl0, delta, q_sum_l);
            s1 = __uint_as_float(d1.alpha_k_bits << 16) * (s1 + mean_part) +
                 record_score<GL>(d1.kpl, dl1, delta, q_sum_l);
        }
        float score0 = quad_sum_fast(lane_active ? s0 : 0.f);
        float score1 = quad_sum_fast(lane_active ? s1 : 0.f);
        score0 = valid0 ? score0 : -INFINITY;
        score1 = valid1 ? score1 : -INFINITY;

        const float unit_max = wave_max(fmaxf(score0, score1));
        if (unit_max > m) {
            const float factor = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - unit_max);
#pragma unroll
            for (int i = 0; i < 32; ++i) acc[i] *= factor;
            cst0 *= factor;
            cst1 *= factor;
            l *= factor;
            m = unit_max;
        }
        const float prob0 = valid0 ? __builtin_amdgcn_exp2f(score0 - m) : 0.f;
        const float prob1 = valid1 ? __builtin_amdgcn_exp2f(score1 - m) : 0.f;
        l += prob0 + prob1;
        accumulate(d0, prob0, valid0);
        accumulate(d1, prob1, valid1);
    };

    // Each iteration streams two consecutive 16-token units of the split
    // (the first iteration's were loaded before the query preparation).
    const int iterations =
        first < range.unit_end ? (int)((range.unit_end - first + 2 * kWaves - 1) / (2 * kWaves)) : 0;
    const StreamPriority priority(iterations, p.stream_priority != 0);
    int step = 0;
    for (int64_t u = first; u < range.unit_end; u += 2 * kWaves, ++step) {
        priority.set(step);
        if (u != first) {
            ok0 = load_unit(blocks.first, u, d0);
            ok1 = load_unit(blocks.second, u + 1, d1);
            blocks = pair_blocks(u + 2 * kWaves);
        }
        process(d0, d1, ok0, ok1, u);
    }
    __builtin_amdgcn_s_setprio(0);

#pragma unroll
    for (int i = 0; i < 16; ++i) {
        acc[i] += cst0;
        acc[16 + i] += cst1;
    }
    if (p.splits == 1) {
        finish_single<D>(p, row, head, prep_lds[1],
                         [&] { return merge_waves<D>(acc, m, l, lane, wave, lane_active, scratch_lds); });
    } else {
        write_partial<D>(merge_waves<D>(acc, m, l, lane, wave, lane_active, scratch_lds), partial);
        finish_split<D>(p, row, head);
    }
}

// ------------------------------------------------------------------ D = 96 packed decode
//
// decode_kernel maps lane = token x 32-channel quarter, which leaves one lane
// in four idle at D = 96.  The D = 96 kernel below gives every lane one
// token's 48-channel half instead: lane = 2 * slot + half, and a wave
// iteration covers two 16-token units (slots 0..15: unit u, slots 16..31:
// unit u + 1).  A half is three 16-channel blocks: six INT4 or three INT2 code
// words; block b of half h belongs to group (3h + b) * 16 / G.

template <int Bits>
struct HalfCodes {
    static constexpr int kWords = Bits == 4 ? 6 : 3;
    uint32_t w[kWords];
};

// Raw FP8 scale/offset bytes of a half's groups, first group in byte 0:
// three groups for G16 (one per block), two for G32 (groups h and h + 1),
// read as the two aligned dwords at or below the first byte and shifted into
// place (v_alignbyte).
template <int G>
struct HalfParams {
    uint32_t s, o;
    // Scale and offset of each of the three blocks of half `upper`.
    __device__ __forceinline__ void decode(bool upper, float (&scale)[3], float (&offset)[3]) const {
        if constexpr (G == 16) {
            scale[0] = fp8_f32<0>(s); scale[1] = fp8_f32<1>(s); scale[2] = fp8_f32<2>(s);
            offset[0] = fp8_f32<0>(o); offset[1] = fp8_f32<1>(o); offset[2] = fp8_f32<2>(o);
        } else {
            const float s0 = fp8_f32<0>(s), s1 = fp8_f32<1>(s);
            const float o0 = fp8_f32<0>(o), o1 = fp8_f32<1>(o);
            scale[0] = s0; scale[1] = upper ? s1 : s0; scale[2] = s1;
            offset[0] = o0; offset[1] = upper ? o1 : o0; offset[2] = o1;
        }
    }
};

// Integer q'.codes of the half's three blocks.  planes[i][j] (LDS): nibble
// plane j of the half's i-th plane word (INT4: code word i; INT2: even (2b) /
// odd (2b + 1) channels of code word b), one 16-byte read per word.
template <int Bits>
__device__ __forceinline__ void half_dots(const HalfCodes<Bits>& c, const uint32_t (*planes)[4], int (&dot)[3]) {
    uint32_t d[3][4] = {};
    uint32_t n[3] = {0u, 0u, 0u};
    constexpr uint32_t kOnes = 0x11111111u;
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            const int b = i >> 1;
            const uint4 q = *reinterpret_cast<const uint4*>(planes[i]);
            const uint32_t qj[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) d[b][j] = __builtin_amdgcn_udot8(qj[j], c.w[i], d[b][j], false);
            n[b] = __builtin_amdgcn_udot8(kOnes, c.w[i], n[b], false);
        }
    } else {
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            const uint32_t even = c.w[b] & 0x33333333u, odd = (c.w[b] >> 2) & 0x33333333u;
            const uint4 qe = *reinterpret_cast<const uint4*>(planes[2 * b]);
            const uint4 qo = *reinterpret_cast<const uint4*>(planes[2 * b + 1]);
            const uint32_t ej[4] = {qe.x, qe.y, qe.z, qe.w};
            const uint32_t oj[4] = {qo.x, qo.y, qo.z, qo.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                d[b][j] = __builtin_amdgcn_udot8(ej[j], even, d[b][j], false);
                d[b][j] = __builtin_amdgcn_udot8(oj[j], odd, d[b][j], false);
            }
            n[b] = __builtin_amdgcn_udot8(kOnes, even, __builtin_amdgcn_udot8(kOnes, odd, n[b], false), false);
        }
    }
#pragma unroll
    for (int b = 0; b < 3; ++b)
        dot[b] = (int)(d[b][0] + 16u * d[b][1] + 256u * d[b][2] + 4096u * d[b][3]) - 32768 * (int)n[b];
}

// Lane part of one record's score: sum over the half's blocks of
// scale * delta * (q_int . codes) + offset * sum(q').
__device__ __forceinline__ float half_score(const float (&scale)[3], const float (&offset)[3], const int (&dot)[3],
                                            float delta, const float (&q_sum)[3]) {
    float s = 0.f;
#pragma unroll
    for (int b = 0; b < 3; ++b) s += scale[b] * (delta * (float)dot[b]) + offset[b] * q_sum[b];
    return s;
}

// acc[16b + i] += weight[b] * code over the half's 48 channels (codes are
// FP8 E4M3 values c * 2^-9 when held in a byte, as in accumulate_codes).
template <int Bits>
__device__ __forceinline__ void accumulate_half(const HalfCodes<Bits>& c, const float (&weight)[3],
                                                float (&acc)[48]) {
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            const float w = weight[i >> 1];
            const int lo = (int)(c.w[i] & 0x0f0f0f0fu);
            const int hi = (int)((c.w[i] >> 4) & 0x0f0f0f0fu);
            const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
            const auto l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            float* a = acc + 8 * i;
            a[0] = fmaf(w, l01[0], a[0]);
            a[2] = fmaf(w, l01[1], a[2]);
            a[4] = fmaf(w, l23[0], a[4]);
            a[6] = fmaf(w, l23[1], a[6]);
            a[1] = fmaf(w, h01[0], a[1]);
            a[3] = fmaf(w, h01[1], a[3]);
            a[5] = fmaf(w, h23[0], a[5]);
            a[7] = fmaf(w, h23[1], a[7]);
        }
    } else {
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            const float w = weight[b];
            float* a = acc + 16 * b;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int part = (int)((c.w[b] >> (2 * k)) & 0x03030303u);  // byte j: channel 4j + k
                const auto c01 = __builtin_amdgcn_cvt_pk_f32_fp8(part, false);
                const auto c23 = __builtin_amdgcn_cvt_pk_f32_fp8(part, true);
                a[k] = fmaf(w, c01[0], a[k]);
                a[4 + k] = fmaf(w, c01[1], a[4 + k]);
                a[8 + k] = fmaf(w, c23[0], a[8 + k]);
                a[12 + k] = fmaf(w, c23[1], a[12 + k]);
            }
        }
    }
}

// Max over the wave of one value per token slot (the two lanes of a slot
// agree), broadcast to every lane.
__device__ __forceinline__ float slot_wave_max(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xF, 0xF, true)));  // row_ror:2
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xF, 0xF, true)));  // row_ror:4
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, true)));  // row_ror:8
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The four waves' (m, l, acc) of one split in the half layout, merged
// in LDS: thread c < 96 gets channel c of the unnormalized output, every
// thread gets m and l.  Slot pairs are added with DPP first, so the LDS holds
// [wave][slot pair][96] (kWaves * 16 * 96 floats of `lds`).
__device__ __forceinline__ SplitResult merge_waves_half(float (&acc)[48], float m, float l_lane, int lane,
                                                        int wave, float* lds) {
    constexpr int D = 96;
    float (*red_acc)[16][D] = reinterpret_cast<float (*)[16][D]>(lds);
    __shared__ float red_m[kWaves], red_l[kWaves];
    const float l_wave = rows_sum(row_sum16(l_lane));  // carried by the half-0 lanes only
    if (lane == 0) {
        red_m[wave] = m;
        red_l[wave] = l_wave;
    }
    __syncthreads();
    float m_all = red_m[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m_all = fmaxf(m_all, red_m[w]);
    const float wave_scale = m == -INFINITY ? 0.f : exp2f(m - m_all);
    float pair[48];
#pragma unroll
    for (int i = 0; i < 48; ++i) pair[i] = (acc[i] + quad_xor2(acc[i])) * wave_scale;  // slots 2k, 2k + 1
    if ((lane & 2) == 0) {
        float* dst = &red_acc[wave][lane >> 2][48 * (lane & 1)];
#pragma unroll
        for (int i = 0; i < 48; i += 4) *reinterpret_cast<float4*>(dst + i) = make_float4(pair[i], pair[i + 1], pair[i + 2], pair[i + 3]);
    }
    __syncthreads();
    SplitResult r;
    r.m = m_all;
    r.l = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) r.l += red_m[w] == -INFINITY ? 0.f : red_l[w] * exp2f(red_m[w] - m_all);
    r.sum = 0.f;
    const int c = threadIdx.x;
    if (c < D) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int k = 0; k < 16; ++k) r.sum += red_acc[w][k][c];
    }
    return r;
}

// Registers of one lane's token: K/V codes, raw FP8 parameters, alphas.
template <int BA, int GA, int BL, int GL, bool HasL>
struct HalfUnit {
    HalfCodes<BA> kca, vca;
    HalfParams<GA> kpa, vpa;
    HalfCodes<BL> kcl, vcl;
    HalfParams<GL> kpl, vpl;
    uint32_t alpha_k_bits, alpha_v_bits;
};

// ------------------------------------------------------------------ D = 96 decode with DMA-staged pages
//
// The half-lane arithmetic above, with each wave iteration's page spans
// staged in LDS by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds)
// instead of per-lane register loads.  A 1 KB DMA load moves 64 lane-linear 16-byte
// chunks of the staged spans (the loop record with its alphas, then the
// anchor record without them, async_copy.cuh:24-42), so one iteration's two
// pages of K and V take 6 loads (C4 schedule) where the register form issues
// 16 narrow loads per lane; and the staged bytes sit in LDS, not in
// registers, so each wave keeps kDma96Stages iterations of loads in flight.
// A no-arithmetic gather of a C4 residual call through such rings measured
// 56.8 us against 71.7 us for per-lane register loads of the same spans.
// Lanes then read their token half's code words, FP8 parameters and alpha
// from LDS (lane = 2 * slot + half).  The per-lane 32-bit page offsets
// address one buffer resource per plane, so launch_decode uses this kernel
// when a plane fits in 4 GiB of buffer offsets.
constexpr int kDma96Stages = 3;

template <int PT, int BA, int GA, int BL, int GL, bool HasL>
struct Dma96Layout {
    static constexpr int D = 96;
    static constexpr int CodeA = D * BA / 8, GroupsA = D / GA;
    static constexpr int CodeL = D * BL / 8, GroupsL = D / GL;
    static constexpr int BytesA = CodeA + 2 * GroupsA + 2, BytesL = CodeL + 2 * GroupsL + 2;
    static constexpr int SpanL = HasL ? PT * BytesL : 0;       // the loop record, alphas included
    static constexpr int SpanA = PT * (BytesA - 2);            // the anchor record without its alphas
    static constexpr int PageBytes = SpanL + SpanA;            // staged bytes of one page and plane
    static constexpr int Pages = 32 / PT;                      // pages of one wave iteration (32 tokens)
    static constexpr int PlaneChunks = Pages * PageBytes / 16;
    static constexpr int PlaneLoads = (PlaneChunks + 63) / 64;  // 1 KB DMA loads per plane and iteration
    static constexpr int PlaneBytes = PlaneLoads * 1024;
    static constexpr int StageBytes = 2 * PlaneBytes;          // K region, then V region
    // One stage of the ring, [wave][K region, V region], plus 64 bytes: a
    // lane's FP8 parameter words are read as two aligned dwords, which can
    // reach 4 bytes past the last staged span.
    static constexpr int RingStageBytes = kWaves * StageBytes + 64;
    static_assert(SpanL % 16 == 0 && SpanA % 16 == 0, "staged spans are whole 16-byte chunks");
};

typedef __attribute__((address_space(3))) void LdsVoid96;

// One DMA load: lane l's 16 bytes at `offset` of the resource go to lds + 16 l
// (lds wave-uniform).  A __device__ function, not a call inside a kernel's
// lambda: there the host pass drops the kernel's launch stub.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, uint32_t offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LdsVoid96*)lds, 16, offset, 0, 0, kStreamPolicy);
}

// s_waitcnt vmcnt(N) (bits [3:0] and [15:14]), not waiting on expcnt or lgkmcnt.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt takes 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int PT, int BA, int GA, int BL, int GL, bool HasL>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(2)))
void decode96_dma_kernel(AttentionParams p) {
    using L = Dma96Layout<PT, BA, GA, BL, GL, HasL>;
    constexpr int D = 96;
    constexpr int UnitsPerPage = PT / kUnitTokens;
    constexpr int CodeA = L::CodeA, GroupsA = L::GroupsA, CodeL = L::CodeL, GroupsL = L::GroupsL;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = lane >> 1;          // token slot of the iteration, 0..31
    const int h = lane & 1;              // channel half
    const bool upper = slot >= 16;       // slot on the iteration's second unit
    const int tok = PT == 32 ? slot : (slot & 15);  // token row inside the slot's page
    const int page_of_slot = PT == 32 ? 0 : (upper ? 1 : 0);
    const int split = blockIdx.x % p.splits;
    const int64_t rh = blockIdx.x / p.splits;
    const int head = (int)(rh % p.heads);
    const int64_t row = rh / p.heads;
    __shared__ __attribute__((aligned(16))) float prep_lds[kPrepFloats];
    __shared__ __attribute__((aligned(16))) uint32_t half_planes[2][2][6][4];
    __shared__ int request_counts[kWaves];
    // The three stages of the staging ring are separate LDS objects: the
    // compiler makes an LDS read wait for every DMA load in flight that may
    // write the object it reads, so with one object for all stages the
    // reads of one stage would wait for the loads of the others.  Stage 2
    // also holds the wave merge (kWaves x 16 x D floats), after the last
    // load.
    constexpr int kScratchBytes = (int)sizeof(float) * kWaves * 16 * D;
    __shared__ __attribute__((aligned(16))) uint8_t ring0[L::RingStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t ring1[L::RingStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t ring2[L::RingStageBytes > kScratchBytes ? L::RingStageBytes
                                                                                           : kScratchBytes];
    float* scratch_lds = reinterpret_cast<float*>(ring2);

    SplitRange range;
    PrepareInputs<D, kDecodeThreads> in;
    if (p.fused_prepare) {
        prepare_load<D, kDecodeThreads>(p, row, head, in);
        range = fused_range(p, row, split, request_counts);
    } else {
        range = split_range(p, p.row_request[row], split);
    }
    if (range.request < 0) return;
    range.request = __builtin_amdgcn_readfirstlane(range.request);
    range.history = uniform64(range.history);
    range.unit_begin = uniform64(range.unit_begin);
    range.unit_end = uniform64(range.unit_end);
    float* partial = p.partials + (rh * p.splits + split) * (int64_t)(D + 2);

    const ConstantInt32* table =
        (const ConstantInt32*)(p.block_table + (int64_t)range.request * p.block_table_stride);
    const uint32_t page_bytes = (uint32_t)PT * (uint32_t)p.page_width;
    const __amdgpu_buffer_rsrc_t kplane = page_resource(p.cache, (uint32_t)p.plane_stride);
    const __amdgpu_buffer_rsrc_t vplane = page_resource(p.cache + p.plane_stride, (uint32_t)p.plane_stride);
    // A page that is missing (past the split or an invalid block id) is
    // addressed past every plane: its loads return zeros and fetch nothing.
    constexpr uint32_t kMissing = 0xFFFF0000u;

    // Each lane's chunks of the DMA loads: load j of a plane moves chunks
    // 64 j + lane of the iteration's staged bytes (page-major, then the loop
    // record's span, then the anchor's), i.e. page q = chunk / (PageBytes /
    // 16) at byte offset chunk_offset[j] of that page.  Chunks past the end
    // repeat the first (their LDS bytes are never read).
    uint32_t chunk_offset[L::PlaneLoads];
    bool chunk_second[L::PlaneLoads];
#pragma unroll
    for (int j = 0; j < L::PlaneLoads; ++j) {
        int c = 64 * j + lane;
        c = c < L::PlaneChunks ? c : 0;
        const int q = c / (L::PageBytes / 16);
        const int b = 16 * (c % (L::PageBytes / 16));
        chunk_second[j] = q == 1;
        chunk_offset[j] = b < L::SpanL ? (uint32_t)p.residual.offset + b : (uint32_t)p.anchor.offset + (b - L::SpanL);
    }

    // Iteration g of this wave covers units (u, u + 1), u = first + 2 kWaves g.
    const int64_t first = range.unit_begin + 2 * wave;
    const int64_t unit_step = 2 * kWaves;
    const int iterations = first < range.unit_end ? (int)((range.unit_end - first + unit_step - 1) / unit_step) : 0;
    struct PagePair {
        uint32_t base0, base1;  // page byte offsets in the plane (kMissing if absent)
    };
    auto pages_of = [&](int g) -> PagePair {
        const int64_t u = first + unit_step * g;
        PagePair r{kMissing, kMissing};
        if (g < iterations) {
            const int b0 = table[u / UnitsPerPage];
            if (b0 >= 0 && b0 < p.num_blocks) r.base0 = ((uint32_t)b0 * (uint32_t)p.heads + (uint32_t)head) * page_bytes;
            if (PT == 16 && u + 1 < range.unit_end) {
                const int b1 = table[(u + 1) / UnitsPerPage];
                if (b1 >= 0 && b1 < p.num_blocks)
                    r.base1 = ((uint32_t)b1 * (uint32_t)p.heads + (uint32_t)head) * page_bytes;
            }
        }
        return r;
    };
    auto stage_base = [&](auto stage_constant) __attribute__((always_inline)) {
        constexpr int stage = decltype(stage_constant)::value;
        return (stage == 0 ? ring0 : stage == 1 ? ring1 : ring2) + wave * L::StageBytes;
    };
    using Stage0 = std::integral_constant<int, 0>;
    using Stage1 = std::integral_constant<int, 1>;
    using Stage2 = std::integral_constant<int, 2>;
    uint32_t dma_offset[L::PlaneLoads];
    auto issue = [&](const PagePair& pages, auto stage_constant) __attribute__((always_inline)) {
        uint8_t* dst = stage_base(stage_constant);
#pragma unroll
        for (int j = 0; j < L::PlaneLoads; ++j) {
            const uint32_t base = chunk_second[j] ? pages.base1 : pages.base0;
            dma_offset[j] = base == kMissing ? kMissing : base + chunk_offset[j];
            dma16(kplane, dst + 1024 * j, dma_offset[j]);
        }
#pragma unroll
        for (int j = 0; j < L::PlaneLoads; ++j) dma16(vplane, dst + L::PlaneBytes + 1024 * j, dma_offset[j]);
    };

    // The first two stages' loads are in flight while the query record is
    // prepared.  The stages' page pairs live in three variables (an array
    // indexed by the loop counter would sit in scratch memory, whose loads
    // share vmcnt with the DMA loads).
    static_assert(kDma96Stages == 3, "the loop below rotates three stages");
    PagePair pages0 = pages_of(0), pages1 = pages_of(1), pages2;
    if (!p.fused_prepare) {
        const float* src = p.prep + rh * (int64_t)kPrepFloats;
        for (int i = threadIdx.x; i < kPrepFloats; i += kDecodeThreads) prep_lds[i] = src[i];
    }
    // The prologue's own loads (R_k, q) may still be in flight: they are
    // older than the page loads, so the query preparation waits for them
    // only, and every wait of the loop below, which counts the page loads
    // issued after the stage it consumes, also covers them.  The
    // prologue's barriers order LDS only, so the first stages stream while
    // the query record is prepared.
    issue(pages0, Stage0{});
    issue(pages1, Stage1{});

    if (p.fused_prepare) prepare_record<D, kDecodeThreads>(p, head, in, prep_lds);
    else lds_barrier();
    const float* prep = prep_lds;
    const float delta = prep[0];
    const float q_mean_anchor = h == 0 ? prep[2] : 0.f;  // added once per token
    float q_sum[3];
#pragma unroll
    for (int b = 0; b < 3; ++b) q_sum[b] = prep[3 + 3 * h + b];
    // Nibble planes per half, [record (anchor, loop)][half][word][plane].
    if (threadIdx.x < 96) {
        const int record = threadIdx.x / 48, half = (threadIdx.x / 24) & 1;
        const int word = (threadIdx.x >> 2) % 6, plane = threadIdx.x & 3;
        const int bits = record == 0 ? BA : BL;
        const uint32_t* base = reinterpret_cast<const uint32_t*>(prep + kPrepScalars + kPrepQuery) +
                               (bits == 2 ? kPrepPlanes : 0);
        half_planes[record][half][word][plane] = base[plane * 16 + 6 * half + word];
    }
    lds_barrier();
    const uint32_t (*planes_a)[4] = half_planes[0][h];
    const uint32_t (*planes_l)[4] = half_planes[1][h];

    // Byte offsets of the lane's fields inside a staged page (plane region).
    const uint32_t first_a = tok * GroupsA + (GA == 16 ? 3 * h : h);
    const uint32_t first_l = tok * GroupsL + (GL == 16 ? 3 * h : h);
    const uint32_t shift_a = first_a & 3u, shift_l = first_l & 3u;
    const uint32_t lds_page = page_of_slot * L::PageBytes;
    const uint32_t at_codes_a = lds_page + L::SpanL + tok * CodeA + h * (CodeA / 2);
    const uint32_t at_scale_a = lds_page + L::SpanL + PT * CodeA + (first_a & ~3u);
    const uint32_t at_offs_a = at_scale_a + PT * GroupsA;
    const uint32_t at_codes_l = lds_page + tok * CodeL + h * (CodeL / 2);
    const uint32_t at_scale_l = lds_page + PT * CodeL + (first_l & ~3u);
    const uint32_t at_offs_l = at_scale_l + PT * GroupsL;
    const uint32_t at_alpha = lds_page + PT * (CodeL + 2 * GroupsL) + 2 * tok;

    auto word_at = [](const uint8_t* base, uint32_t at) { return *reinterpret_cast<const uint32_t*>(base + at); };
    auto codes_at = [&](const uint8_t* plane, uint32_t at, auto& c) __attribute__((always_inline)) {
        // INT4: 24 bytes at an 8-byte boundary; INT2: 12 bytes at a 4-byte boundary.
        constexpr int Words = std::remove_reference_t<decltype(c)>::kWords;
        if constexpr (Words == 6) {
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                const uint2 v = *reinterpret_cast<const uint2*>(plane + at + 8 * i);
                c.w[2 * i] = v.x;
                c.w[2 * i + 1] = v.y;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 3; ++i) c.w[i] = word_at(plane, at + 4 * i);
        }
    };
    auto params_at = [&](const uint8_t* plane, uint32_t at_scale, uint32_t at_offs, uint32_t shift, auto& prm)
        __attribute__((always_inline)) {
        prm.s = __builtin_amdgcn_alignbyte(word_at(plane, at_scale + 4), word_at(plane, at_scale), shift);
        prm.o = __builtin_amdgcn_alignbyte(word_at(plane, at_offs + 4), word_at(plane, at_offs), shift);
    };

    float acc[48];
#pragma unroll
    for (int i = 0; i < 48; ++i) acc[i] = 0.f;
    float cst[3] = {0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    // Iteration g consumes stage g % 3 after issuing stage (g + 2) % 3
    // (iteration g - 1's stage, whose reads are complete).
    const StreamPriority priority(iterations, p.stream_priority != 0);
    auto iteration = [&](int g, auto stage_constant) __attribute__((always_inline)) {
        constexpr int stage = decltype(stage_constant)::value;
        constexpr int ahead = (stage + 2) % 3;
        priority.set(g);
        const PagePair next = pages_of(g + 2);
        issue(next, std::integral_constant<int, ahead>{});
        const PagePair cur = stage == 0 ? pages0 : stage == 1 ? pages1 : pages2;
        if constexpr (ahead == 0)
            pages0 = next;
        else if constexpr (ahead == 1)
            pages1 = next;
        else
            pages2 = next;
        wait_vmcnt<2 * 2 * L::PlaneLoads>();
        const uint8_t* kst = stage_base(stage_constant);
        const uint8_t* vst = kst + L::PlaneBytes;
        const int64_t u = first + unit_step * g;
        const int64_t unit = u + (upper ? 1 : 0);
        // Branch-free (a divergent branch here makes the compiler wait for
        // every DMA load in flight before the stage's first LDS read).
        const bool ok = (page_of_slot ? cur.base1 : cur.base0) != kMissing;
        const bool valid = ok & (unit < range.unit_end) & (16 * unit + (slot & 15) < range.history);
        HalfUnit<BA, GA, BL, GL, HasL> d;
        codes_at(kst, at_codes_a, d.kca);
        params_at(kst, at_scale_a, at_offs_a, shift_a, d.kpa);
        if constexpr (HasL) {
            codes_at(kst, at_codes_l, d.kcl);
            params_at(kst, at_scale_l, at_offs_l, shift_l, d.kpl);
            d.alpha_k_bits = *reinterpret_cast<const uint16_t*>(kst + at_alpha);
        }

        float sa[3], oa[3];
        d.kpa.decode(h != 0, sa, oa);
        int da[3];
        half_dots<BA>(d.kca, planes_a, da);
        float s = half_score(sa, oa, da, delta, q_sum);
        if constexpr (HasL) {
            float sl[3], ol[3];
            d.kpl.decode(h != 0, sl, ol);
            int dl[3];
            half_dots<BL>(d.kcl, planes_l, dl);
            s = __uint_as_float(d.alpha_k_bits << 16) * (s + q_mean_anchor) + half_score(sl, ol, dl, delta, q_sum);
        }
        float score = s + quad_xor1(s);  // the token's two halves
        score = valid ? score : -INFINITY;

        const float unit_max = slot_wave_max(score);
        if (unit_max > m) {
            const float factor = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - unit_max);
#pragma unroll
            for (int i = 0; i < 48; ++i) acc[i] *= factor;
#pragma unroll
            for (int b = 0; b < 3; ++b) cst[b] *= factor;
            l *= factor;
            m = unit_max;
        }
        const float prob = valid ? __builtin_amdgcn_exp2f(score - m) : 0.f;
        l += h == 0 ? prob : 0.f;

        codes_at(vst, at_codes_a, d.vca);
        params_at(vst, at_scale_a, at_offs_a, shift_a, d.vpa);
        if constexpr (HasL) {
            codes_at(vst, at_codes_l, d.vcl);
            params_at(vst, at_scale_l, at_offs_l, shift_l, d.vpl);
            d.alpha_v_bits = *reinterpret_cast<const uint16_t*>(vst + at_alpha);
        }
        // Values: acc += p * (alpha_v * deq_A + deq_L); offsets go to cst.  A
        // token past the history (or of a missing page) has p = 0, but its
        // bytes may be anything (0 x NaN is NaN): its raw scale, offset and
        // alpha bits are selected to 0 before they are converted.
        const float p512 = prob * 512.0f;
        HalfParams<GA> vpa = d.vpa;
        vpa.s = valid ? vpa.s : 0u;
        vpa.o = valid ? vpa.o : 0u;
        float sva[3], ova[3];
        vpa.decode(h != 0, sva, ova);
        float w_a[3];
        if constexpr (HasL) {
            HalfParams<GL> vpl = d.vpl;
            vpl.s = valid ? vpl.s : 0u;
            vpl.o = valid ? vpl.o : 0u;
            const float alpha_v = __uint_as_float((valid ? d.alpha_v_bits : 0u) << 16);
            const float pa = prob * alpha_v;
            const float pa512 = p512 * alpha_v;
            float svl[3], ovl[3];
            vpl.decode(h != 0, svl, ovl);
            float w_l[3];
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                w_a[b] = pa512 * sva[b];
                w_l[b] = p512 * svl[b];
                cst[b] += fmaf(pa, ova[b], prob * ovl[b]);
            }
            accumulate_half<BL>(d.vcl, w_l, acc);
        } else {
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                w_a[b] = p512 * sva[b];
                cst[b] += prob * ova[b];
            }
        }
        accumulate_half<BA>(d.vca, w_a, acc);
        // This stage's LDS reads are complete before the next iteration's
        // DMA into it can land.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int g = 0; g < iterations; g += 3) {
        iteration(g, Stage0{});
        if (g + 1 < iterations) iteration(g + 1, Stage1{});
        if (g + 2 < iterations) iteration(g + 2, Stage2{});
    }
    __builtin_amdgcn_s_setprio(0);
    // The loads of the stages past the last iteration (zero-byte fetches of
    // missing pages) have landed before the LDS is reused or the wave exits.
    wait_vmcnt<0>();

#pragma unroll
    for (int b = 0; b < 3; ++b)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[16 * b + i] += cst[b];
    if (p.splits == 1) {
        finish_single<D>(p, row, head, prep_lds[1],
                         [&] { return merge_waves_half(acc, m, l, lane, wave, scratch_lds); });
    } else {
        write_partial<D>(merge_waves_half(acc, m, l, lane, wave, scratch_lds), partial);
        finish_split<D>(p, row, head);
    }
}

// ------------------------------------------------------------------ adjacent mode, loops > 0
//
// Adjacent mode stores each loop as a residual of the previous loop, so the
// key and value of loop L are the BF16 restore chain over records 0..L
// (compute.cuh:120-197, :506-528; the chain arithmetic is in rq_chain.h).
// The chain is not linear in the codes, so decode_chain_kernel rebuilds each
// token's K and V (lane = token x 32-channel quarter, one 16-token unit per
// wave iteration) and scores and accumulates them.

// Links = records in the chain (2..4).  A wave's units are software
// pipelined: the raw bytes of its next unit are loaded before the current
// unit is decoded, scored and accumulated.
template <int D, int PT, int Links>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(2)))
void decode_chain_kernel(AttentionParams p) {
    constexpr int Quarters = D / 32;
    constexpr int UnitsPerPage = PT / kUnitTokens;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = lane >> 2;
    const int qd = lane & 3;
    const bool lane_active = qd < Quarters;
    const int lq = lane_active ? qd : 0;
    const int split = blockIdx.x % p.splits;
    const int64_t rh = blockIdx.x / p.splits;
    const int head = (int)(rh % p.heads);
    const int64_t row = rh / p.heads;
    __shared__ __attribute__((aligned(16))) float prep_lds[kPrepFloats];
    // bf16(mu_r) of records 0 .. L - 1 (the K plane's chain), FP32.
    __shared__ __attribute__((aligned(16))) float mean_lds[kMaxRecords][128];
    __shared__ __attribute__((aligned(16))) float scratch_lds[kWaves * 16 * 128];
    // q' as BF16 pairs of channels (2j, 2j + 1): [0] bf16(q'), [1] bf16(q' - bf16(q')).
    __shared__ __attribute__((aligned(16))) uint32_t qpair_lds[2][64];
    __shared__ int request_counts[kWaves];

    SplitRange range;
    PrepareInputs<D, kDecodeThreads> in;
    if (p.fused_prepare) {
        prepare_load<D, kDecodeThreads>(p, row, head, in);
        range = fused_range(p, row, split, request_counts);
    } else {
        range = split_range(p, p.row_request[row], split);
    }
    if (range.request < 0) return;
    range.request = __builtin_amdgcn_readfirstlane(range.request);
    range.history = uniform64(range.history);
    range.unit_begin = uniform64(range.unit_begin);
    range.unit_end = uniform64(range.unit_end);
    float* partial = p.partials + (rh * p.splits + split) * (int64_t)(D + 2);

    for (int i = threadIdx.x; i < (Links - 1) * 128; i += kDecodeThreads) {
        const int r = i / 128, c = i % 128;
        mean_lds[r][c] = (p.key_mean_all != nullptr && c < D)
                             ? bf16_f32(bf16_rn(p.key_mean_all[((int64_t)r * p.heads + head) * D + c]))
                             : 0.f;
    }
    if (p.fused_prepare) {
        prepare_record<D, kDecodeThreads>(p, head, in, prep_lds);
    } else {
        const float* src = p.prep + rh * (int64_t)kPrepFloats;
        for (int i = threadIdx.x; i < kPrepFloats; i += kDecodeThreads) prep_lds[i] = src[i];
        __syncthreads();
    }
    // q' (FP32, log2 units, scale folded in) as a high and a low BF16 pair
    // per two channels (16 bits of mantissa: relative error 2^-17), so the
    // score is two v_dot2_f32_bf16 per channel pair.  It stays in LDS and is
    // read per unit: registers are what limits the kernel to two waves per SIMD.
    if (threadIdx.x < 64) {
        const float a = prep_lds[kPrepScalars + 2 * threadIdx.x], b = prep_lds[kPrepScalars + 2 * threadIdx.x + 1];
        const uint32_t hi = bf16_pack(a, b);
        qpair_lds[0][threadIdx.x] = hi;
        qpair_lds[1][threadIdx.x] = bf16_pack(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
    }
    __syncthreads();
    const uint4* qhi4 = reinterpret_cast<const uint4*>(&qpair_lds[0][16 * lq]);
    const uint4* qlo4 = reinterpret_cast<const uint4*>(&qpair_lds[1][16 * lq]);
    // The pairs (1, 0) and (0, 1) of the mean add, in registers.
    uint32_t pick_lo = 0x00003f80u, pick_hi = 0x3f800000u;
    asm("" : "+v"(pick_lo), "+v"(pick_hi));

    const ConstantInt32* table =
        (const ConstantInt32*)(p.block_table + (int64_t)range.request * p.block_table_stride);
    const int64_t page_bytes = (int64_t)PT * p.page_width;
    const bool has_mean = p.key_mean_all != nullptr;
    RecordRegion regs[Links];
#pragma unroll
    for (int r = 0; r < Links; ++r) regs[r] = p.chain[r];

    // Raw bytes of every record of a unit, K and V planes.  Units past the
    // split read zeros (an empty page resource).
    ChainRaw rk[Links], rv[Links];
    struct UnitPages {
        __amdgpu_buffer_rsrc_t k, v;
        int tok;
        bool ok;
    };
    auto unit_pages = [&](int64_t u) {
        const bool inside = u < range.unit_end;
        const int block = inside ? table[u / UnitsPerPage] : -1;
        const bool ok = block >= 0 && block < p.num_blocks;
        const uint8_t* kbase = p.cache + (ok ? ((int64_t)block * p.heads + head) * page_bytes : 0);
        const uint32_t bytes = ok ? (uint32_t)page_bytes : 0u;
        return UnitPages{page_resource(kbase, bytes), page_resource(kbase + (ok ? p.plane_stride : 0), bytes),
                         (int)(u % UnitsPerPage) * kUnitTokens + t, ok};
    };
    auto load_plane = [&](__amdgpu_buffer_rsrc_t page, int tok, ChainRaw (&raw)[Links]) {
#pragma unroll
        for (int r = 0; r < Links; ++r)
            chain_load<PT, PagePolicy<D>::kCodes, PagePolicy<D>::kParams>(page, regs[r], tok, lq, r > 0, raw[r]);
    };
    // One plane's chain over the lane's channels [16 H, 16 H + 16): a plane is
    // built and consumed 16 channels at a time, so the chain's temporaries
    // take 32 registers, not 64.  `live` false zeroes a token past the
    // history (its scores are replaced by -inf, so the key plane needs no
    // such care).
    auto build_chain = [&](auto half, const ChainRaw (&raw)[Links], bool key_plane, bool live, float (&x)[16]) {
        constexpr int H = decltype(half)::value;
        chain_build<H, Links>(
            raw, regs, key_plane && has_mean,
            [&](int r, int i) __attribute__((always_inline)) { return mean_lds[r][32 * lq + 16 * H + i]; }, live,
            pick_lo, pick_hi, x);
    };
    using Half0 = std::integral_constant<int, 0>;
    using Half1 = std::integral_constant<int, 1>;

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
    float m = -INFINITY, l = 0.f;

    // Software pipeline over a wave's units: a plane's raw registers take the
    // next unit's bytes as soon as this unit's chain of that plane is built,
    // so the loads overlap the rest of the unit (the other plane's chain, the
    // softmax and the accumulation).
    int64_t u = range.unit_begin + wave;
    UnitPages pages = unit_pages(u);
    load_plane(pages.k, pages.tok, rk);
    load_plane(pages.v, pages.tok, rv);
    for (; u < range.unit_end; u += kWaves) {
        const int64_t pos = u * kUnitTokens + t;
        const bool valid = pages.ok && lane_active && pos < range.history;
        const UnitPages next = unit_pages(u + kWaves);
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        auto score_half = [&](auto half, const float (&x)[16]) {
            constexpr int H = decltype(half)::value;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 hi = qhi4[2 * H + i], lo = qlo4[2 * H + i];
                const uint32_t h[4] = {hi.x, hi.y, hi.z, hi.w}, l[4] = {lo.x, lo.y, lo.z, lo.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t k = bf16_pack(x[8 * i + 2 * j], x[8 * i + 2 * j + 1]);
                    s[j] = bf16_dot2(k, h[j], s[j]);
                    s[j] = bf16_dot2(k, l[j], s[j]);
                }
            }
        };
        {
            float x[16];
            build_chain(Half0{}, rk, true, true, x);
            score_half(Half0{}, x);
            build_chain(Half1{}, rk, true, true, x);
            score_half(Half1{}, x);
        }
        load_plane(next.k, next.tok, rk);
        float score = quad_sum_fast(lane_active ? (s[0] + s[1]) + (s[2] + s[3]) : 0.f);
        score = valid ? score : -INFINITY;
        const float unit_max = wave_max(score);
        if (unit_max > m) {
            const float factor = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - unit_max);
#pragma unroll
            for (int i = 0; i < 32; ++i) acc[i] *= factor;
            l *= factor;
            m = unit_max;
        }
        const float prob = valid ? __builtin_amdgcn_exp2f(score - m) : 0.f;
        l += prob;
        auto accumulate_half = [&](auto half, const float (&x)[16]) {
            constexpr int H = decltype(half)::value;
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const uint32_t v = bf16_pack(x[i], x[i + 1]);
                acc[16 * H + i] = fmaf(prob, __uint_as_float(v << 16), acc[16 * H + i]);
                acc[16 * H + i + 1] = fmaf(prob, __uint_as_float(v & 0xffff0000u), acc[16 * H + i + 1]);
            }
        };
        {
            float x[16];
            build_chain(Half0{}, rv, false, valid, x);
            accumulate_half(Half0{}, x);
            build_chain(Half1{}, rv, false, valid, x);
            accumulate_half(Half1{}, x);
        }
        load_plane(next.v, next.tok, rv);
        pages = next;
    }

    if (p.splits == 1) {
        finish_single<D>(p, row, head, prep_lds[1],
                         [&] { return merge_waves<D>(acc, m, l, lane, wave, lane_active, scratch_lds); });
    } else {
        write_partial<D>(merge_waves<D>(acc, m, l, lane, wave, lane_active, scratch_lds), partial);
        finish_split<D>(p, row, head);
    }
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

    const SplitRange range = split_range(p, p.row_request[row], split);
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
            // A token past the history may hold any bytes: its values count as 0.
            const uint32_t w[4] = {valid ? vv[i].x : 0u, valid ? vv[i].y : 0u, valid ? vv[i].z : 0u,
                                   valid ? vv[i].w : 0u};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[8 * i + 2 * j] = fmaf(prob, __uint_as_float(w[j] << 16), acc[8 * i + 2 * j]);
                acc[8 * i + 2 * j + 1] = fmaf(prob, __uint_as_float(w[j] & 0xffff0000u), acc[8 * i + 2 * j + 1]);
            }
        }
    }
    __shared__ __attribute__((aligned(16))) float scratch_lds[kWaves * 16 * 128];
    write_partial<D>(merge_waves<D>(acc, m, l, lane, wave, lane_active, scratch_lds), partial);
}

// ------------------------------------------------------------------ launch

// The launch parameters with stream_priority set: whether `blocks`
// workgroups of `kernel` fit the device at once.
inline AttentionParams with_priority(const AttentionParams& params, int per_cu, int64_t blocks) {
    AttentionParams p = params;
    p.stream_priority = blocks <= (int64_t)per_cu * p.compute_units ? 1 : 0;
    return p;
}

template <int D, int PT, int BA, int GA, int BL, int GL, bool HasL>
void launch_decode(const AttentionParams& p, hipStream_t stream) {
    const unsigned blocks = (unsigned)(p.rows * p.heads * p.splits);
    if constexpr (D == 96) {
        // Per-lane page offsets are 32-bit buffer offsets into one plane.
        if (p.plane_stride > 0 && p.plane_stride <= (int64_t)UINT32_MAX - 0x10000) {
            const auto kernel = decode96_dma_kernel<PT, BA, GA, BL, GL, HasL>;
            static const int per_cu = resident_per_cu(reinterpret_cast<const void*>(kernel), kDecodeThreads);
            hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kDecodeThreads), 0, stream, with_priority(p, per_cu, blocks));
            return;
        }
    }
    const auto kernel = decode_kernel<D, PT, BA, GA, BL, GL, HasL>;
    static const int per_cu = resident_per_cu(reinterpret_cast<const void*>(kernel), kDecodeThreads);
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kDecodeThreads), 0, stream, with_priority(p, per_cu, blocks));
}

template <int D, int PT, int BA, int GA>
bool dispatch_residual(const AttentionParams& p, hipStream_t stream) {
    if (!p.has_residual) {
        launch_decode<D, PT, BA, GA, 2, 32, false>(p, stream);
        return true;
    }
    const int bits = p.residual.bits, group = p.residual.group;
    if (bits == 2 && group == 32) launch_decode<D, PT, BA, GA, 2, 32, true>(p, stream);
    else if (bits == 2 && group == 16) launch_decode<D, PT, BA, GA, 2, 16, true>(p, stream);
    else if (bits == 4 && group == 32) launch_decode<D, PT, BA, GA, 4, 32, true>(p, stream);
    else if (bits == 4 && group == 16) launch_decode<D, PT, BA, GA, 4, 16, true>(p, stream);
    else return false;
    return true;
}

template <int D, int PT>
bool dispatch_anchor_pt(const AttentionParams& p, hipStream_t stream) {
    const int bits = p.anchor.bits, group = p.anchor.group;
    if (bits == 4 && group == 32) return dispatch_residual<D, PT, 4, 32>(p, stream);
    if (bits == 4 && group == 16) return dispatch_residual<D, PT, 4, 16>(p, stream);
    if (bits == 2 && group == 32) return dispatch_residual<D, PT, 2, 32>(p, stream);
    if (bits == 2 && group == 16) return dispatch_residual<D, PT, 2, 16>(p, stream);
    return false;
}

template <int D>
bool dispatch_anchor(const AttentionParams& p, hipStream_t stream) {
    if (p.page_tokens == 16) return dispatch_anchor_pt<D, 16>(p, stream);
    if (p.page_tokens == 32) return dispatch_anchor_pt<D, 32>(p, stream);
    return false;
}

template <int D, int PT, int Links>
void launch_chain_links(const AttentionParams& p, hipStream_t stream) {
    const unsigned blocks = (unsigned)(p.rows * p.heads * p.splits);
    const auto kernel = decode_chain_kernel<D, PT, Links>;
    static const int per_cu = resident_per_cu(reinterpret_cast<const void*>(kernel), kDecodeThreads);
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kDecodeThreads), 0, stream, with_priority(p, per_cu, blocks));
}

template <int D, int PT>
bool launch_chain_pt(const AttentionParams& p, hipStream_t stream) {
    switch (p.chain_length) {
        case 2: launch_chain_links<D, PT, 2>(p, stream); return true;
        case 3: launch_chain_links<D, PT, 3>(p, stream); return true;
        case 4: launch_chain_links<D, PT, 4>(p, stream); return true;
        default: return false;
    }
}

template <int D>
bool launch_chain(const AttentionParams& p, hipStream_t stream) {
    if (p.page_tokens == 16) return launch_chain_pt<D, 16>(p, stream);
    if (p.page_tokens == 32) return launch_chain_pt<D, 32>(p, stream);
    return false;
}

template <int D>
hipError_t launch_all(const AttentionParams& p, hipStream_t stream, hipEvent_t begin, hipEvent_t end,
                      bool bf16) {
    // The timed window holds every launch of the call.
    if (begin) (void)hipEventRecord(begin, stream);
    if (bf16 || !p.fused_prepare)
        hipLaunchKernelGGL((prepare_kernel<D>), dim3((unsigned)p.rows, (unsigned)p.heads), dim3(128), 0,
                           stream, p);
    if (bf16) {
        const unsigned blocks = (unsigned)(p.rows * p.heads * p.splits);
        hipLaunchKernelGGL((decode_bf16_kernel<D>), dim3(blocks), dim3(kDecodeThreads), 0, stream, p);
    } else if (p.chain_length > 1) {
        if (!launch_chain<D>(p, stream)) return hipErrorInvalidValue;
    } else if (!dispatch_anchor<D>(p, stream)) {
        return hipErrorInvalidValue;
    }
    if (bf16)
        hipLaunchKernelGGL((merge_kernel<D>), dim3((unsigned)p.rows, (unsigned)p.heads), dim3(kMergeThreads), 0,
                           stream, p);
    if (end) (void)hipEventRecord(end, stream);
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
