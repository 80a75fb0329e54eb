// Adjacent-mode restore chain on the device, shared by the per-row chain
// decode kernel (attention.hip) and the multi-row kernels (multirow.hip).
//
// In adjacent mode every loop is a residual of the previous loop
// (compute.cuh:120-197, :506-528): X_0 = bf16(c s + o), X_r = bf16(alpha_r
// X_{r-1} + bf16(c s + o)), the K plane adding bf16(mu_r) to each record's
// value except the current loop's (the live score carries -q'.mu_L).  Each
// chain step is
//   X_r = dot2(pack(X_{r-1}, k_r), (alpha_r, 1)),
// one v_cvt_pk_bf16_f32 that rounds the previous link and the record's value
// to BF16 (RNE) and one v_dot2_f32_bf16 that forms alpha X + k in FP32; the
// BF16 rounding of X_r happens where it is next packed.  The reference rounds
// the exact value once; the FP32 sum of the dot (which may differ from an FMA
// by one FP32 ulp in the last place) is rounded again to BF16, and the two
// differ only when that sum sits within an FP32 ulp of a BF16 midpoint
// (within the attention tolerance).
//
// A lane holds 32 channels [32 lq, 32 lq + 32) of one token (lane = token x
// 32-channel quarter) and builds them 16 at a time (H = 0, 1).
#pragma once

#include "rq_device.h"

namespace rq {

// FP8 E4M3 byte `sel` of v to FP32.  gfx950 converts OCP E4M3 in hardware.
template <int Sel>
__device__ __forceinline__ float fp8_f32(uint32_t v) {
    return __builtin_amdgcn_cvt_f32_fp8((int)v, Sel);
}

typedef __bf16 ChainBf16x2 __attribute__((ext_vector_type(2)));
typedef float ChainF32x2 __attribute__((ext_vector_type(2)));

// RNE to BF16 of two FP32 values, packed (lo = a, hi = b): v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16_pack(float a, float b) {
    const ChainF32x2 f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, ChainBf16x2));
}
// a.lo * b.lo + a.hi * b.hi + c over BF16 pairs, FP32 sum: v_dot2_f32_bf16.
// Keep constant pairs for `b` in registers: the compiler may encode a packed
// BF16 constant as an FP32 inline constant, which the instruction reads as
// the pair (0, hi 16 bits of the FP32 value).
__device__ __forceinline__ float bf16_dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ChainBf16x2, a), __builtin_bit_cast(ChainBf16x2, b), c,
                                           false);
}
// a.lo * b.lo + a.hi * b.hi with no addend, as the three-operand VOP3P form:
// through the builtin the compiler picks the two-operand v_dot2c_f32_bf16,
// whose accumulator is its destination, and spends a v_mov of 0 on each.
__device__ __forceinline__ float bf16_dot2_zero(uint32_t a, uint32_t b) {
    float r;
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// The raw bytes of one record of one token that a lane needs for its 32
// channels [32 lq, 32 lq + 32): code words (16 bytes INT4, 8 bytes INT2), the
// FP8 scale and offset of its groups (one byte each for G32, two for G16) and
// the BF16 alpha.  Loading every record of a unit before decoding any lets all
// of their round trips overlap.
struct ChainRaw {
    uint4 codes;
    uint32_t params;  // FP8 scale byte(s) in the low 16 bits, offset byte(s) in the high 16
    uint32_t alpha;
};

// Loads one record's bytes of token `tok` of a page (buffer resource `page`);
// CodesPolicy / ParamsPolicy are the cache-policy operands of the code words
// and of the FP8 parameter and alpha bytes.
template <int PT, int CodesPolicy, int ParamsPolicy>
__device__ __forceinline__ void chain_load(__amdgpu_buffer_rsrc_t page, const RecordRegion& reg, int tok, int lq,
                                           bool with_alpha, ChainRaw& raw) {
    const uint32_t params = reg.offset + PT * reg.code_bytes + tok * reg.groups;
    uint32_t scale, offset;
    if (reg.group == 32) {
        scale = __builtin_amdgcn_raw_buffer_load_b8(page, params + lq, 0, ParamsPolicy);
        offset = __builtin_amdgcn_raw_buffer_load_b8(page, params + PT * reg.groups + lq, 0, ParamsPolicy);
    } else {
        scale = __builtin_amdgcn_raw_buffer_load_b16(page, params + 2 * lq, 0, ParamsPolicy);
        offset = __builtin_amdgcn_raw_buffer_load_b16(page, params + PT * reg.groups + 2 * lq, 0, ParamsPolicy);
    }
    raw.params = scale | (offset << 16);
    const uint32_t codes = reg.offset + tok * reg.code_bytes;
    if (reg.bits == 4) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(page, codes + 16 * lq, 0, CodesPolicy);
        raw.codes = make_uint4(v[0], v[1], v[2], v[3]);
    } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(page, codes + 8 * lq, 0, CodesPolicy);
        raw.codes = make_uint4(v[0], v[1], 0u, 0u);
    }
    raw.alpha = with_alpha ? __builtin_amdgcn_raw_buffer_load_b16(
                                 page, reg.offset + PT * (reg.code_bytes + 2 * reg.groups) + 2 * tok, 0, ParamsPolicy)
                           : 0u;
}

// FP32 code * scale + offset of channels [16 H, 16 H + 16) of the lane's 32
// channels of one record, before the BF16 rounding (which happens where the
// value is packed).
template <int H>
__device__ __forceinline__ void chain_decode(const ChainRaw& raw, const RecordRegion& reg, float (&out)[16]) {
    float scale, offset;
    if (reg.group == 32) {
        scale = fp8_f32<0>(raw.params) * 512.0f;
        offset = fp8_f32<2>(raw.params);
    } else {
        scale = fp8_f32<H>(raw.params) * 512.0f;
        offset = fp8_f32<2 + H>(raw.params);
    }
    // A code c held in a byte is the FP8 E4M3 value c * 2^-9 (scale carries 2^9).
    const uint32_t w[4] = {raw.codes.x, raw.codes.y, raw.codes.z, raw.codes.w};
    if (reg.bits == 4) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t word = w[2 * H + i];
            const int lo = (int)(word & 0x0f0f0f0fu), hi = (int)((word >> 4) & 0x0f0f0f0fu);
            const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
            const auto l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            const float c[8] = {l01[0], h01[0], l01[1], h01[1], l23[0], h23[0], l23[1], h23[1]};
#pragma unroll
            for (int k = 0; k < 8; ++k) out[8 * i + k] = fmaf(c[k], scale, offset);
        }
    } else {
        // Byte j of part k holds channel 4j + k.  The channels are written in
        // index order, as in the INT4 branch: stores to different elements in
        // the two branches get merged through a pointer, which keeps `out` in
        // scratch memory.
        float c[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int part = (int)((w[H] >> (2 * k)) & 0x03030303u);
            const auto c01 = __builtin_amdgcn_cvt_pk_f32_fp8(part, false);
            const auto c23 = __builtin_amdgcn_cvt_pk_f32_fp8(part, true);
            c[0][k] = c01[0];
            c[1][k] = c01[1];
            c[2][k] = c23[0];
            c[3][k] = c23[1];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) out[4 * j + k] = fmaf(c[j][k], scale, offset);
    }
}

// The chain X_0 = bf16(c s + o), X_r = bf16(alpha_r X_{r-1} + bf16(c s + o))
// of one plane over the lane's channels [16 H, 16 H + 16), the K plane
// (`add_mean`) adding bf16(mu_r) to every record but the last (k =
// bf16(bf16(c s + o) + bf16(mu_r)): one pack per channel pair and a dot with
// (1, 0) or (0, 1) whose FP32 addend is bf16(mu_r)).  mean_at(r, i) returns
// bf16(mu_r) (FP32) of the half's channel i.  x holds the last link before
// its BF16 rounding.
// `live` false: a token past the history, whose slot may hold any bytes; its
// FP8 parameters and alphas count as zero, so its values are zero.  pick_lo
// and pick_hi are the BF16 pairs (1, 0) and (0, 1), kept in registers.
// Plain `inline`, not always_inline: inlined after its own optimization, it
// takes 200 registers in the per-row chain kernel at four records, against
// 224 when inlined first (loop 3 at B32 x 8k: 641 against 662 us).
template <int H, int Links, class MeanAt>
__device__ inline void chain_build(const ChainRaw (&raw)[Links], const RecordRegion (&regs)[Links],
                                            bool add_mean, MeanAt mean_at, bool live, uint32_t pick_lo,
                                            uint32_t pick_hi, float (&x)[16]) {
#pragma unroll
    for (int r = 0; r < Links; ++r) {
        // One record at a time: interleaved by the scheduler, the records'
        // temporaries would raise the register count.
        __builtin_amdgcn_sched_barrier(0);
        ChainRaw record = raw[r];
        record.params = live ? record.params : 0u;
        record.alpha = live ? record.alpha : 0u;
        float xr[16];
        chain_decode<H>(record, regs[r], xr);
        if (add_mean && r + 1 < Links) {
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const uint32_t pair = bf16_pack(xr[i], xr[i + 1]);
                xr[i] = bf16_dot2(pair, pick_lo, mean_at(r, i));
                xr[i + 1] = bf16_dot2(pair, pick_hi, mean_at(r, i + 1));
            }
        }
        if (r == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = xr[i];
        } else {
            const uint32_t weights = (record.alpha & 0xffffu) | 0x3f800000u;  // (alpha_r, 1)
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = bf16_dot2_zero(bf16_pack(x[i], xr[i]), weights);
        }
    }
}

}  // namespace rq
