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
// k-ascending FP32 rotation, per-lane fmaf chains plus the 16,8,4,2,1 xor
// butterfly for the LS sums, IEEE division/sqrt, RNE satfinite FP8, single
// rounded BF16 restores.  Contraction is disabled for this file.
//
// Work mapping: one workgroup = 8 tokens x 1 head x 1 plane, 256 threads.
// Each 32-lane half-wave owns one token; lane l owns channels 4l..4l+3 of
// every record, so the coefficient butterfly and the group min/max stay inside
// the half-wave and the rotated rows never leave registers.
#include "rq_device.h"
#include "rq_kernels.h"

#pragma clang fp contract(off)

namespace rq {

namespace {

constexpr int kTileTokens = 8;
constexpr int kQuantizeThreads = 256;

__device__ __forceinline__ float shfl_xor32(float v, int mask) { return __shfl_xor(v, mask, 32); }

// Commit one record of one token (kernel.cuh:33-228).  All 32 lanes of the
// half-wave call this together; `store` masks the global writes only.
template <int D>
__device__ __forceinline__ void commit_record(const float (&y)[4], bool is_anchor, bool restore,
                                              int coefficient, const float (&mean)[4],
                                              bool has_mean, uint32_t (&reference)[4],
                                              const RecordRegion& region, uint8_t* page,
                                              int token, int page_tokens, int lane, bool store) {
    const bool active = lane * 4 < D;
    float previous[4] = {0.f, 0.f, 0.f, 0.f};
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = active ? y[i] : 0.f;
        if (!is_anchor && active) previous[i] = bf16_f32(reference[i]);
    }

    float alpha = 1.0f;
    if (!is_anchor && coefficient != RQ_COEF_UNIT_) {
        float numerator = 0.f, denominator = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            numerator = coefficient == RQ_COEF_NORM_ ? fmaf(x[i], x[i], numerator)
                                                     : fmaf(x[i], previous[i], numerator);
            denominator = fmaf(previous[i], previous[i], denominator);
        }
#pragma unroll
        for (int distance = 16; distance; distance >>= 1) {
            numerator += shfl_xor32(numerator, distance);
            denominator += shfl_xor32(denominator, distance);
        }
        if (coefficient == RQ_COEF_NORM_)
            alpha = denominator > 0.f ? sqrtf(numerator) / fmaxf(sqrtf(denominator), 1e-6f) : 0.f;
        else
            alpha = numerator / fmaxf(denominator, 1e-12f);
    }
    const uint32_t stored_alpha = bf16_rn(alpha);
    alpha = bf16_f32(stored_alpha);

    float low = __uint_as_float(0x7f800000u), high = __uint_as_float(0xff800000u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (!is_anchor) x[i] = fmaf(-previous[i], alpha, x[i]);
        if (has_mean) x[i] = x[i] - mean[i];
        if (active) {
            low = min_z(low, x[i]);
            high = max_z(high, x[i]);
        }
    }
    // A group spans 4 lanes (G16) or 8 lanes (G32).
    if (region.group == 32) {
        low = min_z(low, shfl_xor32(low, 4));
        high = max_z(high, shfl_xor32(high, 4));
    }
    low = min_z(low, shfl_xor32(low, 2));
    high = max_z(high, shfl_xor32(high, 2));
    low = min_z(low, shfl_xor32(low, 1));
    high = max_z(high, shfl_xor32(high, 1));

    const int bits = region.bits;
    const float center = (low + high) * 0.5f;
    const float radius = bits == 2 ? ((high - low) * 0.9f) * 0.5f : (high - low) * 0.5f;
    const float levels = bits == 2 ? 3.0f : 15.0f;
    const uint32_t offset_code = e4m3_rn(center - radius);
    const uint32_t scale_code = e4m3_rn((2.0f * radius) / levels);
    const float scale = e4m3_f32(scale_code);
    const float offset = e4m3_f32(offset_code);

    uint32_t packed = 0;
    uint32_t codes[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t code = 0;
        if (scale > 0.f) {
            const float normalized = (x[i] - offset) / scale;
            const float lower = floorf(normalized);
            float rounded = lower + ((normalized - lower) > 0.5f ? 1.0f : 0.0f);
            rounded = fminf(fmaxf(rounded, 0.0f), levels);
            code = (uint32_t)rounded;
        }
        codes[i] = code;
        packed |= code << (i * bits);
    }

    if (restore) {
        float mean_bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) mean_bf[i] = bf16_f32(bf16_rn(mean[i]));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t value = bf16_fma_rn((float)codes[i], scale, offset);
            if (has_mean) value = bf16_add_rn(bf16_f32(value), mean_bf[i]);
            if (!is_anchor) value = bf16_fma_rn(bf16_f32(reference[i]), alpha, bf16_f32(value));
            reference[i] = value;
        }
    }

    if (store && active) {
        uint8_t* record = page + region.offset;
        uint8_t* token_codes = record + (int64_t)token * region.code_bytes;
        if (bits == 2) {
            token_codes[lane] = (uint8_t)packed;
        } else {
            *reinterpret_cast<uint16_t*>(token_codes + 2 * lane) = (uint16_t)packed;
        }
        const int lanes_per_group = region.group / 4;
        if (lane % lanes_per_group == 0) {
            uint8_t* parameters = record + (int64_t)page_tokens * region.code_bytes;
            const int index = token * region.groups + lane / lanes_per_group;
            parameters[index] = (uint8_t)scale_code;
            parameters[page_tokens * region.groups + index] = (uint8_t)offset_code;
        }
        if (lane == 0) {
            uint8_t* target = record + (int64_t)page_tokens * (region.code_bytes + 2 * region.groups) +
                              2 * token;
            *reinterpret_cast<uint16_t*>(target) = (uint16_t)stored_alpha;
        }
    }
}

template <int D, int R, int A>
__global__ __launch_bounds__(kQuantizeThreads) void quantize_kernel(QuantizeParams p) {
    // Rotation kept as FP16 in LDS (converted by v_fma_mix on use) plus the
    // tile's inputs transposed to [token][channel][record] FP32.
    __shared__ _Float16 rotation_lds[D * D];
    __shared__ float input_lds[kTileTokens * D * R];

    const int plane = blockIdx.z;
    const int head = blockIdx.y;
    const int half = threadIdx.x >> 5;
    const int lane = threadIdx.x & 31;
    const int64_t first = (int64_t)blockIdx.x * kTileTokens;
    const int64_t n = first + half;

    int64_t slot = -1;
    if (n < p.tokens) slot = p.slots[n];
    const bool valid = slot >= 0 && slot / p.page_tokens < p.num_blocks;

    const uint16_t* rotation = plane == 0 ? p.key_rotation : p.value_rotation;
    float y[R][4];

    if (rotation != nullptr) {
        const uint16_t* matrix = rotation + (int64_t)head * D * D;
        for (int i = threadIdx.x; i < D * D; i += kQuantizeThreads)
            rotation_lds[i] = __builtin_bit_cast(_Float16, matrix[i]);
        for (int i = threadIdx.x; i < kTileTokens * R * D; i += kQuantizeThreads) {
            const int t = i / (R * D);
            const int r = (i / D) % R;
            const int k = i % D;
            const int64_t nn = first + t;
            float v = 0.f;
            if (nn < p.tokens) {
                const int64_t s = p.slots[nn];
                if (s >= 0 && s / p.page_tokens < p.num_blocks) {
                    const uint16_t* src = plane == 0 ? p.key_ptrs[r] + nn * p.key_strides[r]
                                                     : p.value_ptrs[r] + nn * p.value_strides[r];
                    v = bf16_f32(src[head * D + k]);
                }
            }
            input_lds[(t * D + k) * R + r] = v;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[r][i] = 0.f;
        if (lane * 4 < D) {
            const float* row_inputs = input_lds + half * D * R;
            for (int k = 0; k < D; ++k) {
                const _Float16* rk = rotation_lds + k * D + lane * 4;
                float rv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) rv[i] = (float)rk[i];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float xv = row_inputs[k * R + r];
#pragma unroll
                    for (int i = 0; i < 4; ++i) y[r][i] = fmaf(xv, rv[i], y[r][i]);
                }
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint16_t* src = nullptr;
            if (valid)
                src = (plane == 0 ? p.key_ptrs[r] + n * p.key_strides[r]
                                  : p.value_ptrs[r] + n * p.value_strides[r]) +
                      head * D;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = lane * 4 + i;
                y[r][i] = (valid && c < D) ? bf16_f32(src[c]) : 0.f;
            }
        }
    }

    uint8_t* page = nullptr;
    int token = 0;
    if (valid) {
        const int64_t block = slot / p.page_tokens;
        token = (int)(slot % p.page_tokens);
        page = p.cache + plane * p.plane_stride +
               (block * p.heads + head) * (int64_t)p.page_tokens * p.page_width;
    }

    uint32_t reference[4] = {0u, 0u, 0u, 0u};
    const bool has_mean = plane == 0 && p.key_mean != nullptr;
    // Anchor first, then every other record ascending (kernel.cuh:321-329).
#pragma unroll
    for (int step = 0; step < R; ++step) {
        const int r = step == 0 ? A : (step - 1 < A ? step - 1 : step);
        float mean[4] = {0.f, 0.f, 0.f, 0.f};
        if (has_mean) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = lane * 4 + i;
                if (c < D) mean[i] = p.key_mean[((int64_t)r * p.heads + head) * D + c];
            }
        }
        const bool is_anchor = r == A;
        commit_record<D>(y[r], is_anchor, is_anchor || p.adjacent, p.coefficient, mean, has_mean,
                         reference, p.region[r], page, token, p.page_tokens, lane, valid);
    }
}

template <int D, int R, int A>
hipError_t launch_quantize_kernel(const QuantizeParams& p, hipStream_t stream) {
    const dim3 grid((unsigned)((p.tokens + kTileTokens - 1) / kTileTokens), (unsigned)p.heads, 2);
    hipLaunchKernelGGL((quantize_kernel<D, R, A>), grid, dim3(kQuantizeThreads), 0, stream, p);
    return hipGetLastError();
}

template <int D, int R>
hipError_t dispatch_anchor(const QuantizeParams& p, int anchor, hipStream_t stream) {
    switch (anchor) {
        case 0: return launch_quantize_kernel<D, R, 0>(p, stream);
        case 1: if constexpr (R > 1) return launch_quantize_kernel<D, R, 1>(p, stream); break;
        case 2: if constexpr (R > 2) return launch_quantize_kernel<D, R, 2>(p, stream); break;
        case 3: if constexpr (R > 3) return launch_quantize_kernel<D, R, 3>(p, stream); break;
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
