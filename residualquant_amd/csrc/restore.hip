// Restore of packed records to BF16 (gfx950): the reference's record
// reconstruction (plugins/residual_quantization/csrc/quantize/kernel.cuh:160-203,
// attention/compute.cuh:28-197), evaluated per channel with single-rounded
// BF16 steps:  X_base = bf16(code*scale + offset) [+ bf16(mu) on K], then
// X_r = bf16(alpha_r * X_prev + X_r) along the chain.  Bit-exact with the
// oracle; contraction disabled.
#include "rq_device.h"
#include "rq_kernels.h"

#pragma clang fp contract(off)

namespace rq {

namespace {

__global__ __launch_bounds__(128) void restore_kernel(RestoreParams p) {
    const int64_t n = blockIdx.x;
    const int head = blockIdx.y;
    const int c = threadIdx.x;
    if (c >= p.head_dim) return;
    const int64_t out_index = (n * p.heads + head) * p.head_dim + c;
    const int64_t slot = p.slots[n];
    if (slot < 0 || slot / p.page_tokens >= p.num_blocks) {
        p.key_out[out_index] = 0;
        p.value_out[out_index] = 0;
        return;
    }
    const int64_t block = slot / p.page_tokens;
    const int token = (int)(slot % p.page_tokens);
    for (int plane = 0; plane < 2; ++plane) {
        const uint8_t* page = p.cache + plane * p.plane_stride +
                              (block * p.heads + head) * (int64_t)p.page_tokens * p.page_width;
        uint32_t value = 0;
        for (int i = 0; i < p.chain_length; ++i) {
            const int r = p.chain[i];
            const RecordRegion& region = p.region[r];
            const uint8_t* record = page + region.offset;
            const uint8_t* codes = record + (int64_t)token * region.code_bytes;
            const uint32_t code =
                (codes[(c * region.bits) >> 3] >> ((c * region.bits) & 7)) & ((1u << region.bits) - 1u);
            const uint8_t* scales = record + (int64_t)p.page_tokens * region.code_bytes;
            const int g = c / region.group;
            const float scale = e4m3_f32(scales[token * region.groups + g]);
            const float offset = e4m3_f32(scales[p.page_tokens * region.groups + token * region.groups + g]);
            uint32_t v = bf16_fma_rn((float)code, scale, offset);
            if (plane == 0 && p.key_mean != nullptr) {
                const float mean = p.key_mean[((int64_t)r * p.heads + head) * p.head_dim + c];
                v = bf16_add_rn(bf16_f32(v), bf16_f32(bf16_rn(mean)));
            }
            if (i > 0) {
                const uint8_t* a = record + (int64_t)p.page_tokens * (region.code_bytes + 2 * region.groups) +
                                   2 * token;
                const uint32_t alpha = (uint32_t)a[0] | ((uint32_t)a[1] << 8);
                v = bf16_fma_rn(bf16_f32(value), bf16_f32(alpha), bf16_f32(v));
            }
            value = v;
        }
        (plane == 0 ? p.key_out : p.value_out)[out_index] = (uint16_t)value;
    }
}

}  // namespace

hipError_t launch_restore(const RestoreParams& p, hipStream_t stream) {
    if (p.tokens == 0) return hipSuccess;
    hipLaunchKernelGGL(restore_kernel, dim3((unsigned)p.tokens, (unsigned)p.heads), dim3(128), 0, stream, p);
    return hipGetLastError();
}

}  // namespace rq
