// Fused elementwise kernels of the looped-model decode step (the callers on
// either side of the packed attention in one Ouro layer,
// plugins/looped_transformers/src/looped_transformers/ouro.py:102-146):
// residual add + RMSNorm, rotary embedding of Q/K with the K/V staging copy,
// and SiLU(gate) * up.  One launch each instead of a dozen elementwise ops.
#include "rq_device.h"
#include "rq_kernels.h"

namespace rq {

namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int distance = 32; distance; distance >>= 1) v += __shfl_xor(v, distance);
    return v;
}

// Sum of one float per thread over the 256-thread workgroup (`partial` holds
// one float per wave; the trailing barrier lets the caller reuse it).
__device__ __forceinline__ float block_sum(float v, float* partial) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = v;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) total += partial[w];
    __syncthreads();
    return total;
}

// values[e] = bf16(bf16(values[e] * rsqrt(mean(values^2) + eps)) * w[e]) over the row.
__device__ __forceinline__ void normalize_row(float (&values)[8], const uint16_t* weight, int i, bool active,
                                              int hidden, float eps, float* partial) {
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum = fmaf(values[e], values[e], sum);
    const float scale = rsqrtf(block_sum(sum, partial) / (float)hidden + eps);
    if (!active) return;
    const uint4 wraw = *reinterpret_cast<const uint4*>(weight + i);
    const uint32_t wv[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        values[2 * e] = bf16_f32(bf16_rn(bf16_f32(bf16_rn(values[2 * e] * scale)) * bf16_f32(wv[e] & 0xffffu)));
        values[2 * e + 1] =
            bf16_f32(bf16_rn(bf16_f32(bf16_rn(values[2 * e + 1] * scale)) * bf16_f32(wv[e] >> 16)));
    }
}

// One workgroup per row, 8 channels per thread (rows of at most 8 * 256
// channels, a multiple of 8).  Optionally x is first normalized with
// pre_weight (a norm whose output feeds a fused add, as input_layernorm_2
// feeds post_attention_layernorm, ouro.py:154-155); then, with a residual,
// total = bf16(x + residual) is written to residual_out and normalized:
// y = bf16(bf16(total * rsqrt(mean(total^2) + eps)) * weight).
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const uint16_t* x, int64_t x_stride,
                                                                const uint16_t* pre_weight,
                                                                const uint16_t* residual, int64_t residual_stride,
                                                                uint16_t* residual_out, int64_t residual_out_stride,
                                                                const uint16_t* weight, uint16_t* y, int64_t y_stride,
                                                                int hidden, float eps) {
    __shared__ float partial[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const int i = 8 * threadIdx.x;
    const bool active = i < hidden;
    float values[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    uint4 rres = make_uint4(0, 0, 0, 0);
    if (active) {
        const uint4 raw = *reinterpret_cast<const uint4*>(x + row * x_stride + i);
        if (residual != nullptr) rres = *reinterpret_cast<const uint4*>(residual + row * residual_stride + i);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            values[2 * e] = bf16_f32(w[e] & 0xffffu);
            values[2 * e + 1] = bf16_f32(w[e] >> 16);
        }
    }
    if (pre_weight != nullptr) normalize_row(values, pre_weight, i, active, hidden, eps, partial);
    if (residual != nullptr && active) {
        const uint32_t r[4] = {rres.x, rres.y, rres.z, rres.w};
        uint32_t packed[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = bf16_rn(values[2 * e] + bf16_f32(r[e] & 0xffffu));
            const uint32_t hi = bf16_rn(values[2 * e + 1] + bf16_f32(r[e] >> 16));
            values[2 * e] = bf16_f32(lo);
            values[2 * e + 1] = bf16_f32(hi);
            packed[e] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(residual_out + row * residual_out_stride + i) =
            make_uint4(packed[0], packed[1], packed[2], packed[3]);
    }
    normalize_row(values, weight, i, active, hidden, eps, partial);
    if (active) {
        uint32_t out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = bf16_rn(values[2 * e]) | (bf16_rn(values[2 * e + 1]) << 16);
        *reinterpret_cast<uint4*>(y + row * y_stride + i) = make_uint4(out[0], out[1], out[2], out[3]);
    }
}

// Rotary embedding (rotate-half form) of the Q and K heads of a fused QKV row,
// plus plain copies of K (rotated) and V into staging rows.  Grid (rows,
// 2 * heads): y < heads rotates Q head y, else K head y - heads (and copies V).
// Positions outside the cos/sin tables are clamped to them: the tables are
// read from device-resident positions that the host cannot check.
__global__ __launch_bounds__(64) void rope_kernel(const uint16_t* qkv, int64_t qkv_stride, const int64_t* positions,
                                                  const float* cos_table, const float* sin_table,
                                                  int64_t table_rows, int heads,
                                                  int head_dim, uint16_t* q_out, int64_t q_stride, uint16_t* k_out,
                                                  int64_t k_stride, uint16_t* k_stage, uint16_t* v_stage,
                                                  int64_t stage_stride) {
    const int64_t row = blockIdx.x;
    const int which = blockIdx.y;
    const bool is_key = which >= heads;
    const int head = is_key ? which - heads : which;
    const int half = head_dim / 2;
    const int64_t position = min(max(positions[row], (int64_t)0), table_rows - 1);
    const uint16_t* src = qkv + row * qkv_stride + (int64_t)(is_key ? heads + head : head) * head_dim;
    for (int i = threadIdx.x; i < half; i += 64) {
        const float c = cos_table[position * half + i], s = sin_table[position * half + i];
        const float x1 = bf16_f32(src[i]), x2 = bf16_f32(src[i + half]);
        const uint16_t a = (uint16_t)bf16_rn(x1 * c - x2 * s), b = (uint16_t)bf16_rn(x2 * c + x1 * s);
        if (!is_key) {
            q_out[row * q_stride + head * head_dim + i] = a;
            q_out[row * q_stride + head * head_dim + i + half] = b;
        } else {
            k_out[row * k_stride + head * head_dim + i] = a;
            k_out[row * k_stride + head * head_dim + i + half] = b;
            if (k_stage != nullptr) {
                k_stage[row * stage_stride + head * head_dim + i] = a;
                k_stage[row * stage_stride + head * head_dim + i + half] = b;
            }
        }
    }
    if (is_key && v_stage != nullptr) {
        const uint16_t* v = qkv + row * qkv_stride + (int64_t)(2 * heads + head) * head_dim;
        for (int i = threadIdx.x; i < head_dim; i += 64) v_stage[row * stage_stride + head * head_dim + i] = v[i];
    }
}

// act = bf16(silu(gate) * up) with gate/up the two halves of a [rows, 2 * width] row.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gate_up, int64_t gate_up_stride, uint16_t* out,
                                                       int64_t out_stride, int width) {
    const int64_t row = blockIdx.y;
    const int i = 2 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= width) return;
    const uint32_t g = *reinterpret_cast<const uint32_t*>(gate_up + row * gate_up_stride + i);
    const uint32_t u = *reinterpret_cast<const uint32_t*>(gate_up + row * gate_up_stride + width + i);
    const float g0 = bf16_f32(g & 0xffffu), g1 = bf16_f32(g >> 16);
    const float a = g0 / (1.0f + __expf(-g0)) * bf16_f32(u & 0xffffu);
    const float b = g1 / (1.0f + __expf(-g1)) * bf16_f32(u >> 16);
    *reinterpret_cast<uint32_t*>(out + row * out_stride + i) = bf16_rn(a) | (bf16_rn(b) << 16);
}


// y[m, n] = bf16(sum_k x[m, k] * w[n, k]) for a few rows m: the decode step's
// projections at small batch, where a GEMM is a weight stream.  One
// workgroup computes Cols output columns for every row.  Thread t takes the
// 16-byte chunks t, t + 256, ... of each weight row (one load instruction
// covers 4 KB of a row, so the weights are read once, non-temporal) and the
// same chunks of the x rows (kept in registers); FP32 partial sums meet in a
// wave reduction and then across the 4 waves through LDS.
constexpr int kLinearThreads = 256;

template <int M, int Cols, int Chunks>
__global__ __launch_bounds__(kLinearThreads) void linear_rows_kernel(const uint16_t* x, int64_t x_stride,
                                                                     const uint16_t* w, uint16_t* y, int64_t y_stride,
                                                                     int out_features, int in_features) {
    __shared__ float partial[kLinearThreads / 64][M * Cols];
    const int t = threadIdx.x;
    const int chunks = in_features / 8;
    const int n0 = blockIdx.x * Cols;
    const Chunk16 zero = {0u, 0u, 0u, 0u};
    Chunk16 wv[Cols][Chunks];
#pragma unroll
    for (int col = 0; col < Cols; ++col) {
        const bool row_ok = n0 + col < out_features;
        const Chunk16* row = reinterpret_cast<const Chunk16*>(w + (int64_t)(row_ok ? n0 + col : 0) * in_features);
#pragma unroll
        for (int j = 0; j < Chunks; ++j) {
            const int c = t + kLinearThreads * j;
            wv[col][j] = (row_ok && c < chunks) ? __builtin_nontemporal_load(row + c) : zero;
        }
    }
    Chunk16 xv[M][Chunks];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const Chunk16* row = reinterpret_cast<const Chunk16*>(x + m * x_stride);
#pragma unroll
        for (int j = 0; j < Chunks; ++j) {
            const int c = t + kLinearThreads * j;
            xv[m][j] = c < chunks ? row[c] : zero;
        }
    }
    // Each chunk's x values are widened once and shared by every column.
    float acc[M][Cols];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int col = 0; col < Cols; ++col) acc[m][col] = 0.f;
#pragma unroll
    for (int j = 0; j < Chunks; ++j) {
        float xf[M][8];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xf[m][2 * e] = __uint_as_float(xv[m][j][e] << 16);
                xf[m][2 * e + 1] = __uint_as_float(xv[m][j][e] & 0xffff0000u);
            }
#pragma unroll
        for (int col = 0; col < Cols; ++col) {
            float wf[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wf[2 * e] = __uint_as_float(wv[col][j][e] << 16);
                wf[2 * e + 1] = __uint_as_float(wv[col][j][e] & 0xffff0000u);
            }
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[m][col] = fmaf(wf[e], xf[m][e], acc[m][col]);
        }
    }
    // Reduce-scatter over the wave: each exchange at distance d halves the
    // values a lane keeps (lanes with bit d set keep the upper half and add
    // the partner's copy of it), so after log2(V) exchanges lane l holds the
    // wave total of value l / (64 / V), summed over the remaining lane bits.
    constexpr int V = M * Cols;
    static_assert(V <= 64, "at most 64 values per lane");
    float v[64];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int col = 0; col < Cols; ++col) v[m * Cols + col] = acc[m][col];
    constexpr int P = V <= 1 ? 1 : V <= 2 ? 2 : V <= 4 ? 4 : V <= 8 ? 8 : V <= 16 ? 16 : V <= 32 ? 32 : 64;
#pragma unroll
    for (int i = V; i < P; ++i) v[i] = 0.f;
    const int lane = t & 63;
    int n = P;
#pragma unroll
    for (int d = 32; d >= 64 / P; d >>= 1) {
        const bool upper = (lane & d) != 0;
        n >>= 1;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            if (i < n) {
                const float send = upper ? v[i] : v[i + n];
                const float keep = upper ? v[i + n] : v[i];
                v[i] = keep + __shfl_xor(send, d);
            }
        }
    }
    float total = v[0];
#pragma unroll
    for (int d = 64 / P / 2; d >= 1; d >>= 1) total += __shfl_xor(total, d);
    const int index = lane / (64 / P);
    if ((lane & (64 / P - 1)) == 0 && index < V) partial[t >> 6][index] = total;
    __syncthreads();
    if (t < M * Cols) {
        const int m = t / Cols, col = t % Cols;
        if (n0 + col < out_features) {
            float sum = 0.f;
#pragma unroll
            for (int wave = 0; wave < kLinearThreads / 64; ++wave) sum += partial[wave][t];
            y[m * y_stride + n0 + col] = (uint16_t)bf16_rn(sum);
        }
    }
}

}  // namespace

hipError_t launch_rms_norm(const StepNormParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)p.rows), dim3(kNormThreads), 0, stream, p.x, p.x_stride,
                       p.pre_weight, p.residual, p.residual_stride, p.residual_out, p.residual_out_stride, p.weight, p.y,
                       p.y_stride, p.hidden, p.eps);
    return hipGetLastError();
}

hipError_t launch_rope(const StepRopeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)p.rows, (unsigned)(2 * p.heads)), dim3(64), 0, stream, p.qkv,
                       p.qkv_stride, p.positions, p.cos_table, p.sin_table, p.table_rows, p.heads, p.head_dim, p.q, p.q_stride, p.k,
                       p.k_stride, p.k_stage, p.v_stage, p.stage_stride);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* gate_up, int64_t gate_up_stride, uint16_t* out, int64_t out_stride,
                           int64_t rows, int width, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((width / 2 + 255) / 256), (unsigned)rows), dim3(256), 0,
                       stream, gate_up, gate_up_stride, out, out_stride, width);
    return hipGetLastError();
}

hipError_t launch_linear_rows(const uint16_t* x, int64_t x_stride, const uint16_t* w, uint16_t* y, int64_t y_stride,
                              int rows, int out_features, int in_features, hipStream_t stream) {
    if (rows == 0 || out_features == 0) return hipSuccess;
    // Chunks per thread from in_features; columns per workgroup so that the
    // weight, x and accumulator registers stay near 128 per lane.
    const int chunks = (in_features / 8 + kLinearThreads - 1) / kLinearThreads;
    const int cols = chunks == 1 ? 8 : (chunks == 2 || rows <= 4 ? 4 : 2);
    const dim3 grid((unsigned)((out_features + cols - 1) / cols));
#define RQ_LINEAR_CASE(M)                                                                                         \
    case M:                                                                                                       \
        if (chunks == 1)                                                                                          \
            hipLaunchKernelGGL((linear_rows_kernel<M, 8, 1>), grid, dim3(kLinearThreads), 0, stream, x, x_stride, \
                               w, y, y_stride, out_features, in_features);                                        \
        else if (chunks == 2)                                                                                     \
            hipLaunchKernelGGL((linear_rows_kernel<M, 4, 2>), grid, dim3(kLinearThreads), 0, stream, x, x_stride, \
                               w, y, y_stride, out_features, in_features);                                        \
        else                                                                                                      \
            hipLaunchKernelGGL((linear_rows_kernel<M, (M <= 4 ? 4 : 2), 3>), grid, dim3(kLinearThreads), 0, stream, \
                               x, x_stride,                                                                       \
                               w, y, y_stride, out_features, in_features);                                        \
        break;
    switch (rows) {
        RQ_LINEAR_CASE(1)
        RQ_LINEAR_CASE(2)
        RQ_LINEAR_CASE(3)
        RQ_LINEAR_CASE(4)
        RQ_LINEAR_CASE(5)
        RQ_LINEAR_CASE(6)
        RQ_LINEAR_CASE(7)
        RQ_LINEAR_CASE(8)
        default:
            return hipErrorInvalidValue;
    }
#undef RQ_LINEAR_CASE
    return hipGetLastError();
}

}  // namespace rq
