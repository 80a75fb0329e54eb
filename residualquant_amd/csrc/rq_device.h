// Device-side scalar formats and packed-page layout helpers shared by the
// quantize, restore and attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rq {

// ------------------------------------------------------------------ BF16

// __float2bfloat16_rn semantics: one round-to-nearest-even of an FP32 value,
// a NaN kept with its upper payload bits and the quiet bit set.  gfx950's
// v_cvt_pk_bf16_f32 (under the default rounding and denormal modes these
// kernels run with) gives exactly the integer form
//   NaN ? (u >> 16) | 0x40 : (u + 0x7fff + ((u >> 16) & 1)) >> 16
// for all 2^32 FP32 inputs (checked on the device, both halves of the pair),
// in one instruction for two values instead of six per value.
typedef __bf16 Bf16Pair __attribute__((ext_vector_type(2)));
typedef float F32Pair __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t bf16_rn(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// bf16_rn of a and b packed (a in the low half): one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16x2_rn(float a, float b) {
    const F32Pair f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, Bf16Pair));
}

__device__ __forceinline__ float bf16_f32(uint32_t h) { return __uint_as_float(h << 16); }

// One RNE rounding to BF16 of s + err, where (s, err) is an exact TwoSum
// pair.  BF16 midpoints are FP32 values: only a sum that lands exactly on
// one of them needs the error term to decide the direction.
__device__ __forceinline__ uint32_t bf16_round_pair(float s, float err) {
    uint32_t u = __float_as_uint(s);
    if ((u & 0xffffu) == 0x8000u && err != 0.0f) {
        const bool away = (err > 0.0f) == (s > 0.0f);
        u = away ? u + 1u : u - 1u;
        s = __uint_as_float(u);
    }
    return bf16_rn(s);
}

// BF16(a*b + c) with a single rounding (the __hfma2 result).  a*b of two
// BF16 values is exact in FP32; TwoSum recovers the addition error.
__device__ __forceinline__ uint32_t bf16_fma_rn(float a, float b, float c) {
    const float p = a * b;
    const float s = p + c;
    const float bb = s - p;
    const float err = (p - (s - bb)) + (c - bb);
    return bf16_round_pair(s, err);
}

// BF16(a + b) with a single rounding (the __hadd2 result).
__device__ __forceinline__ uint32_t bf16_add_rn(float a, float b) {
    const float s = a + b;
    const float bb = s - a;
    const float err = (a - (s - bb)) + (b - bb);
    return bf16_round_pair(s, err);
}

// ------------------------------------------------------------------ FP8

// OCP E4M3 decode (bias 7, subnormals m*2^-9), exact in FP32.
__device__ __forceinline__ float e4m3_f32(uint32_t v) {
    const uint32_t e = (v >> 3) & 0xfu;
    const uint32_t m = v & 7u;
    float magnitude = e ? __uint_as_float(((e + 120u) << 23) | (m << 20))
                        : (float)m * 0.001953125f;
    if ((v & 0x7fu) == 0x7fu) magnitude = __uint_as_float(0x7fc00000u);
    return (v & 0x80u) ? -magnitude : magnitude;
}

// OCP E4M3 encode: round-to-nearest-even, saturating to +-448, keeping the
// sign of zero (the satfinite __nv_fp8_e4m3(float) conversion).
__device__ __forceinline__ uint32_t e4m3_rn(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 24) & 0x80u;
    const float a = fabsf(f);
    if (a != a) return sign | 0x7fu;
    if (a >= 448.0f) return sign | 0x7eu;
    if (a < 0.015625f) return sign | (uint32_t)rintf(a * 512.0f);
    const uint32_t ua = __float_as_uint(a);
    int exponent = (int)(ua >> 23) - 127;
    const uint32_t mantissa = ua & 0x7fffffu;
    uint32_t kept = mantissa >> 20;
    const uint32_t round_bit = (mantissa >> 19) & 1u;
    const uint32_t sticky = mantissa & 0x7ffffu;
    if (round_bit && (sticky || (kept & 1u))) kept++;
    if (kept == 8u) {
        kept = 0;
        exponent++;
    }
    uint32_t code = ((uint32_t)(exponent + 7) << 3) | kept;
    if (code > 0x7eu) code = 0x7eu;
    return sign | code;
}

// ------------------------------------------------------------------ order

// min/max with -0 ordered below +0 (commutative for every non-NaN pair).
__device__ __forceinline__ float min_z(float a, float b) {
    return (a < b || (a == b && __float_as_uint(a) >> 31)) ? a : b;
}
__device__ __forceinline__ float max_z(float a, float b) {
    return (a > b || (a == b && !(__float_as_uint(a) >> 31))) ? a : b;
}

// Sixteen bytes as four 32-bit words in one vector register group (a vector
// type, unlike HIP's uint4 struct, stays in registers inside structs and
// arrays).
typedef uint32_t Chunk16 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ cross-workgroup hand-off
//
// A workgroup that hands data to another workgroup of the same launch (the
// last-arriving split reads every split's partial) writes and reads it with
// buffer stores and loads carrying the sc1 cache policy, which are coherent
// across the XCDs' L2 caches (what agent-scope atomic loads and stores
// compile to on gfx950), instead of an agent-scope fence (__threadfence: a
// whole-L2 write-back and invalidate per workgroup).  Plain buffer
// operations, unlike atomics, let the compiler keep many loads in flight.
// The writer waits for its stores to be acknowledged (vmcnt counts stores on
// gfx9) before the workgroup barrier and the arrival atomic; the reader
// issues its loads after observing the final arrival.

constexpr int kCoherentPolicy = 16;  // cache-policy operand: sc1

// Cache-policy operand nt (non-temporal) for page loads that stream: a
// decode call reads each page span once, so such loads pass the caches
// instead of displacing lines that are reused (rotations, queries, block
// tables).  A no-arithmetic gather of one B32 x 8192-token residual-loop call
// measured 163 us with nt against 177 us without.  Which page loads carry it
// is chosen per head dimension (PagePolicy in attention.hip).
constexpr int kStreamPolicy = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t handoff_resource(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void handoff_store(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, byte_offset, 0, kCoherentPolicy);
}

__device__ __forceinline__ void handoff_store4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset, float a, float b,
                                               float c, float d) {
    typedef uint32_t U32x4 __attribute__((ext_vector_type(4)));
    const U32x4 v = {__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_offset, 0, kCoherentPolicy);
}

__device__ __forceinline__ float2 handoff_load2(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_offset, 0, kCoherentPolicy);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

__device__ __forceinline__ float4 handoff_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, kCoherentPolicy);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}

// A value known to be equal in every lane, moved to scalar registers.
__device__ __forceinline__ int64_t uniform64(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Global memory read through the scalar cache (constant address space):
// loads from a wave-uniform address compile to s_load.  Only for data no
// kernel writes while the reading kernel runs.
typedef const int32_t __attribute__((address_space(4))) ConstantInt32;

// s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15): only outstanding vector memory
// operations (loads and stores) are waited for.
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0xF70); }

// Wave priority by the progress of a page stream of `steps` steps: 3 for
// the first 10/16 of the steps, then 2, 1 and from 15/16 on 0.  Two
// workgroups whose waves share the SIMDs of a compute unit otherwise
// progress unevenly (the older wave issues first), so one finishes well
// before the other, which then streams alone at a lower rate; with the
// priority falling as a wave advances, the one behind issues first and the
// two finish together.  The last bucket is short because the two waves' lag
// at the end is at most its length.  Only for grids whose workgroups all fit
// the device at once (`enabled`): with more, uneven finishes let the waiting
// workgroups start as soon as a slot frees, and a workgroup that starts late
// with the top priority holds back the older ones (decode at 1024
// workgroups on 768 slots: residual call 334 -> 362 us with the priority).
struct StreamPriority {
    int to2, to1, to0;  // the first steps at priority 2, 1 and 0 (all 0: always 0)
    __device__ StreamPriority(int steps, bool enabled)
        : to2(enabled ? (10 * steps + 15) / 16 : 0),
          to1(enabled ? (13 * steps + 15) / 16 : 0),
          to0(enabled ? (15 * steps + 15) / 16 : 0) {}
    __device__ __forceinline__ void set(int step) const {
        if (step < to2)
            __builtin_amdgcn_s_setprio(3);
        else if (step < to1)
            __builtin_amdgcn_s_setprio(2);
        else if (step < to0)
            __builtin_amdgcn_s_setprio(1);
        else
            __builtin_amdgcn_s_setprio(0);
    }
};

// Request of `row` for a workgroup of whole waves (at most 16): the number of boundaries
// qsl[1..requests] at or below the row (qsl is nondecreasing), -1 if the row
// lies outside [qsl[0], qsl[requests]).  One round of parallel loads instead
// of a dependent binary search.
__device__ __forceinline__ int find_request_parallel(const int32_t* qsl, int64_t requests, int64_t row,
                                                     int* lds_counts) {
    const int c = threadIdx.x;
    const int threads = blockDim.x;
    // The range bounds are loaded with the counts, before the barrier.
    const int32_t lo = requests > 0 ? qsl[0] : 0;
    const int32_t hi = requests > 0 ? qsl[requests] : 0;
    int count = 0;
    for (int64_t j = 1 + c; j <= requests; j += threads) count += qsl[j] <= row ? 1 : 0;
#pragma unroll
    for (int d = 32; d; d >>= 1) count += __shfl_xor(count, d);
    if ((c & 63) == 0) lds_counts[c >> 6] = count;
    __syncthreads();
    if (requests <= 0 || row < lo || row >= hi) return -1;
    int total = 0;
    for (int w = 0; w < threads / 64; ++w) total += lds_counts[w];
    return total;
}

// Counts this workgroup's arrival at `counter` (after every thread's shared
// stores) and returns true in every thread of the workgroup that arrives last
// of `expected`.  Nothing waits for other workgroups.
__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* lds_flag) {
    wait_vector_memory();
    __syncthreads();
    if (threadIdx.x == 0)
        *lds_flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expected - 1;
    __syncthreads();
    return *lds_flag != 0;
}

// ------------------------------------------------------------------ layout

// Bytes of one token of record (bits, group) at head_dim D
// (QuantizationRecord::Bytes, common/cache.cuh:14-17).
__host__ __device__ constexpr int record_bytes(int head_dim, int bits, int group) {
    return head_dim * bits / 8 + 2 * head_dim / group + 2;
}

constexpr int kMaxRecords = 8;

// Host-resolved description of one record's region inside a page.
struct RecordRegion {
    int offset;      // page_tokens * StorageOffset(record), bytes from the page base
    int bits;        // 2 or 4
    int group;       // 16 or 32
    int code_bytes;  // head_dim * bits / 8
    int groups;      // head_dim / group
};

}  // namespace rq
