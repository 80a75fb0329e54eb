// Bandwidth probe for the decode roofline: a contiguous streaming read of a
// C2-sized packed cache (B32 x 8192 tokens x 16 heads, page width 200) versus
// the exact page-gather pattern of one residual-loop decode call (per page and
// plane: the anchor record's codes/scales/offsets at offset 2016 and loop 0's
// record at offset 0, 1824 bytes), with no arithmetic beyond an xor.
//   lane_gather: the decode kernel's loads (lane = token x 32-channel quarter,
//                7 buffer loads per plane), PPI pages per wave iteration;
//   span_gather: the same bytes as lane-linear 16-byte chunks of the two spans;
// each with the default cache policy and with nt (non-temporal).  Prints
// microseconds and GB/s of algorithmic bytes; not part of librq_hip.so.
//
//   make -C residualquant_amd/csrc probe && residualquant_amd/csrc/build/bandwidth_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include <algorithm>
#include <random>
typedef uint32_t U4 __attribute__((ext_vector_type(4)));
typedef uint32_t U2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* b, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(b), (short)0, (int)n, 0x00020000);
}

__global__ __launch_bounds__(256) void stream_read(const uint4* __restrict__ p, size_t n16, unsigned* out) {
    unsigned acc = 0;
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
        uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x12345678u) out[0] = acc;
}

// Span gather: per page and plane the two spans [0,672) and [2016,3168) as 16-byte chunks,
// lane-linear (228 chunks per page over both planes), PPI pages per wave iteration.
template <int PPI, int AUX>
__global__ __launch_bounds__(256) void span_gather(const unsigned char* __restrict__ cache, const int* __restrict__ table,
                                                   int pages, int heads, int splits, long plane_stride, unsigned* out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int split = blockIdx.x % splits; const int rh = blockIdx.x / splits;
    const int head = rh % heads, row = rh / heads;
    const int pb = split * pages / splits, pe = (split + 1) * pages / splits;
    const auto kr = rsrc(cache, (uint32_t)plane_stride), vr = rsrc(cache + plane_stride, (uint32_t)plane_stride);
    // chunk c in [0,228): plane = c / 114, j = c % 114; j < 42 -> offset 16j, else 2016 + 16(j-42)
    uint32_t off[4]; bool vpl[4]; bool ok[4];
    for (int i = 0; i < 4; ++i) {
        int c = lane + 64 * i; ok[i] = c < 228; int cc = ok[i] ? c : 0;
        vpl[i] = cc >= 114; int j = cc % 114;
        off[i] = j < 42 ? 16 * j : 2016 + 16 * (j - 42);
    }
    unsigned acc = 0;
    for (int pg = pb + wave * PPI; pg < pe; pg += 4 * PPI) {
        U4 v[PPI][4];
        for (int q = 0; q < PPI; ++q) {
            int p = pg + q < pe ? pg + q : pg;
            const int block = __builtin_amdgcn_readfirstlane(table[row * pages + p]);
            const uint32_t base = (uint32_t)(((long)block * heads + head) * 3200);
            for (int i = 0; i < 4; ++i) {
                auto r = vpl[i] ? vr : kr;
                v[q][i] = ok[i] ? __builtin_amdgcn_raw_buffer_load_b128(r, base + off[i], 0, AUX) : U4{0,0,0,0};
            }
        }
        for (int q = 0; q < PPI; ++q) for (int i = 0; i < 4; ++i) acc ^= v[q][i].x ^ v[q][i].y ^ v[q][i].z ^ v[q][i].w;
    }
    if (acc == 0x12345678u) out[0] = acc;
}

// Kernel-like gather: lane = (token, quarter), 7 buffer loads per plane, PPI pages per iteration.
template <int PPI, int AUX>
__global__ __launch_bounds__(256) void lane_gather(const unsigned char* __restrict__ cache, const int* __restrict__ table,
                                                   int pages, int heads, int splits, long plane_stride, unsigned* out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int split = blockIdx.x % splits; const int rh = blockIdx.x / splits;
    const int head = rh % heads, row = rh / heads;
    const int t = lane >> 2, qd = lane & 3;
    const int pb = split * pages / splits, pe = (split + 1) * pages / splits;
    const auto kr = rsrc(cache, (uint32_t)plane_stride), vr = rsrc(cache + plane_stride, (uint32_t)plane_stride);
    unsigned acc = 0;
    for (int pg = pb + wave * PPI; pg < pe; pg += 4 * PPI) {
        unsigned x[PPI][2][8];
        for (int q = 0; q < PPI; ++q) {
            int p = pg + q < pe ? pg + q : pg;
            const int block = __builtin_amdgcn_readfirstlane(table[row * pages + p]);
            const uint32_t base = (uint32_t)(((long)block * heads + head) * 3200);
            for (int pl = 0; pl < 2; ++pl) {
                auto r = pl ? vr : kr;
                U4 a = __builtin_amdgcn_raw_buffer_load_b128(r, base + 2016 + t * 64 + qd * 16, 0, AUX);
                U2 l = __builtin_amdgcn_raw_buffer_load_b64(r, base + t * 32 + qd * 8, 0, AUX);
                unsigned s0 = __builtin_amdgcn_raw_buffer_load_b8(r, base + 3040 + t * 4 + qd, 0, AUX);
                unsigned o0 = __builtin_amdgcn_raw_buffer_load_b8(r, base + 3104 + t * 4 + qd, 0, AUX);
                unsigned s1 = __builtin_amdgcn_raw_buffer_load_b8(r, base + 512 + t * 4 + qd, 0, AUX);
                unsigned o1 = __builtin_amdgcn_raw_buffer_load_b8(r, base + 576 + t * 4 + qd, 0, AUX);
                unsigned al = __builtin_amdgcn_raw_buffer_load_b16(r, base + 640 + 2 * t, 0, AUX);
                x[q][pl][0] = a.x ^ a.y; x[q][pl][1] = a.z ^ a.w; x[q][pl][2] = l.x ^ l.y;
                x[q][pl][3] = s0; x[q][pl][4] = o0; x[q][pl][5] = s1; x[q][pl][6] = o1; x[q][pl][7] = al;
            }
        }
        for (int q = 0; q < PPI; ++q) for (int pl = 0; pl < 2; ++pl) for (int i = 0; i < 8; ++i) acc ^= x[q][pl][i];
    }
    if (acc == 0x12345678u) out[0] = acc;
}

#define CHECK(x)                                                              \
    do {                                                                      \
        hipError_t e_ = (x);                                                  \
        if (e_ != hipSuccess) {                                               \
            printf("%s: %s\n", #x, hipGetErrorString(e_));                   \
            return 1;                                                         \
        }                                                                     \
    } while (0)

typedef void (*GatherFn)(const unsigned char*, const int*, int, int, int, long, unsigned*);

int main() {
    const int rows = 32, heads = 16, pages = 512;
    const long blocks = (long)rows * pages;
    const long plane = blocks * heads * 3200;
    unsigned char* cache; unsigned* out; int* table;
    CHECK(hipMalloc(&cache, 2 * plane)); CHECK(hipMalloc(&out, 4)); CHECK(hipMalloc(&table, rows * pages * 4));
    CHECK(hipMemset(cache, 1, 2 * plane));
    std::vector<int> ids(rows * pages); for (int i = 0; i < rows * pages; ++i) ids[i] = i;
    std::shuffle(ids.begin(), ids.end(), std::mt19937(5));
    CHECK(hipMemcpy(table, ids.data(), ids.size() * 4, hipMemcpyHostToDevice));
    hipEvent_t e0, e1; CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
    float ms;
    for (int grid : {2048, 4096}) {
        for (int w = 0; w < 2; ++w) stream_read<<<grid, 256>>>((const uint4*)cache, 2 * plane / 16, out);
        CHECK(hipEventRecord(e0));
        for (int r = 0; r < 10; ++r) stream_read<<<grid, 256>>>((const uint4*)cache, 2 * plane / 16, out);
        CHECK(hipEventRecord(e1)); CHECK(hipEventSynchronize(e1)); CHECK(hipEventElapsedTime(&ms, e0, e1));
        printf("stream_read grid=%d: %.1f us -> %.0f GB/s\n", grid, ms / 10 * 1e3, 2.0 * plane / (ms / 10 * 1e-3) / 1e9);
    }
    struct V { const char* name; GatherFn f; };
    V vs[] = {{"lane ppi1", lane_gather<1, 0>}, {"lane ppi2", lane_gather<2, 0>}, {"lane ppi2 nt", lane_gather<2, 2>},
              {"lane ppi4", lane_gather<4, 0>},
              {"span ppi1", span_gather<1, 0>}, {"span ppi2", span_gather<2, 0>}, {"span ppi2 nt", span_gather<2, 2>},
              {"span ppi4", span_gather<4, 0>}};
    double alg = (double)rows * pages * heads * 2 * 1824;
    for (auto& v : vs) {
        for (int splits : {1, 2, 4}) {
            int grid = rows * heads * splits;
            for (int w = 0; w < 2; ++w) v.f<<<grid, 256>>>(cache, table, pages, heads, splits, plane, out);
            CHECK(hipEventRecord(e0));
            for (int r = 0; r < 20; ++r) v.f<<<grid, 256>>>(cache, table, pages, heads, splits, plane, out);
            CHECK(hipEventRecord(e1)); CHECK(hipEventSynchronize(e1)); CHECK(hipEventElapsedTime(&ms, e0, e1));
            printf("%-14s splits=%d: %.1f us -> %.0f GB/s algorithmic\n", v.name, splits, ms / 20 * 1e3, alg / (ms / 20 * 1e-3) / 1e9);
        }
    }
    CHECK(hipGetLastError());
    return 0;
}
