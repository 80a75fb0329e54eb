// Bandwidth probe for the C4 decode roofline: the page-gather pattern of one
// Huginn-shaped residual-loop call (B8 x 4096 tokens x 55 heads, D96, page
// 16 x 170 bytes: loop 0's [2,16] record at [0, 608) and the [4,32] anchor at
// [1824, 2688) of each K and V page), lane-linear 16-byte chunks, one
// workgroup per (row, head), with no arithmetic beyond an xor; default cache
// policy and nt.  Prints microseconds and GB/s of algorithmic page bytes; not
// part of librq_hip.so.
//
//   make -C residualquant_amd/csrc probe && residualquant_amd/csrc/build/bandwidth_probe_c4
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include <algorithm>
#include <random>
typedef uint32_t U4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* b, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(b), (short)0, (int)n, 0x00020000);
}
// C4 residual-loop gather: page 16 x 170 = 2720 B; loop-0 record [0, 608), anchor [1824, 2688).
template <int PPI, int AUX>
__global__ __launch_bounds__(256) void span_gather(const unsigned char* __restrict__ cache, const int* __restrict__ table,
                                                   int pages, int heads, long plane_stride, unsigned* out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rh = blockIdx.x; const int head = rh % heads, row = rh / heads;
    const auto kr = rsrc(cache, (uint32_t)plane_stride), vr = rsrc(cache + plane_stride, (uint32_t)plane_stride);
    uint32_t off[3]; bool vpl[3]; bool ok[3];
    for (int i = 0; i < 3; ++i) {
        int c = lane + 64 * i; ok[i] = c < 184; int cc = ok[i] ? c : 0;
        vpl[i] = cc >= 92; int j = cc % 92;
        off[i] = j < 38 ? 16 * j : 1824 + 16 * (j - 38);
    }
    unsigned acc = 0;
    for (int pg = wave * PPI; pg < pages; pg += 4 * PPI) {
        U4 v[PPI][3];
        for (int q = 0; q < PPI; ++q) {
            int p = pg + q < pages ? pg + q : pg;
            const int block = __builtin_amdgcn_readfirstlane(table[row * pages + p]);
            const uint32_t base = (uint32_t)(((long)block * heads + head) * 2720);
            for (int i = 0; i < 3; ++i) {
                auto r = vpl[i] ? vr : kr;
                v[q][i] = ok[i] ? __builtin_amdgcn_raw_buffer_load_b128(r, base + off[i], 0, AUX) : U4{0,0,0,0};
            }
        }
        for (int q = 0; q < PPI; ++q) for (int i = 0; i < 3; ++i) acc ^= v[q][i].x ^ v[q][i].y ^ v[q][i].z ^ v[q][i].w;
    }
    if (acc == 0x12345678u) out[0] = acc;
}
typedef void (*Fn)(const unsigned char*, const int*, int, int, long, unsigned*);
#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("%s: %s\n", #x, hipGetErrorString(e_)); return 1; } } while (0)
int main() {
    const int rows = 8, heads = 55, pages = 256;
    const long blocks = (long)rows * pages;
    const long plane = blocks * heads * 2720;
    unsigned char* cache; unsigned* out; int* table;
    CHECK(hipMalloc(&cache, 2 * plane)); CHECK(hipMalloc(&out, 4)); CHECK(hipMalloc(&table, rows * pages * 4));
    CHECK(hipMemset(cache, 1, 2 * plane));
    std::vector<int> ids(rows * pages); for (int i = 0; i < rows * pages; ++i) ids[i] = i;
    std::shuffle(ids.begin(), ids.end(), std::mt19937(5));
    CHECK(hipMemcpy(table, ids.data(), ids.size() * 4, hipMemcpyHostToDevice));
    hipEvent_t e0, e1; CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
    float ms;
    struct V { const char* n; Fn f; };
    V vs[] = {{"ppi1", span_gather<1, 0>}, {"ppi2", span_gather<2, 0>}, {"ppi1 nt", span_gather<1, 2>}, {"ppi2 nt", span_gather<2, 2>}};
    double alg = (double)rows * pages * heads * 2 * (608 + 864);
    for (auto& v : vs) {
        for (int w = 0; w < 2; ++w) v.f<<<rows * heads, 256>>>(cache, table, pages, heads, plane, out);
        CHECK(hipEventRecord(e0));
        for (int r = 0; r < 20; ++r) v.f<<<rows * heads, 256>>>(cache, table, pages, heads, plane, out);
        CHECK(hipEventRecord(e1)); CHECK(hipEventSynchronize(e1)); CHECK(hipEventElapsedTime(&ms, e0, e1));
        printf("C4 gather %-8s: %.1f us -> %.0f GB/s algorithmic (pages only)\n", v.n, ms / 20 * 1e3, alg / (ms / 20 * 1e-3) / 1e9);
    }
    CHECK(hipGetLastError());
    return 0;
}
