// Bandwidth probe for the decode roofline: a contiguous streaming read of a
// C2-sized packed cache (B32 x 8192 tokens x 16 heads, page width 200) versus
// the exact page-gather pattern of one residual-loop decode call (per page and
// plane: the anchor record's codes/scales/offsets at offset 2016 and loop 0's
// record at offset 0, 1824 bytes), with no arithmetic beyond an xor.  Prints
// GB/s; not part of librq_hip.so.
//
//   make -C residualquant_amd/csrc probe && residualquant_amd/csrc/build/bandwidth_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#include <random>

__global__ __launch_bounds__(256) void stream_read(const uint4* __restrict__ p, size_t n16, unsigned* out) {
    unsigned acc = 0;
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
        uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x12345678u) out[0] = acc;
}

// One workgroup per (row, head, split) as in the decode kernel; wave w takes pages w, w+4, ...;
// lane = (token, 32-channel quarter) reads its anchor codes (16 B), loop codes (8 B), the
// FP8 scale/offset bytes of both records and the loop alpha, for K and V.
__global__ __launch_bounds__(256) void gather(const unsigned char* __restrict__ cache, const int* __restrict__ table,
                                              int pages, int heads, int splits, long plane_stride, unsigned* out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int split = blockIdx.x % splits; const int rh = blockIdx.x / splits;
    const int head = rh % heads, row = rh / heads;
    const int t = lane >> 2, qd = lane & 3;
    const int pb = split * pages / splits, pe = (split + 1) * pages / splits;
    unsigned acc = 0;
    for (int pg = pb + wave; pg < pe; pg += 4) {
        const int block = __builtin_amdgcn_readfirstlane(table[row * pages + pg]);
        const unsigned char* k = cache + ((long)block * heads + head) * 3200;
        const unsigned char* v = k + plane_stride;
        for (int pl = 0; pl < 2; ++pl) {
            const unsigned char* b = pl ? v : k;
            uint4 a = *(const uint4*)(b + 2016 + t * 64 + qd * 16);
            uint2 r = *(const uint2*)(b + t * 32 + qd * 8);
            unsigned s0 = b[2016 + 1024 + t * 4 + qd], o0 = b[2016 + 1088 + t * 4 + qd];
            unsigned s1 = b[512 + t * 4 + qd], o1 = b[576 + t * 4 + qd];
            unsigned al = *(const unsigned short*)(b + 640 + 2 * t);
            acc ^= a.x ^ a.y ^ a.z ^ a.w ^ r.x ^ r.y ^ s0 ^ o0 ^ s1 ^ o1 ^ al;
        }
    }
    if (acc == 0x12345678u) out[0] = acc;
}

int main() {
    const int rows = 32, heads = 16, pages = 512;
    const long blocks = (long)rows * pages;
    const long plane = blocks * heads * 3200;
    unsigned char* cache; unsigned* out; int* table;
    hipMalloc(&cache, 2 * plane); hipMalloc(&out, 4); hipMalloc(&table, rows * pages * 4);
    hipMemset(cache, 1, 2 * plane);
    std::vector<int> ids(rows * pages); for (int i = 0; i < rows * pages; ++i) ids[i] = i;
    std::shuffle(ids.begin(), ids.end(), std::mt19937(5));
    hipMemcpy(table, ids.data(), ids.size() * 4, hipMemcpyHostToDevice);
    hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
    float ms;
    // stream read of the whole cache (3.36 GB)
    for (int grid : {1024, 2048, 4096, 8192}) {
        for (int w = 0; w < 2; ++w) stream_read<<<grid, 256>>>((const uint4*)cache, 2 * plane / 16, out);
        hipEventRecord(e0);
        for (int r = 0; r < 10; ++r) stream_read<<<grid, 256>>>((const uint4*)cache, 2 * plane / 16, out);
        hipEventRecord(e1); hipEventSynchronize(e1); hipEventElapsedTime(&ms, e0, e1);
        printf("stream_read grid=%d: %.1f us per 3.36 GB -> %.0f GB/s\n", grid, ms / 10 * 1e3, 2.0 * plane / (ms / 10 * 1e-3) / 1e9);
    }
    for (int splits : {1, 2, 4, 8}) {
        int grid = rows * heads * splits;
        for (int w = 0; w < 2; ++w) gather<<<grid, 256>>>(cache, table, pages, heads, splits, plane, out);
        hipEventRecord(e0);
        for (int r = 0; r < 10; ++r) gather<<<grid, 256>>>(cache, table, pages, heads, splits, plane, out);
        hipEventRecord(e1); hipEventSynchronize(e1); hipEventElapsedTime(&ms, e0, e1);
        double alg = (double)rows * pages * heads * 2 * 1824;
        printf("gather splits=%d: %.1f us -> %.0f GB/s algorithmic (1824 B/page/plane)\n", splits, ms / 10 * 1e3, alg / (ms / 10 * 1e-3) / 1e9);
    }
    return 0;
}
