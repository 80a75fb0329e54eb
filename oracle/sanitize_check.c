/*
 * Sanitizer run of the CPU oracle (test infrastructure, like rq_oracle.c).
 *
 * Built by `make -C oracle asan` together with rq_oracle.c under
 * AddressSanitizer and UndefinedBehaviorSanitizer (no recovery: the first
 * report aborts), then run.  It drives every exported oracle function over
 * the shapes the tests use and the edges of the oracle's fixed-size stack
 * buffers (D = 128, 8 records, 32-token pages), with every buffer allocated
 * at its exact size so that an access one element past a tensor, page, table
 * or row is reported.  It also feeds pages of random bytes (FP8 NaN codes,
 * any alpha) to the restore and attention paths, and checks that arguments
 * outside the oracle's limits are rejected (-1) before any access.
 *
 * Exit status 0 when every call behaved; the sanitizers abort otherwise.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint16_t rq_oracle_bf16_rn(float f);
float rq_oracle_bf16_to_f32(uint16_t h);
float rq_oracle_f16_to_f32(uint16_t h);
uint16_t rq_oracle_bf16_fma_rn(uint16_t a, uint16_t b, uint16_t c);
uint16_t rq_oracle_bf16_add_rn(uint16_t a, uint16_t b);
float rq_oracle_e4m3_to_f32(uint8_t v);
uint8_t rq_oracle_e4m3_from_f32(float f);
int rq_oracle_record_bytes(int head_dim, int bits, int group);
int rq_oracle_page_width(int head_dim, int records, const int* bits, const int* groups);
void rq_oracle_rotate(const uint16_t* x, const uint16_t* matrix, int head_dim, float* y);
int rq_oracle_quantize(int records, const uint16_t* const* key_ptrs, const int64_t* key_strides,
                       const uint16_t* const* value_ptrs, const int64_t* value_strides, uint8_t* cache,
                       int64_t num_blocks, int heads, int page_tokens, int page_width, const int64_t* slot_mapping,
                       int64_t tokens, int head_dim, const uint16_t* key_rotation, const uint16_t* value_rotation,
                       const float* key_mean, const int* bits, const int* groups, int reference_mode,
                       int anchor_index, int coefficient);
int rq_oracle_dequantize(const uint8_t* cache, int64_t num_blocks, int heads, int page_tokens, int page_width,
                         const int64_t* slots, int64_t tokens, int head_dim, const float* key_mean, int records,
                         const int* bits, const int* groups, int reference_mode, int anchor_index, int loop,
                         uint16_t* key_out, uint16_t* value_out);
typedef int (*attention_fn)(const uint16_t*, int64_t, const uint16_t*, int64_t, const uint16_t*, int64_t, double*,
                            int64_t, int, int, const uint8_t*, int64_t, int, int, const int32_t*, const int32_t*,
                            int64_t, const int32_t*, int64_t, const uint16_t*, const uint16_t*, const float*, int,
                            const int*, const int*, int, int, int);
int rq_oracle_attention(const uint16_t*, int64_t, const uint16_t*, int64_t, const uint16_t*, int64_t, double*,
                        int64_t, int, int, const uint8_t*, int64_t, int, int, const int32_t*, const int32_t*,
                        int64_t, const int32_t*, int64_t, const uint16_t*, const uint16_t*, const float*, int,
                        const int*, const int*, int, int, int);
int rq_oracle_attention_prefill(const uint16_t*, int64_t, const uint16_t*, int64_t, const uint16_t*, int64_t,
                                double*, int64_t, int, int, const uint8_t*, int64_t, int, int, const int32_t*,
                                const int32_t*, int64_t, const int32_t*, int64_t, const uint16_t*, const uint16_t*,
                                const float*, int, const int*, const int*, int, int, int);
int rq_oracle_paged_attention_bf16(const uint16_t* query, int64_t query_stride, const uint16_t* key,
                                   int64_t key_stride, const uint16_t* value, int64_t value_stride, double* output,
                                   int64_t rows, int heads, int head_dim, const uint16_t* cache, int64_t num_blocks,
                                   int page_tokens, const int32_t* query_start_loc, const int32_t* seq_lens,
                                   int64_t requests, const int32_t* block_table, int64_t block_table_stride);
int rq_oracle_prefill_attention(const uint16_t* query, int64_t query_stride, const uint16_t* key,
                                int64_t key_stride, const uint16_t* value, int64_t value_stride, double* output,
                                int heads_q, int heads_k, int head_dim, const int32_t* cu_q, const int32_t* cu_k,
                                int64_t batch, double scale, int causal);

static uint64_t state = 0x9e3779b97f4a7c15ull;

static uint32_t next_u32(void) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return (uint32_t)(state >> 16);
}

static float uniform(void) { return (float)(next_u32() & 0xffffff) / 16777216.0f * 2.0f - 1.0f; }

static void* exact(size_t bytes) {
    void* p = malloc(bytes ? bytes : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static uint16_t* bf16_tensor(size_t count, float amplitude) {
    uint16_t* t = exact(sizeof(uint16_t) * count);
    for (size_t i = 0; i < count; ++i) t[i] = rq_oracle_bf16_rn(amplitude * uniform());
    return t;
}

/* FP16 bit patterns of magnitude in [1/8, 1) with random sign. */
static uint16_t* f16_tensor(size_t count) {
    uint16_t* t = exact(sizeof(uint16_t) * count);
    for (size_t i = 0; i < count; ++i) {
        const uint32_t r = next_u32();
        t[i] = (uint16_t)(((r & 1u) << 15) | ((12u + (r >> 1) % 3u) << 10) | ((r >> 4) & 0x3ffu));
    }
    return t;
}

static int failures = 0;

static void expect(int condition, const char* what) {
    if (!condition) {
        fprintf(stderr, "FAILED: %s\n", what);
        ++failures;
    }
}

struct scenario {
    int head_dim, heads, page_tokens, records, mode, anchor, coefficient, rotation, mean;
    int bits[8], groups[8];
};

static void run(const struct scenario* s, int random_pages) {
    const int D = s->head_dim, H = s->heads, PT = s->page_tokens, R = s->records;
    const int width = rq_oracle_page_width(D, R, s->bits, s->groups);
    /* Three requests: histories 0, PT + 3 and 3 * PT, with 1, 3 and 2 new rows. */
    const int requests = 3;
    const int history[3] = {0, PT + 3, 3 * PT};
    const int new_rows[3] = {1, 3, 2};
    const int pages_per_request = 4;
    const int64_t blocks = requests * pages_per_request;
    const size_t plane = (size_t)blocks * H * PT * width;
    uint8_t* cache = exact(2 * plane);
    memset(cache, 0, 2 * plane);
    int32_t* table = exact(sizeof(int32_t) * requests * pages_per_request);
    for (int i = 0; i < requests * pages_per_request; ++i) table[i] = (int32_t)(blocks - 1 - i);

    int64_t tokens = 0;
    for (int b = 0; b < requests; ++b) tokens += history[b];
    int64_t* slots = exact(sizeof(int64_t) * (size_t)(tokens + 1));
    int64_t n = 0;
    for (int b = 0; b < requests; ++b)
        for (int t = 0; t < history[b]; ++t)
            slots[n++] = (int64_t)table[b * pages_per_request + t / PT] * PT + t % PT;
    slots[n] = -1; /* a skipped token */
    const int64_t written = n + 1;

    const uint16_t* keys[8];
    const uint16_t* values[8];
    int64_t strides[8];
    for (int r = 0; r < R; ++r) {
        keys[r] = bf16_tensor((size_t)written * H * D, 3.0f);
        values[r] = bf16_tensor((size_t)written * H * D, 3.0f);
        strides[r] = (int64_t)H * D;
    }
    uint16_t* key_rotation = s->rotation ? f16_tensor((size_t)H * D * D) : NULL;
    uint16_t* value_rotation = s->rotation ? f16_tensor((size_t)H * D * D) : NULL;
    float* mean = NULL;
    if (s->mean) {
        mean = exact(sizeof(float) * (size_t)R * H * D);
        for (size_t i = 0; i < (size_t)R * H * D; ++i) mean[i] = 0.5f * uniform();
    }
    expect(rq_oracle_quantize(R, keys, strides, values, strides, cache, blocks, H, PT, width, slots, written, D,
                              key_rotation, value_rotation, mean, s->bits, s->groups, s->mode, s->anchor,
                              s->coefficient) == 0,
           "quantize");
    if (random_pages)
        for (size_t i = 0; i < 2 * plane; ++i) cache[i] = (uint8_t)next_u32();

    uint16_t* k_out = exact(sizeof(uint16_t) * (size_t)written * H * D);
    uint16_t* v_out = exact(sizeof(uint16_t) * (size_t)written * H * D);
    for (int loop = 0; loop < R; ++loop)
        expect(rq_oracle_dequantize(cache, blocks, H, PT, width, slots, written, D, mean, R, s->bits, s->groups,
                                    s->mode, s->anchor, loop, k_out, v_out) == 0,
               "dequantize");

    /* Decode (one row per request) and prefill over packed history (several). */
    for (int prefill = 0; prefill < 2; ++prefill) {
        int32_t qsl[4] = {0};
        int32_t seq[3];
        for (int b = 0; b < requests; ++b) {
            const int rows_b = prefill ? new_rows[b] : 1;
            qsl[b + 1] = qsl[b] + rows_b;
            seq[b] = history[b] + rows_b;
        }
        const int64_t rows = qsl[requests];
        uint16_t* q = bf16_tensor((size_t)rows * H * D, 1.0f);
        uint16_t* k = bf16_tensor((size_t)rows * H * D, 1.0f);
        uint16_t* v = bf16_tensor((size_t)rows * H * D, 1.0f);
        double* out = exact(sizeof(double) * (size_t)rows * H * D);
        attention_fn fn = prefill ? rq_oracle_attention_prefill : rq_oracle_attention;
        for (int loop = 0; loop < R; ++loop) {
            const int rc = fn(q, (int64_t)H * D, k, (int64_t)H * D, v, (int64_t)H * D, out, rows, H, D, cache, blocks,
                              PT, width, qsl, seq, requests, table, pages_per_request, key_rotation,
                              value_rotation, mean, R, s->bits, s->groups, s->mode, s->anchor, loop);
            expect(rc == 0, prefill ? "attention_prefill" : "attention");
            if (!random_pages)
                for (size_t i = 0; i < (size_t)rows * H * D; ++i) expect(isfinite(out[i]), "finite attention");
        }
        free(q);
        free(k);
        free(v);
        free(out);
    }

    free(cache);
    free(table);
    free(slots);
    for (int r = 0; r < R; ++r) {
        free((void*)keys[r]);
        free((void*)values[r]);
    }
    free(key_rotation);
    free(value_rotation);
    free(mean);
    free(k_out);
    free(v_out);
}

static void run_bf16_baselines(void) {
    for (int D = 32; D <= 128; D += 32) {
        const int H = 3, PT = 16, requests = 2, pages = 3;
        const int64_t blocks = requests * pages;
        uint16_t* cache = bf16_tensor((size_t)2 * blocks * H * PT * D, 2.0f);
        int32_t table[6] = {5, 3, 1, 0, 2, 4};
        int32_t qsl[3] = {0, 1, 2};
        int32_t seq[2] = {1, pages * PT};
        uint16_t* q = bf16_tensor((size_t)2 * H * D, 1.0f);
        double* out = exact(sizeof(double) * 2 * H * D);
        expect(rq_oracle_paged_attention_bf16(q, (int64_t)H * D, q, (int64_t)H * D, q, (int64_t)H * D, out, 2, H, D,
                                              cache, blocks, PT, qsl, seq, requests, table, pages) == 0,
               "paged_attention_bf16");
        free(cache);
        free(q);
        free(out);
    }
    /* Varlen causal and full attention with grouped heads, and a query with no key. */
    const int D = 128, hq = 4, hk = 2;
    int32_t cu_q[4] = {0, 5, 5, 12};
    int32_t cu_k[4] = {0, 3, 6, 18};
    uint16_t* q = bf16_tensor((size_t)12 * hq * D, 1.0f);
    uint16_t* kv = bf16_tensor((size_t)20 * hk * D, 1.0f);
    double* out = exact(sizeof(double) * 12 * hq * D);
    for (int causal = 0; causal < 2; ++causal)
        expect(rq_oracle_prefill_attention(q, (int64_t)hq * D, kv, (int64_t)hk * D, kv, (int64_t)hk * D, out, hq, hk,
                                           D, cu_q, cu_k, 3, 0.088, causal) == 0,
               "prefill_attention");
    free(q);
    free(kv);
    free(out);
}

static void run_rejections(void) {
    int bits[9] = {2, 2, 2, 2, 2, 2, 2, 2, 2}, groups[9] = {32, 32, 32, 32, 32, 32, 32, 32, 32};
    uint8_t cache[16] = {0};
    int64_t slot = 0;
    uint16_t out[16];
    /* Head dim beyond the oracle's buffers, too many records, a group that does not divide D. */
    expect(rq_oracle_dequantize(cache, 1, 1, 1, rq_oracle_page_width(160, 1, bits, groups), &slot, 1, 160, NULL, 1,
                                bits, groups, 0, 0, 0, out, out) == -1,
           "reject D 160");
    expect(rq_oracle_dequantize(cache, 1, 1, 1, rq_oracle_page_width(32, 9, bits, groups), &slot, 1, 32, NULL, 9, bits,
                                groups, 0, 0, 0, out, out) == -1,
           "reject 9 records");
    int odd_group[1] = {24};
    expect(rq_oracle_dequantize(cache, 1, 1, 1, rq_oracle_page_width(32, 1, bits, odd_group), &slot, 1, 32, NULL, 1,
                                bits, odd_group, 0, 0, 0, out, out) == -1,
           "reject group 24 at D 32");
    int three_bits[1] = {3};
    expect(rq_oracle_dequantize(cache, 1, 1, 1, 64, &slot, 1, 32, NULL, 1, three_bits, groups, 0, 0, 0, out, out) == -1,
           "reject INT3");
    double dout[1];
    int32_t zero = 0;
    expect(rq_oracle_paged_attention_bf16(out, 0, out, 0, out, 0, dout, 0, 1, 160, out, 1, 1, &zero, &zero, 0, &zero,
                                          1) == -1,
           "reject bf16 D 160");
}

int main(void) {
    const int g32[8] = {32, 32, 32, 32, 32, 32, 32, 32};
    const int g16[8] = {16, 16, 16, 32, 16, 16, 16, 16};
    const int ouro_bits[8] = {2, 2, 2, 4, 2, 2, 2, 2};
    struct scenario list[] = {
        /* D, H, PT, R, mode, anchor, coefficient, rotation, mean */
        {128, 2, 16, 4, 0, 3, 2, 1, 1, {0}, {0}},
        {128, 2, 32, 4, 0, 3, 1, 0, 1, {0}, {0}},
        {96, 3, 16, 4, 0, 3, 2, 1, 1, {0}, {0}},
        {96, 2, 32, 4, 1, 0, 0, 1, 0, {0}, {0}},
        {128, 1, 16, 8, 1, 0, 2, 1, 1, {0}, {0}},
        {128, 1, 32, 8, 0, 5, 2, 0, 1, {0}, {0}},
        {32, 2, 16, 1, 0, 0, 2, 1, 1, {0}, {0}},
        {64, 2, 16, 2, 0, 1, 1, 1, 0, {0}, {0}},
    };
    const int count = (int)(sizeof(list) / sizeof(list[0]));
    for (int i = 0; i < count; ++i) {
        struct scenario s = list[i];
        const int* groups = (i % 2) ? g32 : g16;
        for (int r = 0; r < s.records; ++r) {
            s.bits[r] = ouro_bits[r];
            s.groups[r] = s.head_dim % groups[r] ? 32 : groups[r];
        }
        if (s.records == 1) s.bits[0] = 4;
        for (int random_pages = 0; random_pages < 2; ++random_pages) run(&s, random_pages);
        printf("scenario %d: D %d, %d records, PT %d, %s mode: ok\n", i, s.head_dim, s.records, s.page_tokens,
               s.mode ? "adjacent" : "anchor");
    }
    run_bf16_baselines();
    run_rejections();
    /* Scalar helpers over edge values. */
    const float edges[] = {0.0f, -0.0f, 1e-40f, 448.0f, 464.0f, -1e30f, INFINITY, NAN};
    for (size_t i = 0; i < sizeof(edges) / sizeof(edges[0]); ++i) {
        (void)rq_oracle_e4m3_from_f32(edges[i]);
        (void)rq_oracle_bf16_rn(edges[i]);
    }
    for (int v = 0; v < 256; ++v) (void)rq_oracle_e4m3_to_f32((uint8_t)v);
    for (uint32_t h = 0; h < 65536; h += 7) {
        (void)rq_oracle_bf16_to_f32((uint16_t)h);
        (void)rq_oracle_f16_to_f32((uint16_t)h);
        (void)rq_oracle_bf16_add_rn((uint16_t)h, (uint16_t)(h * 31u));
        (void)rq_oracle_bf16_fma_rn((uint16_t)h, (uint16_t)(h * 17u), (uint16_t)(h * 5u));
    }
    uint16_t x[128];
    float y[128];
    uint16_t* m = f16_tensor(128 * 128);
    for (int i = 0; i < 128; ++i) x[i] = rq_oracle_bf16_rn(uniform());
    rq_oracle_rotate(x, m, 128, y);
    free(m);
    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("oracle sanitizer run: ok\n");
    return 0;
}
