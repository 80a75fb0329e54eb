/*
 * CPU oracle for the ResidualQuant packed KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or
 * calls this file: it is the checker that tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the HIP library against.
 *
 * It restates, in plain C with explicit rounding, the semantics of the
 * reference's CUDA extension (heejunkim00/ResidualQuant, paths relative to
 * plugins/residual_quantization/csrc/):
 *
 *   packed page layout        common/cache.cuh:10-106, attention/async_copy.cuh:14-42
 *   quantize-on-write         quantize/kernel.cuh:14-355 (+ rotation.cuh:24-150)
 *   record restore            quantize/kernel.cuh:160-203, attention/compute.cuh:28-197
 *   decode attention          attention/prepare.cuh:13-230, compute.cuh:226-727,
 *                             merge.cuh:8-84, output.cuh:9-31, rotation.cuh:10-84
 *   prefill attention         src/residual_quantization/packed_backend.py:63-77
 *                             (vLLM flash_attn_varlen_func: textbook causal softmax)
 *
 * Canonical arithmetic (the reference binary's own order is not reproducible:
 * it uses TF32 mma.sync with a hardware-defined accumulation order and
 * --use_fast_math division/sqrt, setup.py:44-49):
 *   - rotation y[c] = sum_k x[k]*R[k][c], accumulated k-ascending in FP32 from
 *     +0 with fmaf (every product is exact: 8-bit x 11-bit significands);
 *   - least-squares / norm sums: per 32-lane "lane" l owning channels 4l..4l+3,
 *     a sequential fmaf chain, then the xor butterfly 16,8,4,2,1;
 *   - IEEE division and square root, no flush-to-zero;
 *   - FP8 E4M3 (OCP) encoding with round-to-nearest-even and saturation to
 *     +-448 (the __nv_fp8_e4m3(float) constructor is satfinite RNE);
 *   - every BF16 result (__hfma2/__hadd2/__float2bfloat16_rn) is a single
 *     round-to-nearest-even of the exact value;
 *   - min/max order -0 below +0.
 *
 * Attention is evaluated in FP64: keys as the reference decode kernel scores
 * them (unrounded code*scale+offset terms), values as its BF16 restore.
 *
 * Parity pins (tests/test_oracle_*.py): page widths, bit positions, the
 * exhaustive FP8 table against torch.float8_e4m3fn, BF16 rounding against
 * torch and exact rationals, quantize closed forms (constant groups, grid
 * values, ties, alpha special cases, LS optimality), rotation against float64
 * matmul bounds, attention against torch float64 SDPA.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define RQ_ORACLE_MAX_RECORDS 8
#define RQ_ORACLE_MAX_DIM 128

/* ------------------------------------------------------------------ */
/* scalar formats                                                       */
/* ------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* __float2bfloat16_rn: round-to-nearest-even of an FP32 value. */
uint16_t rq_oracle_bf16_rn(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float rq_oracle_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* FP16 (IEEE binary16) to FP32, exact. */
float rq_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0) {
        float magnitude = (float)mantissa * 5.9604644775390625e-08f; /* 2^-24 */
        return sign ? -magnitude : magnitude;
    }
    if (exponent == 31) return bits_f32(sign | 0x7f800000u | (mantissa << 13));
    return bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/*
 * Single RNE rounding to BF16 of the exact value s + err, where s is an FP32
 * value and |err| is at most half an FP32 ulp of s (an exact TwoSum pair).
 * BF16 midpoints are FP32 values, so only a sum that lands exactly on one
 * needs the error term to break the tie.
 */
static uint16_t bf16_round_pair(float s, float err) {
    uint32_t u = f32_bits(s);
    if ((u & 0xffffu) == 0x8000u && err != 0.0f) {
        /* Exact value lies strictly above or below the midpoint. */
        int away = (err > 0.0f) == (s > 0.0f);
        u = away ? u + 1u : u - 1u;
        s = bits_f32(u);
    }
    return rq_oracle_bf16_rn(s);
}

/* BF16(a*b + c) rounded once; a, b, c are BF16 so a*b is exact in FP32. */
uint16_t rq_oracle_bf16_fma_rn(uint16_t a, uint16_t b, uint16_t c) {
    float p = rq_oracle_bf16_to_f32(a) * rq_oracle_bf16_to_f32(b);
    float q = rq_oracle_bf16_to_f32(c);
    float s = p + q;
    float bb = s - p;
    float err = (p - (s - bb)) + (q - bb);
    return bf16_round_pair(s, err);
}

/* BF16(a + b) rounded once (exact in FP32 whenever it matters). */
uint16_t rq_oracle_bf16_add_rn(uint16_t a, uint16_t b) {
    float p = rq_oracle_bf16_to_f32(a);
    float q = rq_oracle_bf16_to_f32(b);
    float s = p + q;
    float bb = s - p;
    float err = (p - (s - bb)) + (q - bb);
    return bf16_round_pair(s, err);
}

/* OCP FP8 E4M3, bias 7, max 448, NaN = S.1111.111, no infinities. */
float rq_oracle_e4m3_to_f32(uint8_t v) {
    int sign = v >> 7;
    int exponent = (v >> 3) & 0xf;
    int mantissa = v & 7;
    float magnitude;
    if (exponent == 0xf && mantissa == 7) return sign ? -NAN : NAN;
    if (exponent == 0)
        magnitude = (float)mantissa * 0.001953125f; /* 2^-9 */
    else
        magnitude = ldexpf(1.0f + (float)mantissa / 8.0f, exponent - 7);
    return sign ? -magnitude : magnitude;
}

/* RNE with saturation to +-448 (satfinite), sign of zero kept. */
uint8_t rq_oracle_e4m3_from_f32(float f) {
    uint32_t u = f32_bits(f);
    uint8_t sign = (uint8_t)((u >> 31) << 7);
    float a = fabsf(f);
    if (a != a) return (uint8_t)(sign | 0x7f);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7e);
    if (a < 0.015625f) { /* below 2^-6: multiples of 2^-9 */
        float k = nearbyintf(a * 512.0f);
        return (uint8_t)(sign | (uint8_t)k);
    }
    uint32_t ua = f32_bits(a);
    int exponent = (int)(ua >> 23) - 127;
    uint32_t mantissa = ua & 0x7fffffu;
    uint32_t kept = mantissa >> 20;
    uint32_t round_bit = (mantissa >> 19) & 1u;
    uint32_t sticky = mantissa & 0x7ffffu;
    if (round_bit && (sticky || (kept & 1u))) kept++;
    if (kept == 8) {
        kept = 0;
        exponent++;
    }
    uint32_t code = ((uint32_t)(exponent + 7) << 3) | kept;
    if (code > 0x7e) code = 0x7e;
    return (uint8_t)(sign | code);
}

static inline float min_z(float a, float b) {
    return (a < b || (a == b && signbit(a))) ? a : b;
}

static inline float max_z(float a, float b) {
    return (a > b || (a == b && !signbit(a))) ? a : b;
}

/* ------------------------------------------------------------------ */
/* layout (common/cache.cuh:14-29, :78-80)                             */
/* ------------------------------------------------------------------ */

int rq_oracle_record_bytes(int head_dim, int bits, int group) {
    return head_dim * bits / 8 + 2 * head_dim / group + 2;
}

int rq_oracle_page_width(int head_dim, int records, const int* bits, const int* groups) {
    int width = 0;
    for (int r = 0; r < records; ++r) width += rq_oracle_record_bytes(head_dim, bits[r], groups[r]);
    return width;
}

/* The schedules the layout admits (cache.cuh:74-96): D a positive multiple
 * of 32 up to the oracle's buffers, INT2/INT4 records whose group divides D. */
static int valid_schedule(int head_dim, int records, const int* bits, const int* groups) {
    if (records < 1 || records > RQ_ORACLE_MAX_RECORDS) return 0;
    if (head_dim <= 0 || head_dim % 32 || head_dim > RQ_ORACLE_MAX_DIM) return 0;
    for (int r = 0; r < records; ++r) {
        if (bits[r] != 2 && bits[r] != 4) return 0;
        if (groups[r] <= 0 || head_dim % groups[r]) return 0;
    }
    return 1;
}

static int record_offset(int head_dim, int record, const int* bits, const int* groups) {
    int offset = 0;
    for (int r = 0; r < record; ++r) offset += rq_oracle_record_bytes(head_dim, bits[r], groups[r]);
    return offset;
}

/* ------------------------------------------------------------------ */
/* quantize-on-write (quantize/kernel.cuh)                              */
/* ------------------------------------------------------------------ */

/* Rotation y = x.R, k-ascending FP32 (rotation.cuh:5, :44-57 indexing). */
static void rotate_row(const uint16_t* x, const uint16_t* matrix, int head_dim, float* y) {
    for (int c = 0; c < head_dim; ++c) {
        float acc = 0.0f;
        for (int k = 0; k < head_dim; ++k)
            acc = fmaf(rq_oracle_bf16_to_f32(x[k]),
                       rq_oracle_f16_to_f32(matrix[(size_t)k * head_dim + c]), acc);
        y[c] = acc;
    }
}

/* Exported for the rotation pin. */
void rq_oracle_rotate(const uint16_t* x, const uint16_t* matrix, int head_dim, float* y) {
    rotate_row(x, matrix, head_dim, y);
}

/* 32-lane butterfly sum over per-lane partials (kernel.cuh:15-20). */
static float butterfly_sum(const float* partial) {
    float value[32];
    for (int l = 0; l < 32; ++l) value[l] = partial[l];
    for (int distance = 16; distance; distance >>= 1) {
        float next[32];
        for (int l = 0; l < 32; ++l) next[l] = value[l] + value[l ^ distance];
        memcpy(value, next, sizeof(value));
    }
    return value[0];
}

/*
 * One token row, one head, one plane, one record (kernel.cuh:33-228).
 * y: rotated input (FP32).  reference: BF16 restored record used as the LS
 * reference (in/out).  mean: FP32 channel mean of this record or NULL.
 */
static void quantize_record(
    const float* y, int head_dim, int bits, int group, int is_anchor, int restore,
    int coefficient, const float* mean, uint16_t* reference, uint8_t* record_base,
    int page_tokens, int token) {
    float previous[RQ_ORACLE_MAX_DIM] = {0};
    float x[RQ_ORACLE_MAX_DIM];
    float alpha = 1.0f;
    const int code_bytes = head_dim * bits / 8;
    const int groups = head_dim / group;

    if (!is_anchor)
        for (int c = 0; c < head_dim; ++c) previous[c] = rq_oracle_bf16_to_f32(reference[c]);
    for (int c = 0; c < head_dim; ++c) x[c] = y[c];

    if (!is_anchor && coefficient != 0) {
        float numerator[32] = {0}, denominator[32] = {0};
        for (int lane = 0; lane < 32; ++lane) {
            for (int i = 0; i < 4; ++i) {
                int c = lane * 4 + i;
                float xv = c < head_dim ? x[c] : 0.0f;
                float pv = c < head_dim ? previous[c] : 0.0f;
                if (coefficient == 1)
                    numerator[lane] = fmaf(xv, xv, numerator[lane]);
                else
                    numerator[lane] = fmaf(xv, pv, numerator[lane]);
                denominator[lane] = fmaf(pv, pv, denominator[lane]);
            }
        }
        float num = butterfly_sum(numerator);
        float den = butterfly_sum(denominator);
        if (coefficient == 1)
            alpha = den > 0.0f ? sqrtf(num) / fmaxf(sqrtf(den), 1e-6f) : 0.0f;
        else
            alpha = num / fmaxf(den, 1e-12f);
    }
    const uint16_t stored_alpha = rq_oracle_bf16_rn(alpha);
    alpha = rq_oracle_bf16_to_f32(stored_alpha);

    for (int c = 0; c < head_dim; ++c) {
        if (!is_anchor) x[c] = fmaf(-previous[c], alpha, x[c]);
        if (mean) x[c] = x[c] - mean[c];
    }

    uint8_t* codes = record_base + (size_t)token * code_bytes;
    uint8_t* scales = record_base + (size_t)page_tokens * code_bytes;
    uint8_t* offsets = scales + (size_t)page_tokens * groups;
    memset(codes, 0, (size_t)code_bytes);

    const float levels = (float)((1 << bits) - 1);
    for (int g = 0; g < groups; ++g) {
        float low = INFINITY, high = -INFINITY;
        for (int c = g * group; c < (g + 1) * group; ++c) {
            low = min_z(low, x[c]);
            high = max_z(high, x[c]);
        }
        const float center = (low + high) * 0.5f;
        const float radius = bits == 2 ? ((high - low) * 0.9f) * 0.5f : (high - low) * 0.5f;
        const uint8_t offset_code = rq_oracle_e4m3_from_f32(center - radius);
        const uint8_t scale_code = rq_oracle_e4m3_from_f32((2.0f * radius) / levels);
        const float scale = rq_oracle_e4m3_to_f32(scale_code);
        const float offset = rq_oracle_e4m3_to_f32(offset_code);
        scales[token * groups + g] = scale_code;
        offsets[token * groups + g] = offset_code;
        const uint16_t scale_bf = rq_oracle_bf16_rn(scale);
        const uint16_t offset_bf = rq_oracle_bf16_rn(offset);

        for (int c = g * group; c < (g + 1) * group; ++c) {
            unsigned code = 0;
            if (scale > 0.0f) {
                const float normalized = (x[c] - offset) / scale;
                const float lower = floorf(normalized);
                float rounded = lower + ((normalized - lower) > 0.5f ? 1.0f : 0.0f);
                rounded = fminf(fmaxf(rounded, 0.0f), levels);
                code = (unsigned)rounded;
            }
            codes[(c * bits) >> 3] |= (uint8_t)(code << ((c * bits) & 7));

            if (restore) {
                /* hfma2(code, scale, offset): exact in FP32, one rounding. */
                uint16_t value = rq_oracle_bf16_fma_rn(rq_oracle_bf16_rn((float)code), scale_bf, offset_bf);
                if (mean) value = rq_oracle_bf16_add_rn(value, rq_oracle_bf16_rn(mean[c]));
                if (!is_anchor) value = rq_oracle_bf16_fma_rn(reference[c], stored_alpha, value);
                reference[c] = value;
            }
        }
    }
    uint8_t* alpha_bytes = record_base + (size_t)page_tokens * (code_bytes + 2 * groups) + 2 * token;
    alpha_bytes[0] = (uint8_t)(stored_alpha & 0xff);
    alpha_bytes[1] = (uint8_t)(stored_alpha >> 8);
}

/*
 * quantize() (quantize/api.cpp:8-95, kernel.cuh:236-355).
 * key_ptrs[r] / value_ptrs[r]: BF16 [rows, heads, head_dim] with the given
 * token stride in elements.  Rotations: FP16 [heads, D, D] or NULL.
 * key_mean: FP32 [records, heads, D] or NULL.
 * reference_mode: 0 anchor, 1 adjacent.  coefficient: 0 unit, 1 norm, 2 ls.
 * Returns 0, or -1 on an argument the reference rejects.
 */
int rq_oracle_quantize(
    int records, const uint16_t* const* key_ptrs, const int64_t* key_strides,
    const uint16_t* const* value_ptrs, const int64_t* value_strides,
    uint8_t* cache, int64_t num_blocks, int heads, int page_tokens, int page_width,
    const int64_t* slot_mapping, int64_t tokens, int head_dim,
    const uint16_t* key_rotation, const uint16_t* value_rotation, const float* key_mean,
    const int* bits, const int* groups, int reference_mode, int anchor_index,
    int coefficient) {
    if (!valid_schedule(head_dim, records, bits, groups) || heads <= 0 || page_tokens <= 0) return -1;
    if (anchor_index < 0 || anchor_index >= records) return -1;
    if (reference_mode == 1 && anchor_index != 0) return -1;
    if (rq_oracle_page_width(head_dim, records, bits, groups) != page_width) return -1;
    /* A single-record group is always its own anchor (dispatch/schedules.cuh:99-111). */
    const int adjacent = records > 1 && reference_mode == 1;
    const int64_t plane_stride = num_blocks * heads * page_tokens * page_width;

    float y[RQ_ORACLE_MAX_RECORDS][RQ_ORACLE_MAX_DIM];
    uint16_t reference[RQ_ORACLE_MAX_DIM];
    for (int64_t n = 0; n < tokens; ++n) {
        const int64_t slot = slot_mapping[n];
        if (slot < 0) continue;
        const int64_t block = slot / page_tokens;
        const int token = (int)(slot % page_tokens);
        if (block >= num_blocks) return -1;
        for (int plane = 0; plane < 2; ++plane) {
            const uint16_t* rotation = plane == 0 ? key_rotation : value_rotation;
            for (int h = 0; h < heads; ++h) {
                for (int r = 0; r < records; ++r) {
                    const uint16_t* src = plane == 0
                        ? key_ptrs[r] + n * key_strides[r] + (int64_t)h * head_dim
                        : value_ptrs[r] + n * value_strides[r] + (int64_t)h * head_dim;
                    if (rotation)
                        rotate_row(src, rotation + (size_t)h * head_dim * head_dim, head_dim, y[r]);
                    else
                        for (int c = 0; c < head_dim; ++c) y[r][c] = rq_oracle_bf16_to_f32(src[c]);
                }
                uint8_t* page = cache + plane * plane_stride +
                                (block * heads + h) * (int64_t)page_tokens * page_width;
                /* Anchor first, then every other record ascending (kernel.cuh:321-329). */
                for (int step = 0; step < records; ++step) {
                    int r = step == 0 ? anchor_index : (step - 1 < anchor_index ? step - 1 : step);
                    const int is_anchor = r == anchor_index;
                    const float* mean = (plane == 0 && key_mean)
                        ? key_mean + ((size_t)r * heads + h) * head_dim : NULL;
                    uint8_t* record_base = page + (size_t)page_tokens * record_offset(head_dim, r, bits, groups);
                    quantize_record(y[r], head_dim, bits[r], groups[r], is_anchor,
                                    is_anchor || adjacent, coefficient, mean, reference,
                                    record_base, page_tokens, token);
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* restore (dequantize) of one record chain                             */
/* ------------------------------------------------------------------ */

static uint16_t restore_code_value(const uint8_t* record_base, int head_dim, int bits, int group,
                                   int page_tokens, int token, int c) {
    const int code_bytes = head_dim * bits / 8;
    const int groups = head_dim / group;
    const uint8_t* codes = record_base + (size_t)token * code_bytes;
    const uint8_t* scales = record_base + (size_t)page_tokens * code_bytes;
    const uint8_t* offsets = scales + (size_t)page_tokens * groups;
    const unsigned code = (codes[(c * bits) >> 3] >> ((c * bits) & 7)) & ((1u << bits) - 1u);
    const int g = c / group;
    const uint16_t scale_bf = rq_oracle_bf16_rn(rq_oracle_e4m3_to_f32(scales[token * groups + g]));
    const uint16_t offset_bf = rq_oracle_bf16_rn(rq_oracle_e4m3_to_f32(offsets[token * groups + g]));
    return rq_oracle_bf16_fma_rn(rq_oracle_bf16_rn((float)code), scale_bf, offset_bf);
}

static uint16_t record_alpha(const uint8_t* record_base, int head_dim, int bits, int group,
                             int page_tokens, int token) {
    const int code_bytes = head_dim * bits / 8;
    const int groups = head_dim / group;
    const uint8_t* a = record_base + (size_t)page_tokens * (code_bytes + 2 * groups) + 2 * token;
    return (uint16_t)(a[0] | (a[1] << 8));
}

/*
 * Restored BF16 value of `loop` for one (plane, page, token): the record the
 * quantizer keeps as its reference (kernel.cuh:160-203).  Anchor mode:
 * X_A = bf16(c.s+o) [+ bf16(mu_A) on K], X_L = bf16(alpha_L*X_A + bf16(c.s+o)
 * [+ bf16(mu_L)]).  Adjacent mode chains X_r from X_{r-1} (compute.cuh:120-197).
 */
static void restore_token(const uint8_t* page, int head_dim, int records, const int* bits,
                          const int* groups, int page_tokens, int token, int adjacent,
                          int anchor_index, int loop, const float* mean_base, int heads, int h,
                          uint16_t* out) {
    int chain[RQ_ORACLE_MAX_RECORDS];
    (void)records;
    int length = 0;
    if (adjacent) {
        for (int r = 0; r <= loop; ++r) chain[length++] = r;
    } else {
        chain[length++] = anchor_index;
        if (loop != anchor_index) chain[length++] = loop;
    }
    for (int i = 0; i < length; ++i) {
        const int r = chain[i];
        const uint8_t* record_base = page + (size_t)page_tokens * record_offset(head_dim, r, bits, groups);
        const uint16_t alpha = record_alpha(record_base, head_dim, bits[r], groups[r], page_tokens, token);
        for (int c = 0; c < head_dim; ++c) {
            uint16_t value = restore_code_value(record_base, head_dim, bits[r], groups[r], page_tokens, token, c);
            if (mean_base) value = rq_oracle_bf16_add_rn(value, rq_oracle_bf16_rn(mean_base[((size_t)r * heads + h) * head_dim + c]));
            if (i > 0) value = rq_oracle_bf16_fma_rn(out[c], alpha, value);
            out[c] = value;
        }
    }
}

/*
 * Dequantize the given slots for `loop` into BF16 [tokens, heads, D] K and V
 * (rotated space).  Slots < 0 produce zeros.
 */
int rq_oracle_dequantize(const uint8_t* cache, int64_t num_blocks, int heads, int page_tokens,
                         int page_width, const int64_t* slots, int64_t tokens, int head_dim,
                         const float* key_mean, int records, const int* bits, const int* groups,
                         int reference_mode, int anchor_index, int loop, uint16_t* key_out,
                         uint16_t* value_out) {
    if (!valid_schedule(head_dim, records, bits, groups) || heads <= 0 || page_tokens <= 0) return -1;
    if (loop < 0 || loop >= records || anchor_index < 0 || anchor_index >= records) return -1;
    if (rq_oracle_page_width(head_dim, records, bits, groups) != page_width) return -1;
    const int adjacent = records > 1 && reference_mode == 1;
    const int64_t plane_stride = num_blocks * heads * page_tokens * page_width;
    for (int64_t n = 0; n < tokens; ++n) {
        for (int h = 0; h < heads; ++h) {
            uint16_t* kout = key_out + (n * heads + h) * head_dim;
            uint16_t* vout = value_out + (n * heads + h) * head_dim;
            if (slots[n] < 0) {
                memset(kout, 0, sizeof(uint16_t) * head_dim);
                memset(vout, 0, sizeof(uint16_t) * head_dim);
                continue;
            }
            const int64_t block = slots[n] / page_tokens;
            const int token = (int)(slots[n] % page_tokens);
            if (block >= num_blocks) return -1;
            const uint8_t* page = cache + (block * heads + h) * (int64_t)page_tokens * page_width;
            restore_token(page, head_dim, records, bits, groups, page_tokens, token, adjacent,
                          anchor_index, loop, key_mean, heads, h, kout);
            restore_token(page + plane_stride, head_dim, records, bits, groups, page_tokens, token,
                          adjacent, anchor_index, loop, NULL, heads, h, vout);
        }
    }
    return 0;
}

/* Unrounded code*scale + offset of channel c (exact in double). */
static double record_value_exact(const uint8_t* record_base, int head_dim, int bits, int group,
                                 int page_tokens, int token, int c) {
    const int code_bytes = head_dim * bits / 8;
    const int groups = head_dim / group;
    const uint8_t* codes = record_base + (size_t)token * code_bytes;
    const uint8_t* scales = record_base + (size_t)page_tokens * code_bytes;
    const uint8_t* offsets = scales + (size_t)page_tokens * groups;
    const unsigned code = (codes[(c * bits) >> 3] >> ((c * bits) & 7)) & ((1u << bits) - 1u);
    const int g = c / group;
    return (double)code * (double)rq_oracle_e4m3_to_f32(scales[token * groups + g]) +
           (double)rq_oracle_e4m3_to_f32(offsets[token * groups + g]);
}

/*
 * History key of one token as the reference decode kernel scores it, in
 * exact arithmetic.  Anchor mode (compute.cuh:397-505, prepare.cuh:203-229):
 * loop A scores q'.(c.s+o)_A, loop L != A scores
 * alpha_L*(q'.(c.s+o)_A + q'.bf16(mu_A)) + q'.(c.s+o)_L, both shifted by
 * -q'.mu_L against the live score; the key below adds mu_L back, which leaves
 * the softmax unchanged.  Adjacent mode (compute.cuh:120-197, :506-528)
 * scores the BF16 restore chain without the current loop's mean.
 */
static void attention_key(const uint8_t* page, int head_dim, const int* bits, const int* groups,
                          int page_tokens, int token, int adjacent, int anchor_index, int loop,
                          const float* mean_base, int heads, int h, double* out) {
    const float* mean_loop = mean_base ? mean_base + ((size_t)loop * heads + h) * head_dim : NULL;
    if (adjacent) {
        uint16_t chain[RQ_ORACLE_MAX_DIM];
        for (int r = 0; r <= loop; ++r) {
            const uint8_t* record_base = page + (size_t)page_tokens * record_offset(head_dim, r, bits, groups);
            const uint16_t alpha = record_alpha(record_base, head_dim, bits[r], groups[r], page_tokens, token);
            for (int c = 0; c < head_dim; ++c) {
                uint16_t value = restore_code_value(record_base, head_dim, bits[r], groups[r], page_tokens, token, c);
                if (mean_base && r != loop)
                    value = rq_oracle_bf16_add_rn(value, rq_oracle_bf16_rn(mean_base[((size_t)r * heads + h) * head_dim + c]));
                if (r > 0) value = rq_oracle_bf16_fma_rn(chain[c], alpha, value);
                chain[c] = value;
            }
        }
        for (int c = 0; c < head_dim; ++c)
            out[c] = (double)rq_oracle_bf16_to_f32(chain[c]) + (mean_loop ? (double)mean_loop[c] : 0.0);
        return;
    }
    const uint8_t* anchor_base = page + (size_t)page_tokens * record_offset(head_dim, anchor_index, bits, groups);
    const float* mean_anchor = mean_base ? mean_base + ((size_t)anchor_index * heads + h) * head_dim : NULL;
    if (loop == anchor_index) {
        for (int c = 0; c < head_dim; ++c)
            out[c] = record_value_exact(anchor_base, head_dim, bits[anchor_index], groups[anchor_index],
                                        page_tokens, token, c) + (mean_loop ? (double)mean_loop[c] : 0.0);
        return;
    }
    const uint8_t* loop_base = page + (size_t)page_tokens * record_offset(head_dim, loop, bits, groups);
    const double alpha = rq_oracle_bf16_to_f32(record_alpha(loop_base, head_dim, bits[loop], groups[loop],
                                                            page_tokens, token));
    for (int c = 0; c < head_dim; ++c) {
        double anchor = record_value_exact(anchor_base, head_dim, bits[anchor_index], groups[anchor_index],
                                           page_tokens, token, c);
        if (mean_anchor) anchor += rq_oracle_bf16_to_f32(rq_oracle_bf16_rn(mean_anchor[c]));
        out[c] = alpha * anchor +
                 record_value_exact(loop_base, head_dim, bits[loop], groups[loop], page_tokens, token, c) +
                 (mean_loop ? (double)mean_loop[c] : 0.0);
    }
}

/* ------------------------------------------------------------------ */
/* decode attention (FP64 over the restored K/V)                        */
/* ------------------------------------------------------------------ */

/*
 * For each query row i of request b (query_start_loc), head h, loop L:
 *   q' = (q.R_k)/sqrt(D); history t < H_b scores q'.K_L[t] with K_L the
 *   key the reference decode kernel scores (attention_key above) and V_L[t]
 *   the BF16 restore (restore_token, compute.cuh:28-107);
 *   live scores (q.k_j)/sqrt(D) over the live set; p = softmax over history
 *   and live set; out = (sum_t p_t V_L[t]).R_v^T + sum_j p_j v_j
 *   (merge.cuh:66-83, output.cuh:9-31, compute.cuh:688-726, prepare.cuh:13-54).
 * Decode (causal = 0, the reference's attention()): H_b = seq_len - 1 and the
 * live set is the row's own key/value.  Prefill over packed history
 * (causal = 1): the n rows of request b are its last n tokens, H_b =
 * seq_len - n, and row r (0-based within the request) sees the request's
 * new keys/values j <= r.  Output is FP64 [rows, heads, D].
 */
/* One (row i of request b, head h) of attention_rows; -1 on a bad block id. */
static int attention_row_head(
    const uint16_t* query, int64_t query_stride, const uint16_t* key, int64_t key_stride,
    const uint16_t* value, int64_t value_stride, double* output, int heads, int head_dim,
    const uint8_t* cache, int64_t num_blocks, int page_tokens, int page_width, int64_t first, int64_t n,
    int64_t seq_len, const int32_t* table_row, const uint16_t* key_rotation, const uint16_t* value_rotation,
    const float* key_mean, int records, const int* bits, const int* groups, int adjacent, int anchor_index,
    int loop, int causal, int64_t i, int h) {
    const int64_t plane_stride = num_blocks * heads * page_tokens * page_width;
    const double scale = 1.0 / sqrt((double)head_dim);
    const int64_t new_tokens = causal ? n : 1;
    const int64_t history = seq_len > new_tokens ? seq_len - new_tokens : 0;
    const int64_t live_first = causal ? first : i;
    const int64_t live_count = causal ? i - first + 1 : 1;
    uint16_t vbuf[RQ_ORACLE_MAX_DIM];
    double kexact[RQ_ORACLE_MAX_DIM];
    double* scores = (double*)malloc(sizeof(double) * (size_t)(history + live_count + 1));
    if (!scores) return -1;
    double* live_scores = scores + history;
    const uint16_t* q = query + i * query_stride + (int64_t)h * head_dim;
    double qr[RQ_ORACLE_MAX_DIM];
    for (int c = 0; c < head_dim; ++c) {
        double acc = 0.0;
        if (key_rotation) {
            const uint16_t* m = key_rotation + (size_t)h * head_dim * head_dim;
            for (int k = 0; k < head_dim; ++k)
                acc += (double)rq_oracle_bf16_to_f32(q[k]) * (double)rq_oracle_f16_to_f32(m[(size_t)k * head_dim + c]);
        } else {
            acc = rq_oracle_bf16_to_f32(q[c]);
        }
        qr[c] = acc * scale;
    }
    double maximum = -INFINITY;
    for (int64_t j = 0; j < live_count; ++j) {
        const uint16_t* kl = key + (live_first + j) * key_stride + (int64_t)h * head_dim;
        double live = 0.0;
        for (int c = 0; c < head_dim; ++c)
            live += (double)rq_oracle_bf16_to_f32(q[c]) * (double)rq_oracle_bf16_to_f32(kl[c]);
        live_scores[j] = live * scale;
        if (live_scores[j] > maximum) maximum = live_scores[j];
    }
    for (int64_t t = 0; t < history; ++t) {
        const int64_t block = table_row[t / page_tokens];
        if (block < 0 || block >= num_blocks) {
            free(scores);
            return -1;
        }
        const uint8_t* page = cache + (block * heads + h) * (int64_t)page_tokens * page_width;
        attention_key(page, head_dim, bits, groups, page_tokens, (int)(t % page_tokens), adjacent, anchor_index,
                      loop, key_mean, heads, h, kexact);
        double s = 0.0;
        for (int c = 0; c < head_dim; ++c) s += qr[c] * kexact[c];
        scores[t] = s;
        if (s > maximum) maximum = s;
    }
    double denominator = 0.0;
    for (int64_t j = 0; j < live_count; ++j) {
        live_scores[j] = exp(live_scores[j] - maximum);
        denominator += live_scores[j];
    }
    for (int64_t t = 0; t < history; ++t) {
        scores[t] = exp(scores[t] - maximum);
        denominator += scores[t];
    }
    double hist[RQ_ORACLE_MAX_DIM] = {0};
    for (int64_t t = 0; t < history; ++t) {
        const int64_t block = table_row[t / page_tokens];
        const uint8_t* page = cache + plane_stride + (block * heads + h) * (int64_t)page_tokens * page_width;
        restore_token(page, head_dim, records, bits, groups, page_tokens, (int)(t % page_tokens), adjacent,
                      anchor_index, loop, NULL, heads, h, vbuf);
        for (int c = 0; c < head_dim; ++c) hist[c] += scores[t] * (double)rq_oracle_bf16_to_f32(vbuf[c]);
    }
    double* out = output + (i * heads + h) * (int64_t)head_dim;
    for (int c = 0; c < head_dim; ++c) {
        double v = 0.0;
        if (value_rotation) {
            const uint16_t* m = value_rotation + (size_t)h * head_dim * head_dim;
            for (int k = 0; k < head_dim; ++k) v += hist[k] * (double)rq_oracle_f16_to_f32(m[(size_t)c * head_dim + k]);
        } else {
            v = hist[c];
        }
        double live = 0.0;
        for (int64_t j = 0; j < live_count; ++j) {
            const uint16_t* vl = value + (live_first + j) * value_stride + (int64_t)h * head_dim;
            live += live_scores[j] * (double)rq_oracle_bf16_to_f32(vl[c]);
        }
        out[c] = (v + live) / denominator;
    }
    free(scores);
    return 0;
}

static int attention_rows(
    const uint16_t* query, int64_t query_stride, const uint16_t* key, int64_t key_stride,
    const uint16_t* value, int64_t value_stride, double* output, int64_t rows, int heads,
    int head_dim, const uint8_t* cache, int64_t num_blocks, int page_tokens, int page_width,
    const int32_t* query_start_loc, const int32_t* seq_lens, int64_t requests,
    const int32_t* block_table, int64_t block_table_stride, const uint16_t* key_rotation,
    const uint16_t* value_rotation, const float* key_mean, int records, const int* bits,
    const int* groups, int reference_mode, int anchor_index, int loop, int causal) {
    if (!valid_schedule(head_dim, records, bits, groups) || heads <= 0 || page_tokens <= 0) return -1;
    if (loop < 0 || loop >= records || anchor_index < 0 || anchor_index >= records) return -1;
    if (rq_oracle_page_width(head_dim, records, bits, groups) != page_width) return -1;
    const int adjacent = records > 1 && reference_mode == 1;
    /* The request of each row (-1: no request owns it; its output stays 0). */
    int64_t* row_request = (int64_t*)malloc(sizeof(int64_t) * (size_t)(rows > 0 ? rows : 1));
    if (!row_request) return -1;
    for (int64_t i = 0; i < rows; ++i) row_request[i] = -1;
    for (int64_t b = 0; b < requests; ++b)
        for (int64_t i = query_start_loc[b]; i < query_start_loc[b + 1] && i < rows; ++i) row_request[i] = b;
    int failed = 0;
    /* (row, head) pairs are independent: they run in parallel when built with OpenMP. */
#pragma omp parallel for schedule(dynamic, 1) reduction(| : failed)
    for (int64_t w = 0; w < rows * heads; ++w) {
        const int64_t i = w / heads;
        const int h = (int)(w % heads);
        const int64_t b = row_request[i];
        if (b < 0) continue;
        const int64_t first = query_start_loc[b];
        failed |= attention_row_head(query, query_stride, key, key_stride, value, value_stride, output, heads,
                                     head_dim, cache, num_blocks, page_tokens, page_width, first,
                                     query_start_loc[b + 1] - first, seq_lens[b],
                                     block_table + b * block_table_stride, key_rotation, value_rotation, key_mean,
                                     records, bits, groups, adjacent, anchor_index, loop, causal, i, h) != 0;
    }
    free(row_request);
    return failed ? -1 : 0;
}

int rq_oracle_attention(
    const uint16_t* query, int64_t query_stride, const uint16_t* key, int64_t key_stride,
    const uint16_t* value, int64_t value_stride, double* output, int64_t rows, int heads,
    int head_dim, const uint8_t* cache, int64_t num_blocks, int page_tokens, int page_width,
    const int32_t* query_start_loc, const int32_t* seq_lens, int64_t requests,
    const int32_t* block_table, int64_t block_table_stride, const uint16_t* key_rotation,
    const uint16_t* value_rotation, const float* key_mean, int records, const int* bits,
    const int* groups, int reference_mode, int anchor_index, int loop) {
    return attention_rows(query, query_stride, key, key_stride, value, value_stride, output, rows, heads,
                          head_dim, cache, num_blocks, page_tokens, page_width, query_start_loc, seq_lens,
                          requests, block_table, block_table_stride, key_rotation, value_rotation, key_mean,
                          records, bits, groups, reference_mode, anchor_index, loop, 0);
}

int rq_oracle_attention_prefill(
    const uint16_t* query, int64_t query_stride, const uint16_t* key, int64_t key_stride,
    const uint16_t* value, int64_t value_stride, double* output, int64_t rows, int heads,
    int head_dim, const uint8_t* cache, int64_t num_blocks, int page_tokens, int page_width,
    const int32_t* query_start_loc, const int32_t* seq_lens, int64_t requests,
    const int32_t* block_table, int64_t block_table_stride, const uint16_t* key_rotation,
    const uint16_t* value_rotation, const float* key_mean, int records, const int* bits,
    const int* groups, int reference_mode, int anchor_index, int loop) {
    return attention_rows(query, query_stride, key, key_stride, value, value_stride, output, rows, heads,
                          head_dim, cache, num_blocks, page_tokens, page_width, query_start_loc, seq_lens,
                          requests, block_table, block_table_stride, key_rotation, value_rotation, key_mean,
                          records, bits, groups, reference_mode, anchor_index, loop, 1);
}

/*
 * BF16 paged decode attention (the comparison baseline): cache BF16
 * [2, blocks, heads, page_tokens, D], history t < seq_len-1 from the cache,
 * the current token from key/value.  FP64 result [rows, heads, D].
 */
int rq_oracle_paged_attention_bf16(
    const uint16_t* query, int64_t query_stride, const uint16_t* key, int64_t key_stride,
    const uint16_t* value, int64_t value_stride, double* output, int64_t rows, int heads,
    int head_dim, const uint16_t* cache, int64_t num_blocks, int page_tokens,
    const int32_t* query_start_loc, const int32_t* seq_lens, int64_t requests,
    const int32_t* block_table, int64_t block_table_stride) {
    if (heads <= 0 || head_dim <= 0 || head_dim > RQ_ORACLE_MAX_DIM) return -1;
    const int64_t plane_stride = num_blocks * heads * page_tokens * head_dim;
    const double scale = 1.0 / sqrt((double)head_dim);
    for (int64_t b = 0; b < requests; ++b) {
        const int64_t history = seq_lens[b] > 1 ? seq_lens[b] - 1 : 0;
        double* scores = (double*)malloc(sizeof(double) * (size_t)(history + 1));
        if (!scores) return -1;
        for (int64_t i = query_start_loc[b]; i < query_start_loc[b + 1] && i < rows; ++i) {
            for (int h = 0; h < heads; ++h) {
                const uint16_t* q = query + i * query_stride + (int64_t)h * head_dim;
                const uint16_t* kl = key + i * key_stride + (int64_t)h * head_dim;
                const uint16_t* vl = value + i * value_stride + (int64_t)h * head_dim;
                double live = 0.0;
                for (int c = 0; c < head_dim; ++c)
                    live += (double)rq_oracle_bf16_to_f32(q[c]) * (double)rq_oracle_bf16_to_f32(kl[c]);
                live *= scale;
                double maximum = live;
                for (int64_t t = 0; t < history; ++t) {
                    const int64_t block = block_table[b * block_table_stride + t / page_tokens];
                    if (block < 0 || block >= num_blocks) {
                        free(scores);
                        return -1;
                    }
                    const uint16_t* k = cache + ((block * heads + h) * page_tokens + t % page_tokens) * head_dim;
                    double s = 0.0;
                    for (int c = 0; c < head_dim; ++c)
                        s += (double)rq_oracle_bf16_to_f32(q[c]) * (double)rq_oracle_bf16_to_f32(k[c]);
                    scores[t] = s * scale;
                    if (scores[t] > maximum) maximum = scores[t];
                }
                double denominator = exp(live - maximum);
                double hist[RQ_ORACLE_MAX_DIM] = {0};
                for (int64_t t = 0; t < history; ++t) {
                    const int64_t block = block_table[b * block_table_stride + t / page_tokens];
                    const uint16_t* v = cache + plane_stride +
                                        ((block * heads + h) * page_tokens + t % page_tokens) * head_dim;
                    const double p = exp(scores[t] - maximum);
                    denominator += p;
                    for (int c = 0; c < head_dim; ++c) hist[c] += p * (double)rq_oracle_bf16_to_f32(v[c]);
                }
                double* out = output + (i * heads + h) * (int64_t)head_dim;
                const double live_weight = exp(live - maximum);
                for (int c = 0; c < head_dim; ++c)
                    out[c] = (hist[c] + live_weight * (double)rq_oracle_bf16_to_f32(vl[c])) / denominator;
            }
        }
        free(scores);
    }
    return 0;
}

/* Varlen prefill attention in FP64: the flash_attn_varlen_func call of the
 * full-prompt branch (src/residual_quantization/packed_backend.py:63-77).
 * For sequence s (cu_q[s]..cu_q[s+1] queries, cu_k[s]..cu_k[s+1] keys), query
 * head h reads key/value head h / (heads_q / heads_k); query i sees keys
 * j <= i + len_k - len_q when causal (all keys otherwise); a query with no
 * key gets a zero row.  out[i] = sum_j softmax_j(scale * q_i . k_j) v_j. */
int rq_oracle_prefill_attention(const uint16_t* query, int64_t query_stride, const uint16_t* key,
                                int64_t key_stride, const uint16_t* value, int64_t value_stride, double* output,
                                int heads_q, int heads_k, int head_dim, const int32_t* cu_q, const int32_t* cu_k,
                                int64_t batch, double scale, int causal) {
    if (heads_q <= 0 || heads_k <= 0 || heads_q % heads_k || head_dim <= 0 || head_dim > RQ_ORACLE_MAX_DIM)
        return -1;
    const int group = heads_q / heads_k;
    for (int64_t s = 0; s < batch; ++s) {
        const int64_t q_begin = cu_q[s], q_len = cu_q[s + 1] - cu_q[s];
        const int64_t k_begin = cu_k[s], k_len = cu_k[s + 1] - cu_k[s];
        if (q_len < 0 || k_len < 0) return -1;
        int failed = 0;
        /* Query rows are independent: they run in parallel when built with OpenMP. */
#pragma omp parallel for schedule(dynamic, 4) reduction(| : failed)
        for (int64_t i = 0; i < q_len; ++i) {
            int64_t last = causal ? i + k_len - q_len : k_len - 1;
            if (last > k_len - 1) last = k_len - 1;
            double* scores = (double*)malloc(sizeof(double) * (size_t)(k_len > 0 ? k_len : 1));
            if (!scores) {
                failed = 1;
                continue;
            }
            for (int h = 0; h < heads_q; ++h) {
                const int kh = h / group;
                const uint16_t* q = query + (q_begin + i) * query_stride + (int64_t)h * head_dim;
                double* out = output + ((q_begin + i) * heads_q + h) * (int64_t)head_dim;
                for (int c = 0; c < head_dim; ++c) out[c] = 0.0;
                if (last < 0) continue;
                double maximum = -INFINITY;
                for (int64_t j = 0; j <= last; ++j) {
                    const uint16_t* k = key + (k_begin + j) * key_stride + (int64_t)kh * head_dim;
                    double dot = 0.0;
                    for (int c = 0; c < head_dim; ++c)
                        dot += (double)rq_oracle_bf16_to_f32(q[c]) * (double)rq_oracle_bf16_to_f32(k[c]);
                    scores[j] = scale * dot;
                    if (scores[j] > maximum) maximum = scores[j];
                }
                double denominator = 0.0;
                for (int64_t j = 0; j <= last; ++j) {
                    const uint16_t* v = value + (k_begin + j) * value_stride + (int64_t)kh * head_dim;
                    const double p = exp(scores[j] - maximum);
                    denominator += p;
                    for (int c = 0; c < head_dim; ++c) out[c] += p * (double)rq_oracle_bf16_to_f32(v[c]);
                }
                for (int c = 0; c < head_dim; ++c) out[c] /= denominator;
            }
            free(scores);
        }
        if (failed) return -1;
    }
    return 0;
}
