/* Exhaustive CPU checks of the exact arithmetic shortcuts the quantize kernel
 * takes in place of the canonical formulas (test infrastructure).  Each check
 * prints "<name> <mismatches>"; the test asserts every count is 0.
 *
 *  reciprocal_division: q = RN(q0 + RN(a - q0*s) * y), q0 = RN(a*y),
 *      y = RN(1/s), equals the IEEE quotient RN(a/s) for every E4M3 scale
 *      mantissa and every FP32 a in one binade of quotients per sign (the
 *      computation is scale invariant while nothing is subnormal), plus the
 *      binades either side.
 *  half_down_rounding: floor(q) + (q - floor(q) > 0.5) == ceil(q - 0.5) after
 *      the [0, 15] clamp, for every FP32 q within 4096 ulps of each integer and
 *      half-integer up to 32 and on a 1/4099 stride of all |q| < 2^24.
 *  code_restore: code*scale + offset is exact in FP32 for every 4-bit code and
 *      pair of finite E4M3 values, so BF16(fma) == BF16(TwoSum form).
 *  bf16_sum: for every pair of finite BF16 values, RNE of the FP32 sum equals
 *      the single-rounded sum (TwoSum plus midpoint correction).
 *  level_division: the same reciprocal-and-correction form with the divisor
 *      3 or 15 (the code levels of INT2 and INT4) equals RN(v/levels) for
 *      every non-negative FP32 v with biased exponent 0..12 (subnormal
 *      quotients and remainders), 126..128 (the computation is scale
 *      invariant in between) and 250..254 (the largest values).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t u(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }
static uint32_t bf16_rn(float x) {
    uint32_t v = u(x);
    if ((v & 0x7fffffffu) > 0x7f800000u) return (v >> 16) | 0x40u;
    v += 0x7fffu + ((v >> 16) & 1u);
    return v >> 16;
}
static uint32_t round_pair(float s, float err) {
    uint32_t v = u(s);
    if ((v & 0xffffu) == 0x8000u && err != 0.f) {
        int away = (err > 0.f) == (s > 0.f);
        v = away ? v + 1 : v - 1;
        s = f(v);
    }
    return bf16_rn(s);
}
static uint32_t add_rn(float a, float b) { float s = a + b, bb = s - a, e = (a - (s - bb)) + (b - bb); return round_pair(s, e); }
static uint32_t fma_rn(float a, float b, float c) { float p = a * b, s = p + c, bb = s - p, e = (p - (s - bb)) + (c - bb); return round_pair(s, e); }
static float e4m3(uint32_t v) {
    uint32_t e = (v >> 3) & 15, m = v & 7;
    float g = e ? f(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
    return (v & 0x80) ? -g : g;
}
static float clamp15(float x) { return fminf(fmaxf(x, 0.f), 15.f); }

int main(void) {
    long bad = 0;
    for (int m = 8; m < 16; m++) {
        const float s = m / 8.0f, y = 1.0f / s;
        for (uint32_t ua = u(0.5f * s); ua < u(4.0f * s); ua++)
            for (int sign = 0; sign < 2; sign++) {
                const float a = sign ? -f(ua) : f(ua);
                const float q0 = a * y, r = fmaf(-q0, s, a), q = fmaf(r, y, q0);
                bad += u(q) != u(a / s);
            }
    }
    printf("reciprocal_division %ld\n", bad);

    bad = 0;
    for (int n2 = 0; n2 <= 64; n2++) {
        const uint32_t center = u(n2 * 0.5f);
        for (int d = -4096; d <= 4096; d++) {
            if (n2 == 0 && d < 0) continue;
            for (int sign = 0; sign < 2; sign++) {
                const float q = sign ? -f(center + d) : f(center + d);
                const float lower = floorf(q);
                bad += clamp15(lower + ((q - lower) > 0.5f ? 1.f : 0.f)) != clamp15(ceilf(q - 0.5f));
            }
        }
    }
    for (uint32_t uq = 0; uq < 0x4b800000u; uq += 4099)
        for (int sign = 0; sign < 2; sign++) {
            const float q = sign ? -f(uq) : f(uq);
            const float lower = floorf(q);
            bad += clamp15(lower + ((q - lower) > 0.5f ? 1.f : 0.f)) != clamp15(ceilf(q - 0.5f));
        }
    printf("half_down_rounding %ld\n", bad);

    bad = 0;
    for (int c = 0; c < 16; c++)
        for (int s = 0; s < 256; s++)
            for (int o = 0; o < 256; o++) {
                if ((s & 0x7f) == 0x7f || (o & 0x7f) == 0x7f) continue;
                const float fs = e4m3(s), fo = e4m3(o), single = (float)c * fs + fo;
                bad += (double)single != (double)c * fs + fo || fma_rn((float)c, fs, fo) != bf16_rn(single);
            }
    printf("code_restore %ld\n", bad);

    bad = 0;
    for (uint32_t a = 0; a < 65536; a++) {
        if (((a >> 7) & 0xff) == 0xff) continue;
        const float fa = f(a << 16);
        for (uint32_t b = 0; b < 65536; b++) {
            if (((b >> 7) & 0xff) == 0xff) continue;
            const float fb = f(b << 16);
            bad += add_rn(fa, fb) != bf16_rn(fa + fb);
        }
    }
    printf("bf16_sum %ld\n", bad);

    bad = 0;
    for (int levels = 3; levels <= 15; levels += 12) {
        const float l = (float)levels, y = 1.0f / l;
        const uint32_t ranges[3][2] = {{0u, 13u}, {126u, 129u}, {250u, 255u}};
        for (int range = 0; range < 3; range++)
            for (uint32_t uv = ranges[range][0] << 23; uv < ranges[range][1] << 23; uv++) {
                const float v = f(uv);
                const float q0 = v * y, r = fmaf(-q0, l, v), q = fmaf(r, y, q0);
                bad += u(q) != u(v / l);
            }
    }
    printf("level_division %ld\n", bad);
    return 0;
}
