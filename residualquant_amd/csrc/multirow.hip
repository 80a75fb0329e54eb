// Attention of several query rows per request over packed pages, on MFMA
// tiles (gfx950, wave64), for head dims 96 and 128, anchor and adjacent mode.
//
// The decode kernel scores one query row per workgroup with integer dot
// products on the packed codes, so n rows of one request stream the
// request's pages n times.  Here one workgroup takes a tile of up to 32 rows
// of one (request, head) and a split of its history, streams each page once,
// and dequantizes every 32-token tile into LDS as FP16 K and BF16 V (both
// row-major; V is read transposed by ds_read_b64_tr_b16), so that the tile's
// rows share it through MFMA:
//   S^T = K Q'^T     (32 tokens x 32 rows, D / 16 v_mfma_f32_32x32x16_f16)
//   O^T += V^T P^T   (D channels x 32 rows, D / 16 v_mfma_f32_32x32x16_bf16)
// The scores take FP16 operands (11-bit significands; each row of q' is
// scaled by a power of two into [-1, 1], which the scores take back), since
// BF16 operands there put the outlier channels' score error near the
// 1e-3 mean bar on short histories.  P stays in the accumulator registers
// (the token order of each P.V step is permuted to match the accumulator
// layout, and V^T is read with the same permutation).  Each of the four
// waves takes every fourth tile with its own online softmax; the waves meet
// once in LDS at the end and the workgroup writes one partial (m, l, O) per
// row.  The query prologue (q . R_k) runs on MFMA as well.  A finish launch
// per (request, head, 32-row tile) merges the splits, applies R_v^T (on
// MFMA) and adds the live tokens.
//
// Calls whose requests average 16 rows or fewer take 16-row tiles instead:
// the same pages and dequantization, with the tile's products on
// v_mfma_f32_16x16x32 (S^T: 2 token halves x D / 32 steps; O^T: D / 16
// channel blocks, one 32-token step each), which halves the matrix work and
// the softmax's per-lane scores of a tile that would otherwise be half empty.
//
// A lane dequantizes one token's 32-channel quarter of a 16-token unit
// (lane = token x quarter); at D = 96 the fourth quarter's lanes load a copy
// of the first quarter's bytes and store nothing.
//
// Semantics (reference: attention/compute.cuh:397-505 keys, :28-107 values,
// :120-197 and :506-623 the adjacent-mode chain, prepare.cuh:13-54 and
// :203-229 live score and mean shift, merge.cuh:8-84, output.cuh:9-31):
//   anchor mode: keys alpha_L (c.s+o + bf16(mu_A))_A + (c.s+o)_L with the
//     current loop's mean as a per-row shift, values alpha_L (c.s+o)_A +
//     (c.s+o)_L (the reference rounds each restore step to BF16; one
//     rounding here, within the attention tolerance) (AnchorDecoder);
//   adjacent mode past loop 0: keys and values the BF16 restore chain over
//     records 0..L, the key chain adding bf16(mu_r) to every record but the
//     current loop's (rq_chain.h; ChainDecoder);
// P in BF16.
//
// Lane layouts of v_mfma_f32_32x32x16_bf16 (checked on gfx950): A row l % 32,
// k 8 (l / 32) + e; B column l % 32, k 8 (l / 32) + e; C register r holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.  Of v_mfma_f32_16x16x32:
// A row l % 16, k 8 (l / 16) + e; B column l % 16, k 8 (l / 16) + e; C
// register r holds row 4 (l / 16) + r, column l % 16.
#include "rq_chain.h"
#include "rq_device.h"
#include "rq_kernels.h"

namespace rq {

namespace {

typedef __bf16 Bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 F16x8 __attribute__((ext_vector_type(8)));
typedef float F32x16 __attribute__((ext_vector_type(16)));
typedef float F32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kTile = 32;  // tokens per MFMA tile (two 16-token units)
constexpr int kMaxD = 128;

// LDS geometry of the stream kernel for head dim D and TR-row tiles.
template <int D, int TR = 32>
struct Geometry {
    static constexpr int Quarters = D / 32;  // 32-channel quarters a token's lanes cover
    static constexpr int Parts = D / 16;     // 16-channel parts (MFMA k steps of the scores)
    static constexpr int KS = D + 8;         // K tile row stride (halves)
    // V tile [token][VROW] BF16.  At D = 128 the row is unpadded and
    // swizzled by token, which keeps the transposed reads free of bank
    // conflicts: for 32-row tiles (a half-wave reads 4 tokens x 32 channels)
    // its four 32-channel chunks sit at positions q ^ (token % 4), for 16-row
    // tiles (8 tokens x 16 channels) its eight 16-channel units at positions
    // u ^ (token % 8).  At D = 96 the rows are padded instead, to 104 halves
    // (32-row tiles) or 112 (16-row tiles: a stride of 56 banks puts 8
    // consecutive tokens on distinct 8-bank groups); rows stay 16-byte
    // aligned for the stores and 8-byte aligned for the reads.
    static constexpr bool kSwizzleV = D == 128;
    static constexpr int VROW = D == 128 ? D : (TR == 32 ? D + 8 : D + 16);
    static constexpr int kVBytes = D == 128 ? D * (kTile + 8) * 2 : kTile * VROW * 2;
    static constexpr int kWaveBytes = kTile * KS * 2 + kVBytes + kTile * 4;  // K (FP16), V (BF16), alpha_K
    static constexpr int kLdsBytes = kWaves * kWaveBytes;
    // Prologue scratch (aliases the tiles): q scaled into FP16 [32][KS], R_k
    // FP16 [D][KS], q.R_k FP32 [32][QRS], q' FP16 [32][KS], mean dots, row
    // scales and the rows' input exponents.
    static constexpr int QRS = D + 4;
    static constexpr int kQ16Offset = 0;
    static constexpr int kRkOffset = kQ16Offset + 32 * KS * 2;
    static constexpr int kQrawOffset = kRkOffset + D * KS * 2;
    static constexpr int kQpOffset = kQrawOffset + 32 * QRS * 4;
    static constexpr int kQmuOffset = kQpOffset + 32 * KS * 2;
    // Wave merge (aliases the tiles): O [wave][row][MS] FP32 and (m, l) per wave and row.
    static constexpr int MS = D + 4;
    static constexpr int kMlOffset = kWaves * 32 * MS * 4;
    static_assert(kTile * VROW * 2 <= kVBytes, "the row-major V tile fits its region");
    static_assert(kQmuOffset + 128 * 4 <= kLdsBytes, "prologue scratch fits in the tile LDS");
    static_assert(kMlOffset + kWaves * 32 * 2 * 4 <= kLdsBytes, "merge buffer fits in the tile LDS");
    // log2(e) / sqrt(D)
    static constexpr float kScoreScale = D == 128 ? 1.4426950408889634f * 0.08838834764831845f
                                                  : 1.4426950408889634f * 0.10206207261596575f;
};
constexpr float kLog2e = 1.4426950408889634f;
// Pages of one history split at most (its block ids are staged in LDS); the
// host sizes splits so that a split never holds more.
constexpr int kMaxSplitPages = kMultiRowMaxSplitPages;

__device__ __forceinline__ F32x16 mfma(Bf16x8 a, Bf16x8 b, F32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ F32x16 mfma(F16x8 a, F16x8 b, F32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ F32x4 mfma(Bf16x8 a, Bf16x8 b, F32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ F32x4 mfma(F16x8 a, F16x8 b, F32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The O^T accumulator tiles of one lane: D / 32 of 32 x 32 (32-row tiles) or
// D / 16 of 16 x 16 (16-row tiles).
template <int TR>
struct OutTile {
    typedef F32x16 Type;
};
template <>
struct OutTile<16> {
    typedef F32x4 Type;
};

__device__ __forceinline__ uint32_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

__device__ __forceinline__ float f16_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// Round to BF16 (nearest even) and back to FP32.
__device__ __forceinline__ float round_bf16(float x) { return bf16_f32(bf16_rn(x)); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint8_t* page, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(page), (short)0, (int)bytes, 0x00020000);
}

// One record's bytes for the lane's token and 32-channel quarter: 16 code
// bytes (INT4) or 8 (INT2), the FP8 scale and offset byte(s) (one for group
// 32, two for group 16) and, for residual records, the BF16 alpha.
template <int Bits>
struct RecordBytes {
    uint32_t w[Bits];
    uint32_t scale, offset, alpha;
};

template <int Bits, int G>
__device__ __forceinline__ void load_record(__amdgpu_buffer_rsrc_t page, const RecordRegion& r, int page_tokens,
                                            int row, int quarter, bool alpha, RecordBytes<Bits>& out) {
    // A 32-channel quarter holds 4 x Bits code bytes and 32 / G groups.
    const uint32_t codes = (uint32_t)(r.offset + row * r.code_bytes + quarter * 4 * Bits);
    if constexpr (Bits == 4) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(page, codes, 0, kStreamPolicy);
        out.w[0] = v[0]; out.w[1] = v[1]; out.w[2] = v[2]; out.w[3] = v[3];
    } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(page, codes, 0, kStreamPolicy);
        out.w[0] = v[0]; out.w[1] = v[1];
    }
    // The lane's FP8 scale and offset bytes (one group of 32 channels, or two
    // of 16) through the aligned dword holding them, shifted down: the same
    // loads for either group size, so no branch sits between the unit's
    // loads (a conditional load makes the compiler wait for every load in
    // flight, the next unit's included).  Pages are multiples of 16 bytes,
    // so the dword never crosses the page end.
    const uint32_t scales = (uint32_t)(r.offset + page_tokens * r.code_bytes + row * r.groups + quarter * (32 / G));
    const uint32_t offsets = scales + (uint32_t)(page_tokens * r.groups);
    const uint32_t shift = 8u * (scales & 3u);  // offsets sit page_tokens x groups (a multiple of 4) bytes later
    out.scale = __builtin_amdgcn_raw_buffer_load_b32(page, scales & ~3u, 0, 0) >> shift;
    out.offset = __builtin_amdgcn_raw_buffer_load_b32(page, offsets & ~3u, 0, 0) >> shift;
    out.alpha = alpha ? __builtin_amdgcn_raw_buffer_load_b16(
                            page, (uint32_t)(r.offset + page_tokens * (r.code_bytes + 2 * r.groups) + 2 * row), 0, 0)
                      : 0u;
}

// The lane's 32 codes of one record as FP32 code * 2^-9: a code held in a
// byte is that FP8 E4M3 value, so v_cvt_pk_f32_fp8 converts two per
// instruction (the scales carry the 2^9 back).
template <int Bits>
__device__ __forceinline__ void record_codes(const RecordBytes<Bits>& r, float (&c)[32]) {
    if constexpr (Bits == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lo = (int)(r.w[i] & 0x0f0f0f0fu);         // channels 8i + 0, 2, 4, 6
            const int hi = (int)((r.w[i] >> 4) & 0x0f0f0f0fu);  // channels 8i + 1, 3, 5, 7
            const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
            const auto l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            float* a = c + 8 * i;
            a[0] = l01[0]; a[2] = l01[1]; a[4] = l23[0]; a[6] = l23[1];
            a[1] = h01[0]; a[3] = h01[1]; a[5] = h23[0]; a[7] = h23[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float* a = c + 16 * i;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // byte j of part holds channel 4j + k
                const int part = (int)((r.w[i] >> (2 * k)) & 0x03030303u);
                const auto c01 = __builtin_amdgcn_cvt_pk_f32_fp8(part, false);
                const auto c23 = __builtin_amdgcn_cvt_pk_f32_fp8(part, true);
                a[k] = c01[0]; a[4 + k] = c01[1]; a[8 + k] = c23[0]; a[12 + k] = c23[1];
            }
        }
    }
}

// Scale (times 2^9) and offset of the lane's two 16-channel blocks.
template <int G>
__device__ __forceinline__ void record_coefficients(uint32_t scale, uint32_t offset, float (&s)[2], float (&o)[2]) {
    s[0] = __builtin_amdgcn_cvt_f32_fp8((int)scale, 0) * 512.0f;
    o[0] = __builtin_amdgcn_cvt_f32_fp8((int)offset, 0);
    s[1] = G == 32 ? s[0] : __builtin_amdgcn_cvt_f32_fp8((int)scale, 1) * 512.0f;
    o[1] = G == 32 ? o[0] : __builtin_amdgcn_cvt_f32_fp8((int)offset, 1);
}

// One plane's values for the lane's 32 channels in FP32: alpha (c.s+o)_A +
// (c.s+o)_L, evaluated per 16-channel block as c_A (alpha s_A) + (c_L s_L +
// (alpha o_A + o_L)) (two fmas per channel), or (c.s+o)_A without a loop
// record.
template <int BA, int GA, int BL, int GL, bool HasL>
__device__ __forceinline__ void plane_values(const RecordBytes<BA>& a_rec, const RecordBytes<BL>& l_rec, float alpha,
                                             float (&x)[32]) {
    float sa[2], oa[2];
    record_coefficients<GA>(a_rec.scale, a_rec.offset, sa, oa);
    float ca[32];
    record_codes<BA>(a_rec, ca);
    if constexpr (HasL) {
        float sl[2], ol[2];
        record_coefficients<GL>(l_rec.scale, l_rec.offset, sl, ol);
        float cl[32];
        record_codes<BL>(l_rec, cl);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const float a = alpha * sa[b], c = fmaf(alpha, oa[b], ol[b]);
#pragma unroll
            for (int i = 16 * b; i < 16 * b + 16; ++i) x[i] = fmaf(ca[i], a, fmaf(cl[i], sl[b], c));
        }
    } else {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 16 * b; i < 16 * b + 16; ++i) x[i] = fmaf(ca[i], sa[b], oa[b]);
    }
}

typedef float F32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 F16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 Bf16x2 __attribute__((ext_vector_type(2)));
typedef short Short4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) Short4 LdsShort4;

// Two FP32 values rounded (nearest even) to a packed FP16 / BF16 pair, low first.
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(F32x2{a, b}, F16x2));
}
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(F32x2{a, b}, Bf16x2));
}

// ds_read_b64_tr_b16 (gfx950, checked on the device): within each 16 lanes,
// output lane o gets element o % 4 of the 8 bytes addressed by lanes
// o / 4 + 4 p, p = 0..3.
__device__ __forceinline__ Short4 read_transposed(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsShort4*)p);
}

// The LDS writes of a wave before reads of other lanes of the same wave.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The page resources of one 16-token unit (wave-uniform) and the lane's row in the page.
struct UnitPages {
    __amdgpu_buffer_rsrc_t k, v;
    int row;
};

// Anchor mode: K and V of the anchor record and, for a residual loop, the
// loop's record (BA/GA and BL/GL their bits and groups).  Units stream two
// ahead: the loads of the unit two places on are issued before a unit is
// dequantized, so about two units' bytes per wave are in flight while units
// dequantize and the tiles' MFMAs run.
template <int PT, bool HasL, int BA, int GA, int BL, int GL>
struct AnchorDecoder {
    static constexpr bool kAnchorMeanTerm = HasL;  // scores add alpha_K q'.bf16(mu_A)
    struct Bytes {
        RecordBytes<BA> ka, va;
        RecordBytes<BL> kl, vl;
    };
    RecordRegion anchor, residual;
    int lq;
    Bytes ahead1, ahead2;

    __device__ __forceinline__ void fetch(const UnitPages& u, Bytes& b) const {
        load_record<BA, GA>(u.k, anchor, PT, u.row, lq, false, b.ka);
        load_record<BA, GA>(u.v, anchor, PT, u.row, lq, false, b.va);
        if constexpr (HasL) {
            load_record<BL, GL>(u.k, residual, PT, u.row, lq, true, b.kl);
            load_record<BL, GL>(u.v, residual, PT, u.row, lq, true, b.vl);
        }
    }
    __device__ __forceinline__ void prime(const UnitPages& first, const UnitPages& second) {
        fetch(first, ahead1);
        fetch(second, ahead2);
    }
    // Dequantizes the current unit (K, then V, so that only one plane's
    // values are live at a time) after issuing the loads of `two_on`;
    // store_k / store_v take the lane's 32 channels in two halves of 16.
    // Returns the token's K alpha (1 without a loop record).
    template <class StoreK, class StoreV>
    __device__ __forceinline__ float unit(const UnitPages& /*next*/, const UnitPages& two_on, StoreK store_k,
                                          StoreV store_v) {
        const Bytes cur = ahead1;
        ahead1 = ahead2;
        fetch(two_on, ahead2);
        const float alpha_k = HasL ? bf16_f32(cur.kl.alpha) : 1.f;
        {
            float k[32];
            plane_values<BA, GA, BL, GL, HasL>(cur.ka, cur.kl, alpha_k, k);
            store_k(k, k + 16);
        }
        {
            float v[32];
            plane_values<BA, GA, BL, GL, HasL>(cur.va, cur.vl, HasL ? bf16_f32(cur.vl.alpha) : 1.f, v);
            store_v(v, v + 16);
        }
        return alpha_k;
    }
};

// Adjacent mode past loop 0: K and V are the BF16 restore chain over the
// Links records 0..L (rq_chain.h), K adding bf16(mu_r) of records r < L
// (FP32 copies in LDS, `mean`: [Links - 1][kMaxD], or null).  A unit's raw
// bytes of all its records take ~6 registers per record and plane, so units
// stream one ahead: a plane's registers take the next unit's bytes as soon as
// this unit's chain of that plane is built.  Keys are rounded to BF16 (the
// chain's last link) before the FP16 tile takes them, which is exact.
template <int D, int PT, int Links>
struct ChainDecoder {
    static constexpr bool kAnchorMeanTerm = false;
    RecordRegion regs[Links];
    const float* mean;  // [Links - 1][kMaxD] in LDS (zeros without means)
    bool add_mean;
    int lq;
    uint32_t pick_lo, pick_hi;
    ChainRaw k[Links], v[Links];

    __device__ __forceinline__ void fetch_plane(__amdgpu_buffer_rsrc_t page, int row, ChainRaw (&raw)[Links]) const {
#pragma unroll
        for (int r = 0; r < Links; ++r) chain_load<PT, kStreamPolicy, 0>(page, regs[r], row, lq, r > 0, raw[r]);
    }
    __device__ __forceinline__ void prime(const UnitPages& first, const UnitPages& /*second*/) {
        fetch_plane(first.k, first.row, k);
        fetch_plane(first.v, first.row, v);
    }
    // bf16(mu_r) of channel i of the 16 channels from `base` (record r's copy kMaxD floats on).
    __device__ __forceinline__ static auto mean_of(const float* base) {
        return [base](int r, int i) __attribute__((always_inline)) { return base[r * kMaxD + i]; };
    }
    template <class StoreK, class StoreV>
    __device__ __forceinline__ float unit(const UnitPages& next, const UnitPages& /*two_on*/, StoreK store_k,
                                          StoreV store_v) {
        const float* m = mean + 32 * lq;
        float lo[16], hi[16];
        chain_build<0, Links>(k, regs, add_mean, mean_of(m), true, pick_lo, pick_hi, lo);
        chain_build<1, Links>(k, regs, add_mean, mean_of(m + 16), true, pick_lo, pick_hi, hi);
        // The last link's BF16 rounding, one pack per channel pair.
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const uint32_t a = bf16_pack(lo[i], lo[i + 1]), b = bf16_pack(hi[i], hi[i + 1]);
            lo[i] = __uint_as_float(a << 16);
            lo[i + 1] = __uint_as_float(a & 0xffff0000u);
            hi[i] = __uint_as_float(b << 16);
            hi[i + 1] = __uint_as_float(b & 0xffff0000u);
        }
        fetch_plane(next.k, next.row, k);
        store_k(lo, hi);
        chain_build<0, Links>(v, regs, false, mean_of(m), true, pick_lo, pick_hi, lo);
        chain_build<1, Links>(v, regs, false, mean_of(m), true, pick_lo, pick_hi, hi);
        fetch_plane(next.v, next.row, v);
        store_v(lo, hi);
        return 1.f;
    }
};

template <int D, int PT, int TR, class Decoder>
__device__ __forceinline__ void multirow_stream(const MultiRowParams& p, Decoder& dec, uint8_t* lds,
                                                int* split_blocks) {
    using G = Geometry<D, TR>;
    constexpr int KS = G::KS;
    constexpr int QRS = G::QRS;
    const int request = blockIdx.x;
    const int head = blockIdx.y;
    const int split = (int)blockIdx.z % p.splits;
    const int row0 = TR * ((int)blockIdx.z / p.splits);
    const int first = p.query_start_loc[request];
    int n = p.query_start_loc[request + 1] - first;
    if (first < 0 || first >= p.rows) return;  // uniform over the workgroup, before any barrier
    const int new_tokens = p.causal ? n : 1;
    if (n > p.rows - first) n = (int)(p.rows - first);  // rows past the query tensor are not read or written
    if (row0 >= n) return;
    const int seq = p.seq_lens[request];
    int history = seq > new_tokens ? seq - new_tokens : 0;
    // Tokens past the page table are never read.
    if ((int64_t)history > p.max_pages * PT) history = (int)(p.max_pages * PT);
    const int tiles = (history + kTile - 1) / kTile;
    const int per_split = (tiles + p.splits - 1) / p.splits;
    const int tile_begin = split * per_split;
    const int tile_end = tile_begin + per_split < tiles ? tile_begin + per_split : tiles;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // provably wave-uniform
    const int lane = tid & 63;
    const int column = lane & 31;
    const int half = lane >> 5;

    // ---------------------------------------------------------------- q'
    // q' = (q . R_k) * log2(e) / sqrt(D) for the tile's rows, held as FP16
    // q' 2^-e with 2^e the row's power-of-two scale, and the row dots
    // q'.bf16(mu_A) (added per token times alpha_L) and q'.mu_L (the shift of
    // the history scores against the live ones).  The prologue always
    // prepares 32 rows from row0; a 16-row tile uses the first 16.
    uint16_t* q16 = reinterpret_cast<uint16_t*>(lds + G::kQ16Offset);
    uint16_t* r_k = reinterpret_cast<uint16_t*>(lds + G::kRkOffset);
    float* q_raw = reinterpret_cast<float*>(lds + G::kQrawOffset);
    uint16_t* q_p = reinterpret_cast<uint16_t*>(lds + G::kQpOffset);
    float* q_mu = reinterpret_cast<float*>(lds + G::kQmuOffset);  // [0..31] q'.bf16(mu_A), [32..63] q'.mu_L
    float* q_scale = q_mu + 64;                                    // [32] 2^e per row
    float* q_unscale = q_mu + 96;                                  // [32] 2^f per row (the input's scale)
    {
        const int r = tid >> 3, part = tid & 7;  // row, 16-channel part
        const bool part_active = part < G::Parts;
        const int row = row0 + r;
        uint32_t words[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        if (row < n && part_active) {
            const uint2* src = reinterpret_cast<const uint2*>(
                p.query + (int64_t)(first + row) * p.query_stride + head * D + 16 * part);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint2 v = src[i];
                words[2 * i] = v.x;
                words[2 * i + 1] = v.y;
            }
        }
        float x[16];
        float magnitude = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[2 * i] = bf16_f32(words[i] & 0xffffu);
            x[2 * i + 1] = bf16_f32(words[i] >> 16);
            magnitude = fmaxf(magnitude, fmaxf(fabsf(x[2 * i]), fabsf(x[2 * i + 1])));
        }
        if (p.key_rotation) {
            // The row scaled by a power of two 2^-f into [-1, 1]: exact in FP16
            // (a BF16 significand fits), so q.R_k runs on FP16 MFMAs and the
            // product takes 2^f back.
            magnitude = fmaxf(magnitude, __shfl_xor(magnitude, 1));
            magnitude = fmaxf(magnitude, __shfl_xor(magnitude, 2));
            magnitude = fmaxf(magnitude, __shfl_xor(magnitude, 4));
            // (f at most 127, so 2^f stays finite; the scaled row is then within 2.)
            const int f = magnitude > 0.f ? min(__builtin_amdgcn_frexp_expf(magnitude), 127) : 0;
            const float down = ldexpf(1.0f, -f);
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                h[i] = f16_bits(x[2 * i] * down) | (f16_bits(x[2 * i + 1] * down) << 16);
            if (part_active) {
                uint4* dst = reinterpret_cast<uint4*>(&q16[r * KS + 16 * part]);
                dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
                dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
            }
            if (part == 0) q_unscale[r] = ldexpf(1.0f, f);
            // R_k [D][D] FP16 into rows of KS halves, 16 bytes per copy.
            constexpr int kChunks = D / 8;
            const uint4* src = reinterpret_cast<const uint4*>(p.key_rotation + (int64_t)head * D * D);
#pragma unroll
            for (int i = tid; i < D * kChunks; i += kThreads)
                *reinterpret_cast<uint4*>(&r_k[(i / kChunks) * KS + 8 * (i % kChunks)]) = src[i];
        } else if (part_active) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<float4*>(&q_raw[r * QRS + 16 * part + 4 * i]) =
                    make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
        }
    }
    __syncthreads();
    if (p.key_rotation && wave < G::Quarters) {
        // q.R_k on the matrix cores: wave w takes columns 32 w .. 32 w + 31.
        // A: lane l reads scaled row l % 32 at k = 16 m + 8 (l / 32) .. + 7.
        // B: R_k[k][c] for column 32 w + l % 32 and the same k, read
        // transposed from the row-major R_k tile (ds_read_b64_tr_b16: output
        // lane o of 16 gets element o % 4 of the 8 bytes addressed by lanes
        // o / 4 + 4 p, so lane q of a 16-lane group addresses row
        // k0 + q / 4 at columns c0 + 4 (q % 4) .. + 3 and receives column
        // c0 + q of rows k0 .. k0 + 3).
        const int group = lane >> 4, q16_lane = lane & 15;
        const int c0 = 32 * wave + 16 * (group & 1);
        const int k_half = 8 * (group >> 1);
        F32x16 c;
#pragma unroll
        for (int e = 0; e < 16; ++e) c[e] = 0.f;
#pragma unroll
        for (int m = 0; m < G::Parts; ++m) {
            const F16x8 a = *reinterpret_cast<const F16x8*>(&q16[column * KS + 16 * m + 8 * half]);
            const int k0 = 16 * m + k_half;
            const Short4 lo = read_transposed(&r_k[(k0 + (q16_lane >> 2)) * KS + c0 + 4 * (q16_lane & 3)]);
            const Short4 hi = read_transposed(&r_k[(k0 + 4 + (q16_lane >> 2)) * KS + c0 + 4 * (q16_lane & 3)]);
            const F16x8 b = __builtin_bit_cast(F16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            c = mfma(a, b, c);
        }
        // Register e of lane l: row 8 (e / 4) + 4 (l / 32) + e % 4, column 32 w + l % 32.
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int rr = 8 * (e >> 2) + 4 * half + (e & 3);
            q_raw[rr * QRS + 32 * wave + column] = c[e] * q_unscale[rr];
        }
    }
    __syncthreads();
    {
        const int cb = tid & 31, rb = tid >> 5;  // columns 4 cb .. 4 cb + 3, rows 4 rb .. 4 rb + 3
        const bool cb_active = 4 * cb < D;
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = cb_active ? *reinterpret_cast<const float4*>(&q_raw[(4 * rb + i) * QRS + 4 * cb])
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
            acc[i][0] = v.x;
            acc[i][1] = v.y;
            acc[i][2] = v.z;
            acc[i][3] = v.w;
        }
        const float scale = G::kScoreScale;
        float mu_a[4] = {0.f, 0.f, 0.f, 0.f}, mu_l[4] = {0.f, 0.f, 0.f, 0.f};
        if (Decoder::kAnchorMeanTerm && p.key_mean_anchor && cb_active) {
#pragma unroll
            for (int j = 0; j < 4; ++j) mu_a[j] = round_bf16(p.key_mean_anchor[head * D + 4 * cb + j]);
        }
        if (p.key_mean_loop && cb_active) {
#pragma unroll
            for (int j = 0; j < 4; ++j) mu_l[j] = p.key_mean_loop[head * D + 4 * cb + j];
        }
        // Row maxima over the 32 lanes of this half-wave (the same four rows)
        // give each row's power-of-two scale.
        float row_max[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            row_max[i] = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] *= scale;
                row_max[i] = fmaxf(row_max[i], fabsf(acc[i][j]));
            }
        }
#pragma unroll
        for (int d = 16; d; d >>= 1)
#pragma unroll
            for (int i = 0; i < 4; ++i) row_max[i] = fmaxf(row_max[i], __shfl_xor(row_max[i], d));
        float dot_a[4], dot_l[4], row_scale[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // 2^e >= row_max (e from the exponent field; 1 for an all-zero row)
            const int e = row_max[i] > 0.f ? __builtin_amdgcn_frexp_expf(row_max[i]) : 0;
            row_scale[i] = ldexpf(1.0f, e);
            const float inverse = ldexpf(1.0f, -e);
            uint32_t bits[4];
            dot_a[i] = 0.f;
            dot_l[i] = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 h = (_Float16)(acc[i][j] * inverse);
                bits[j] = __builtin_bit_cast(uint16_t, h);
                const float q = (float)h * row_scale[i];
                dot_a[i] = fmaf(q, mu_a[j], dot_a[i]);
                dot_l[i] = fmaf(q, mu_l[j], dot_l[i]);
            }
            if (cb_active)
                *reinterpret_cast<uint2*>(&q_p[(4 * rb + i) * KS + 4 * cb]) =
                    make_uint2(bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16));
        }
        // Sum over the 32 lanes of this half-wave (the same four rows).
#pragma unroll
        for (int d = 16; d; d >>= 1)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dot_a[i] += __shfl_xor(dot_a[i], d);
                dot_l[i] += __shfl_xor(dot_l[i], d);
            }
        if (cb == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q_mu[4 * rb + i] = dot_a[i];
                q_mu[32 + 4 * rb + i] = dot_l[i];
                q_scale[4 * rb + i] = row_scale[i];
            }
        }
    }
    __syncthreads();
    // Q'^T operand (B of S^T = K Q'^T) for the lane's row of the tile,
    // tile_row: chunk m holds channels 16 m + 8 half + e (32-row tiles:
    // tile_row = l % 32, k_group = l / 32) or 32 m + 8 k_group + e (16-row
    // tiles: tile_row = l % 16, k_group = l / 16).
    constexpr int kQChunks = TR == 32 ? G::Parts : D / 32;
    const int tile_row = lane & (TR - 1);
    const int k_group = TR == 32 ? half : lane >> 4;
    F16x8 q_operand[kQChunks];
#pragma unroll
    for (int m = 0; m < kQChunks; ++m)
        q_operand[m] = *reinterpret_cast<const F16x8*>(&q_p[tile_row * KS + (TR == 32 ? 16 : 32) * m + 8 * k_group]);
    const float q_mu_anchor = q_mu[tile_row];
    const float row_scale = q_scale[tile_row];
    if (split == 0 && tid < TR && row0 + tid < n)
        p.row_shift[(int64_t)(first + row0 + tid) * p.heads + head] = q_mu[32 + tid];
    __syncthreads();  // the scratch becomes the tiles

    // ---------------------------------------------------------------- history
    uint16_t* k_tile = reinterpret_cast<uint16_t*>(lds + wave * G::kWaveBytes);
    uint16_t* v_tile = k_tile + kTile * KS;  // [token][VROW] BF16
    float* alpha_tile = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(v_tile) + G::kVBytes);
    // V^T operand reads (ds_read_b64_tr_b16).  32-row tiles: lane 16 g + 4 a
    // + b (g = 2 half + g') addresses token 4 half + a of an 8-token block,
    // channels 32 t + 16 g' + 4 b..+3, and receives channel 32 t + column of
    // tokens 4 half..+3; with the D = 128 swizzle, the 32-channel chunk t
    // sits at position t ^ a.  16-row tiles: lane 16 g + 4 a + b addresses
    // token 4 g + a (and 16 + 4 g + a), channels 16 t + 4 b..+3, and receives
    // channel 16 t + l % 16 of tokens 4 g..+3 (16 + 4 g..+3); with the
    // swizzle, the 16-channel unit t sits at position t ^ (token % 8).
    const int tr_a = (lane >> 2) & 3, tr_b = lane & 3, tr_g = (lane >> 4) & 1;
    const int tr_token = TR == 32 ? 4 * half + tr_a : 4 * k_group + tr_a;
    const int v_lane = TR == 32 ? (G::kSwizzleV ? D * tr_token + 32 * tr_a + 16 * tr_g + 4 * tr_b
                                                : G::VROW * tr_token + 16 * tr_g + 4 * tr_b)
                                : (G::kSwizzleV ? D * tr_token + 16 * (tr_token & 7) + 4 * tr_b
                                                : G::VROW * tr_token + 4 * tr_b);
    auto v_read = [&](int t) __attribute__((always_inline)) {
        constexpr int kStep = TR == 32 ? 32 : 16;
        return G::kSwizzleV ? v_lane ^ (kStep * t) : v_lane + kStep * t;
    };
    const int unit_token = lane >> 2;  // token within a 16-token unit
    const int quarter = lane & 3;      // 32-channel quarter
    const bool quarter_active = quarter < G::Quarters;
    const uint32_t page_bytes = (uint32_t)(PT * p.page_width);
    const int pages = (history + PT - 1) / PT;
    const bool mean_anchor = Decoder::kAnchorMeanTerm && p.key_mean_anchor != nullptr;

    // The split's block ids, once, into LDS (-1 past the history or when invalid).
    const int first_page = tile_begin * kTile / PT;
    int split_pages = tile_end > tile_begin ? ((tile_end * kTile + PT - 1) / PT - first_page) : 0;
    if (split_pages > kMaxSplitPages) split_pages = kMaxSplitPages;  // pages past it read as zeros
    for (int i = tid; i < split_pages; i += kThreads) {
        const int page = first_page + i;
        int block = page < pages ? p.block_table[(int64_t)request * p.block_table_stride + page] : -1;
        split_blocks[i] = (block >= 0 && block < p.num_blocks) ? block : -1;
    }
    __syncthreads();

    // The page resources of one 16-token unit (empty past the history).
    auto unit_pages = [&](int unit_first) __attribute__((always_inline)) {
        const int index = unit_first / PT - first_page;
        // One unit per wave: the block id is wave-uniform, and readfirstlane
        // keeps the page resources in SGPRs (no waterfall loop per load).
        const int block = __builtin_amdgcn_readfirstlane(
            (unit_first < history && index < split_pages) ? split_blocks[index] : -1);
        const uint8_t* k_page = p.cache + ((int64_t)(block >= 0 ? block : 0) * p.heads + head) * page_bytes;
        const uint32_t bytes = block >= 0 ? page_bytes : 0u;
        return UnitPages{page_rsrc(k_page, bytes), page_rsrc(k_page + p.plane_stride, bytes),
                         unit_first % PT + unit_token};
    };

    // O^T: tile t of a 32-row tile holds channels 32 t.. (register r: channel
    // 32 t + 8 (r / 4) + 4 half + r % 4 of row tile_row), of a 16-row tile
    // channels 16 t.. (register r: channel 16 t + 4 k_group + r).
    constexpr int kOutTiles = TR == 32 ? G::Quarters : G::Parts;
    constexpr int kOutRegs = TR == 32 ? 16 : 4;
    typename OutTile<TR>::Type out[kOutTiles];
#pragma unroll
    for (int t = 0; t < kOutTiles; ++t)
#pragma unroll
        for (int r = 0; r < kOutRegs; ++r) out[t][r] = 0.f;
    float running_max = -__builtin_inff();
    float running_sum = 0.f;

    // A wave's units are the two halves of its tiles tile_begin + wave +
    // kWaves k.  The fetches carry no condition (units past the split read
    // zeros through an empty resource), which keeps the compiler's count of
    // loads in flight exact.
    const int first_tile = tile_begin + wave;
    dec.prime(unit_pages(kTile * first_tile), unit_pages(kTile * first_tile + 16));
    // The wave's priority falls as its tiles advance (StreamPriority), which
    // keeps the two workgroups of a compute unit level; it replaced a raised
    // priority over each tile's MFMAs and softmax (residual call 129.3 ->
    // 122.5 us at 16 requests x 16 rows x 8k, A/B on one box).
    const int wave_tiles = first_tile < tile_end ? (tile_end - first_tile + kWaves - 1) / kWaves : 0;
    const StreamPriority priority(wave_tiles, p.stream_priority != 0);
    int step = 0;
    for (int tile = first_tile; tile < tile_end; tile += kWaves, ++step) {
        priority.set(step);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int local = 16 * u + unit_token;
            const bool valid = kTile * tile + local < history;
            // Whole unit inside the history (wave-uniform): nothing to mask.
            const bool unit_valid = kTile * tile + 16 * u + 16 <= history;
            // The unit after this one, and the one after that.
            const int next_first = u == 0 ? kTile * tile + 16 : kTile * (tile + kWaves);
            const int two_on_first = kTile * (tile + kWaves) + 16 * u;
            auto store_k = [&](const float* lo, const float* hi) __attribute__((always_inline)) {
                uint32_t kw[16];
                // No mask: the scores of tokens past the history become -inf below.
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    kw[c] = pack_f16(lo[2 * c], lo[2 * c + 1]);
                    kw[8 + c] = pack_f16(hi[2 * c], hi[2 * c + 1]);
                }
                if (quarter_active) {
                    uint4* k_dst = reinterpret_cast<uint4*>(&k_tile[local * KS + 32 * quarter]);
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        k_dst[c] = make_uint4(kw[4 * c], kw[4 * c + 1], kw[4 * c + 2], kw[4 * c + 3]);
                }
            };
            auto store_v = [&](const float* lo, const float* hi) __attribute__((always_inline)) {
                uint32_t vw[16];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    vw[c] = pack_bf16(lo[2 * c], lo[2 * c + 1]);
                    vw[8 + c] = pack_bf16(hi[2 * c], hi[2 * c + 1]);
                }
                // Slots past the history may hold any bytes (P is zero there,
                // but 0 x NaN is not): zero them in a unit that reaches past it.
                if (!unit_valid) {
                    asm volatile("");
#pragma unroll
                    for (int c = 0; c < 16; ++c) vw[c] = valid ? vw[c] : 0u;
                }
                if (quarter_active) {
                    if (TR == 16 && G::kSwizzleV) {
                        // The lane's two 16-channel units 2 quarter and
                        // 2 quarter + 1 at positions unit ^ (token % 8).
                        uint4* lo_dst = reinterpret_cast<uint4*>(&v_tile[local * G::VROW + 16 * ((2 * quarter) ^ (local & 7))]);
                        uint4* hi_dst =
                            reinterpret_cast<uint4*>(&v_tile[local * G::VROW + 16 * ((2 * quarter + 1) ^ (local & 7))]);
                        lo_dst[0] = make_uint4(vw[0], vw[1], vw[2], vw[3]);
                        lo_dst[1] = make_uint4(vw[4], vw[5], vw[6], vw[7]);
                        hi_dst[0] = make_uint4(vw[8], vw[9], vw[10], vw[11]);
                        hi_dst[1] = make_uint4(vw[12], vw[13], vw[14], vw[15]);
                    } else {
                        // Row-major V: the lane's 4 chunks of 8 channels (at D =
                        // 128 at chunk positions 4 (quarter ^ (token % 4)) + i).
                        const int chunk = G::kSwizzleV ? (quarter ^ (local & 3)) : quarter;
                        uint4* v_dst = reinterpret_cast<uint4*>(&v_tile[local * G::VROW + 32 * chunk]);
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            v_dst[c] = make_uint4(vw[4 * c], vw[4 * c + 1], vw[4 * c + 2], vw[4 * c + 3]);
                    }
                }
            };
            const float alpha_k = dec.unit(unit_pages(next_first), unit_pages(two_on_first), store_k, store_v);
            if (quarter == 0) alpha_tile[local] = alpha_k;
        }
        wave_sync();

        if constexpr (TR == 16) {
            // S^T in two 16-token halves: register r of s[h] holds token
            // 16 h + 4 k_group + r against row tile_row (the A operand's lane
            // l % 16 takes token 16 h + l % 16).
            F32x4 s[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s[h][r] = 0.f;
                const uint16_t* k_row = &k_tile[(16 * h + tile_row) * KS + 8 * k_group];
#pragma unroll
                for (int m = 0; m < kQChunks; ++m)
                    s[h] = mfma(*reinterpret_cast<const F16x8*>(k_row + 32 * m), q_operand[m], s[h]);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int local = 16 * h + 4 * k_group + r;
                    float x = s[h][r] * row_scale;
                    if (mean_anchor) x = fmaf(alpha_tile[local], q_mu_anchor, x);
                    s[h][r] = x;
                }
            if (kTile * tile + kTile > history) {
                asm volatile("");
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        s[h][r] = kTile * tile + 16 * h + 4 * k_group + r < history ? s[h][r] : -__builtin_inff();
            }
            // The row's scores sit in lanes l % 16 + 16 k_group.
            float tile_max = -__builtin_inff();
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) tile_max = fmaxf(tile_max, s[h][r]);
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
            const float new_max = fmaxf(running_max, tile_max);
            const float base = new_max == -__builtin_inff() ? 0.f : new_max;
            const float rescale = __builtin_amdgcn_exp2f(running_max - base);
            running_max = new_max;
            // P^T in BF16 as the B operand of O^T += V^T P^T: k-slot
            // 8 k_group + e is token 4 k_group + e (s[0][e]) for e < 4 and
            // 16 + 4 k_group + e - 4 (s[1][e - 4]) for e >= 4.
            float tile_sum = 0.f;
            Bf16x8 p_operand;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float w = __builtin_amdgcn_exp2f(s[h][r] - base);
                    p_operand[4 * h + r] = (__bf16)w;
                    tile_sum += w;
                }
            tile_sum += __shfl_xor(tile_sum, 16);
            tile_sum += __shfl_xor(tile_sum, 32);
            running_sum = running_sum * rescale + tile_sum;
            if (!__all(rescale == 1.0f)) {
#pragma unroll
                for (int t = 0; t < kOutTiles; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) out[t][r] *= rescale;
            }
#pragma unroll
            for (int t = 0; t < kOutTiles; ++t) {
                // Tokens 4 k_group + 0..3 and 16 + 4 k_group + 0..3, as P^T's k-slots.
                const Short4 lo = read_transposed(v_tile + v_read(t));
                const Short4 hi = read_transposed(v_tile + 16 * G::VROW + v_read(t));
                out[t] = mfma(__builtin_bit_cast(Bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)),
                              p_operand, out[t]);
            }
        } else {
            // S^T: register r of lane l holds token 8 (r / 4) + 4 half + r % 4 against row `column`.
            F32x16 s;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.f;
            const uint16_t* k_row = &k_tile[column * KS + 8 * half];
#pragma unroll
            for (int m = 0; m < G::Parts; ++m)
                s = mfma(*reinterpret_cast<const F16x8*>(k_row + 16 * m), q_operand[m], s);

#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int local = 8 * (r >> 2) + 4 * half + (r & 3);
                float x = s[r] * row_scale;
                if (mean_anchor) x = fmaf(alpha_tile[local], q_mu_anchor, x);
                s[r] = x;
            }
            // Tokens past the history score -inf (only in the tile that reaches past it).
            if (kTile * tile + kTile > history) {
                asm volatile("");
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    s[r] = kTile * tile + 8 * (r >> 2) + 4 * half + (r & 3) < history ? s[r] : -__builtin_inff();
            }
            float tile_max = -__builtin_inff();
#pragma unroll
            for (int r = 0; r < 16; ++r) tile_max = fmaxf(tile_max, s[r]);
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
            const float new_max = fmaxf(running_max, tile_max);
            const float base = new_max == -__builtin_inff() ? 0.f : new_max;
            const float rescale = __builtin_amdgcn_exp2f(running_max - base);
            running_max = new_max;
            // P^T in BF16 as the B operand of O^T += V^T P^T: step j takes
            // registers 8j..8j+7, i.e. k-slot (half, e) is token
            // 16 j + 4 half + e + (e >= 4 ? 4 : 0).
            float tile_sum = 0.f;
            Bf16x8 p_operand[2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float w = __builtin_amdgcn_exp2f(s[8 * j + e] - base);
                    p_operand[j][e] = (__bf16)w;
                    tile_sum += w;
                }
            tile_sum += __shfl_xor(tile_sum, 32);
            running_sum = running_sum * rescale + tile_sum;
            if (!__all(rescale == 1.0f)) {
#pragma unroll
                for (int t = 0; t < G::Quarters; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) out[t][r] *= rescale;
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint16_t* v_rows = v_tile + 16 * j * G::VROW;
#pragma unroll
                for (int t = 0; t < G::Quarters; ++t) {
                    // Tokens 4 half + 0..3 and 4 half + 8..11 of the 16, as P^T's k-slots.
                    const Short4 lo = read_transposed(v_rows + v_read(t));
                    const Short4 hi = read_transposed(v_rows + 8 * G::VROW + v_read(t));
                    out[t] = mfma(__builtin_bit_cast(Bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)),
                                  p_operand[j], out[t]);
                }
            }
        }
        wave_sync();  // the next tile overwrites this one
    }
    __builtin_amdgcn_s_setprio(0);

    // ---------------------------------------------------------------- wave merge
    __syncthreads();  // the merge buffer aliases every wave's tiles
    constexpr int MS = G::MS;
    float* merge_o = reinterpret_cast<float*>(lds);
    float* merge_ml = reinterpret_cast<float*>(lds + G::kMlOffset);
    if constexpr (TR == 16) {
#pragma unroll
        for (int t = 0; t < kOutTiles; ++t)
            *reinterpret_cast<float4*>(&merge_o[(wave * 32 + tile_row) * MS + 16 * t + 4 * k_group]) =
                make_float4(out[t][0], out[t][1], out[t][2], out[t][3]);
    } else {
#pragma unroll
        for (int t = 0; t < kOutTiles; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(&merge_o[(wave * 32 + column) * MS + 32 * t + 8 * g + 4 * half]) =
                    make_float4(out[t][4 * g], out[t][4 * g + 1], out[t][4 * g + 2], out[t][4 * g + 3]);
    }
    if (k_group == 0) {
        merge_ml[(wave * 32 + tile_row) * 2] = running_max;
        merge_ml[(wave * 32 + tile_row) * 2 + 1] = running_sum;
    }
    __syncthreads();
    const int r = tid >> 3, chunk = tid & 7;  // row, 16-channel chunk
    if (r < TR) {
        float m_w[kWaves], total_max = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            m_w[w] = merge_ml[(w * 32 + r) * 2];
            total_max = fmaxf(total_max, m_w[w]);
        }
        float l = 0.f;
        float o[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) o[c] = 0.f;
        const bool chunk_active = chunk < G::Parts;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            if (m_w[w] == -__builtin_inff()) continue;
            const float weight = __builtin_amdgcn_exp2f(m_w[w] - total_max);
            l = fmaf(merge_ml[(w * 32 + r) * 2 + 1], weight, l);
            const float* src = &merge_o[(w * 32 + r) * MS + 16 * (chunk_active ? chunk : 0)];
#pragma unroll
            for (int c = 0; c < 16; ++c) o[c] = fmaf(src[c], weight, o[c]);
        }
        if (row0 + r < n) {
            float* entry = p.partials +
                           (((int64_t)(first + row0 + r) * p.heads + head) * p.splits + split) * kMultiRowEntry;
            if (chunk == 0) *reinterpret_cast<float4*>(entry) = make_float4(total_max, l, 0.f, 0.f);
            if (chunk_active) {
                float4* dst = reinterpret_cast<float4*>(entry + 4 + 16 * chunk);
#pragma unroll
                for (int c = 0; c < 4; ++c) dst[c] = make_float4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
            }
        }
    }
}

template <int D, int PT, int TR, bool HasL, int BA, int GA, int BL, int GL>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void multirow_stream_kernel(MultiRowParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[Geometry<D, TR>::kLdsBytes];
    __shared__ int split_blocks[kMaxSplitPages];  // block ids of the split's pages
    AnchorDecoder<PT, HasL, BA, GA, BL, GL> dec;
    dec.anchor = p.anchor;
    dec.residual = p.residual;
    const int quarter = threadIdx.x & 3;
    dec.lq = quarter < Geometry<D>::Quarters ? quarter : 0;
    multirow_stream<D, PT, TR>(p, dec, lds, split_blocks);
}

template <int D, int PT, int TR, int Links>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void multirow_chain_kernel(MultiRowParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[Geometry<D, TR>::kLdsBytes];
    __shared__ int split_blocks[kMaxSplitPages];  // block ids of the split's pages
    // bf16(mu_r) of records 0 .. L - 1 (the K plane's chain), FP32.
    __shared__ __attribute__((aligned(16))) float mean_lds[Links - 1][kMaxD];
    const int head = blockIdx.y;
    const bool has_mean = p.key_mean_all != nullptr;
    for (int i = threadIdx.x; i < (Links - 1) * kMaxD; i += kThreads) {
        const int r = i / kMaxD, c = i % kMaxD;
        mean_lds[r][c] = (has_mean && c < D) ? bf16_f32(bf16_rn(p.key_mean_all[((int64_t)r * p.heads + head) * D + c]))
                                             : 0.f;
    }
    // (The stream's first barrier orders these stores before any read.)
    ChainDecoder<D, PT, Links> dec;
#pragma unroll
    for (int r = 0; r < Links; ++r) dec.regs[r] = p.chain[r];
    dec.mean = &mean_lds[0][0];
    dec.add_mean = has_mean;
    const int quarter = threadIdx.x & 3;
    dec.lq = quarter < Geometry<D>::Quarters ? quarter : 0;
    // The pairs (1, 0) and (0, 1) of the mean add, in registers.
    uint32_t pick_lo = 0x00003f80u, pick_hi = 0x3f800000u;
    asm("" : "+v"(pick_lo), "+v"(pick_hi));
    dec.pick_lo = pick_lo;
    dec.pick_hi = pick_hi;
    multirow_stream<D, PT, TR>(p, dec, lds, split_blocks);
}

// ---------------------------------------------------------------- finish

// Row strides of the finish kernel's tiles for head dim D: BF16/FP16 rows
// (halves) and the rotated history [row][channel] (FP32).  Region A holds
// the merged rows' FP16 parts for the rotation, then the causal tiles;
// region B the rotated history.
template <int D>
struct FinishGeometry {
    static constexpr int Parts = D / 16;
    static constexpr int FS = D + 8;
    static constexpr int OS = D + 4;
    static constexpr int kRotationBytes = 2 * 32 * FS * 2;                  // high and low FP16 parts
    static constexpr int kCausalBytes = 3 * 32 * FS * 2 + 32 * 33 * 4;     // q, k, v tiles and probabilities
    static constexpr int kRegionABytes = kRotationBytes > kCausalBytes ? kRotationBytes : kCausalBytes;
    static constexpr int kRegionBFloats = 32 * OS;
};

__device__ __forceinline__ float row8_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 1));
    x = fmaxf(x, __shfl_xor(x, 2));
    return fmaxf(x, __shfl_xor(x, 4));
}

__device__ __forceinline__ float row8_sum(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    return x + __shfl_xor(x, 4);
}

// Whether rows of a BF16 tensor at `base` with row stride `stride`
// (elements) start on 16-byte boundaries.  The boundary guarantees 8 bytes
// for queries and keys and 2 bytes for values and outputs.
__device__ __forceinline__ bool aligned_rows(const void* base, int64_t stride) {
    return (reinterpret_cast<uintptr_t>(base) & 15u) == 0 && (stride & 7) == 0;
}

// 16 consecutive BF16 values at `src` (a 32-byte aligned offset of an
// aligned_rows tensor when `vec`) as two 16-byte words.
__device__ __forceinline__ void load_halves16(const uint16_t* src, bool vec, uint4 (&w)[2]) {
    if (vec) {
        w[0] = reinterpret_cast<const uint4*>(src)[0];
        w[1] = reinterpret_cast<const uint4*>(src)[1];
    } else {
        uint32_t x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = (uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 16);
        w[0] = make_uint4(x[0], x[1], x[2], x[3]);
        w[1] = make_uint4(x[4], x[5], x[6], x[7]);
    }
}

// Eight BF16 values of a 16-byte word as FP32.
__device__ __forceinline__ void widen_bf16(uint4 w, float* x) {
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = bf16_f32(v[i] & 0xffffu);
        x[2 * i + 1] = bf16_f32(v[i] >> 16);
    }
}

// One (request, head, 32-row tile) per 256-thread workgroup.  Thread t takes
// row t / 8 of the tile and part p = t % 8 of it: the 16 channels
// 16p..16p+15 of the merge, the query-key dots, the live values and the
// output (parts p < D / 16), and the 4 tokens 4p..4p+3 of a live chunk's
// scores.  The eight threads of a row are adjacent lanes of one wave.
//   1. merge the splits' partials (m, l, O) of each row (log2 units);
//   2. rotate the tile's 32 merged rows by R_v^T on the matrix cores (wave w
//      computes output channels 32 w .. 32 w + 31);
//   3. add the live tokens: in decode semantics the row's own token; in
//      causal semantics the request's new tokens j <= row, 32 at a time with
//      an online softmax over the rows' (m, l, O);
//   4. write O / l in BF16.
template <int D>
__global__ __launch_bounds__(kThreads) void multirow_finish_kernel(MultiRowParams p) {
    using G = FinishGeometry<D>;
    constexpr int FS = G::FS;
    constexpr int OS = G::OS;
    __shared__ __attribute__((aligned(16))) uint8_t region_a[G::kRegionABytes];
    __shared__ __attribute__((aligned(16))) float region_b[G::kRegionBFloats];
    float* hist_rot = region_b;
    uint16_t* q_tile = reinterpret_cast<uint16_t*>(region_a);  // causal: the rows' queries
    uint16_t* k_tile = q_tile + 32 * FS;                      // causal: 32 live keys
    uint16_t* v_tile = k_tile + 32 * FS;                      // causal: their values
    float* probs = reinterpret_cast<float*>(v_tile + 32 * FS);
    const int request = blockIdx.x;
    const int head = blockIdx.y;
    const int row0 = 32 * (int)blockIdx.z;
    const int tid = threadIdx.x;
    const int r = tid >> 3, part = tid & 7;
    const bool part_active = part < G::Parts;
    const bool rotate = p.value_rotation != nullptr;
    const int wave = tid >> 6;
    const bool rotation_wave = wave < D / 32;

    // R_v as the B operand of the rotation MFMAs (16-byte loads issued
    // before the request lookup, so that the two round trips overlap): wave
    // w computes output channels 32 w .. 32 w + 31, lane l takes row
    // 32 w + l % 32 of R_v at features 16 m + 8 (l / 32) .. + 7.
    const int lane = tid & 63;
    F16x8 rv[G::Parts];
    if (rotate && rotation_wave) {
        const uint16_t* src = p.value_rotation + ((int64_t)head * D + 32 * wave + (lane & 31)) * D + 8 * (lane >> 5);
#pragma unroll
        for (int m = 0; m < G::Parts; ++m) rv[m] = *reinterpret_cast<const F16x8*>(src + 16 * m);
    }
    const int first = p.query_start_loc[request];
    int n = p.query_start_loc[request + 1] - first;
    if (first < 0 || first >= p.rows) return;  // uniform over the workgroup, before any barrier
    if (n > p.rows - first) n = (int)(p.rows - first);
    if (row0 >= n) return;

    const bool valid = row0 + r < n;
    const int64_t row = (int64_t)first + row0 + (valid ? r : 0);
    const float scale = Geometry<D>::kScoreScale;  // log2(e) / sqrt(D)
    // The part's 16 channels of a token row (part 0's for an inactive part,
    // whose values are never used).
    const int64_t channels = (int64_t)head * D + 16 * (part_active ? part : 0);

    // The row's query (and, in decode semantics, its own key and value).
    const bool q_vec = aligned_rows(p.query, p.query_stride), k_vec = aligned_rows(p.key, p.key_stride),
               v_vec = aligned_rows(p.value, p.value_stride);
    uint4 qw[2], kw[2], vw[2];
    load_halves16(p.query + row * p.query_stride + channels, q_vec, qw);
    if (!part_active) qw[0] = qw[1] = make_uint4(0u, 0u, 0u, 0u);  // no share of the row's dots
    if (!p.causal) {
        load_halves16(p.key + row * p.key_stride + channels, k_vec, kw);
        load_halves16(p.value + row * p.value_stride + channels, v_vec, vw);
    }
    const float shift = p.row_shift[row * p.heads + head];

    // 1. Merge the splits online, four at a time: every load of a batch is
    // issued before any of its arithmetic (split indices past the last are
    // clamped and weighted zero, so no load sits behind a branch).  Rows past
    // the request merge nothing.
    float m = -__builtin_inff(), l = 0.f, acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    const float* entries = p.partials + (row * p.heads + head) * p.splits * kMultiRowEntry;
    const int entry_part = part_active ? part : 0;
    for (int s0 = 0; s0 < p.splits; s0 += 4) {
        float2 ml[4];
        float4 ox[4][4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int s = s0 + b < p.splits ? s0 + b : p.splits - 1;
            const float* e = entries + s * kMultiRowEntry;
            ml[b] = *reinterpret_cast<const float2*>(e);
#pragma unroll
            for (int c = 0; c < 4; ++c) ox[b][c] = reinterpret_cast<const float4*>(e + 4 + 16 * entry_part)[c];
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float ms = (valid && s0 + b < p.splits) ? ml[b].x : -__builtin_inff();
            const float new_max = fmaxf(m, ms);
            const float base = new_max == -__builtin_inff() ? 0.f : new_max;
            const float keep = __builtin_amdgcn_exp2f(m - base), w = __builtin_amdgcn_exp2f(ms - base);
            m = new_max;
            l = fmaf(l, keep, ml[b].y * w);
            const float x[16] = {ox[b][0].x, ox[b][0].y, ox[b][0].z, ox[b][0].w, ox[b][1].x, ox[b][1].y,
                                 ox[b][1].z, ox[b][1].w, ox[b][2].x, ox[b][2].y, ox[b][2].z, ox[b][2].w,
                                 ox[b][3].x, ox[b][3].y, ox[b][3].z, ox[b][3].w};
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = fmaf(acc[i], keep, x[i] * w);
        }
    }

    // 2. hist . R_v^T for the tile's 32 rows on the matrix cores: the merged
    // rows divided by their sums (convex combinations of values, within the
    // FP16 range) as FP16 high and low parts (~22 significant bits), times
    // R_v (FP16), FP32 accumulation; the sums are multiplied back.
    if (rotate) {
        uint16_t* high = reinterpret_cast<uint16_t*>(region_a);  // [row][FS]
        uint16_t* low = high + 32 * FS;
        const float inverse = l > 0.f ? 1.0f / l : 0.f;
        uint32_t hw[8], lw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x0 = acc[2 * i] * inverse, x1 = acc[2 * i + 1] * inverse;
            const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
            const _Float16 r0 = (_Float16)(x0 - (float)h0), r1 = (_Float16)(x1 - (float)h1);
            hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, r0) | ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
        }
        if (part_active) {
            uint4* hd = reinterpret_cast<uint4*>(&high[r * FS + 16 * part]);
            uint4* ld = reinterpret_cast<uint4*>(&low[r * FS + 16 * part]);
            hd[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
            hd[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
            ld[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            ld[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
        }
        __syncthreads();
        if (rotation_wave) {
            // A operand: lane l takes merged row l % 32 at features 16 m + 8 (l / 32) .. + 7.
            F32x16 rotated;
#pragma unroll
            for (int e = 0; e < 16; ++e) rotated[e] = 0.f;
            const int a_offset = (lane & 31) * FS + 8 * (lane >> 5);
#pragma unroll
            for (int mm = 0; mm < G::Parts; ++mm) {
                rotated = mfma(*reinterpret_cast<const F16x8*>(&high[a_offset + 16 * mm]), rv[mm], rotated);
                rotated = mfma(*reinterpret_cast<const F16x8*>(&low[a_offset + 16 * mm]), rv[mm], rotated);
            }
            // Register e of lane l: row 8 (e / 4) + 4 (l / 32) + e % 4, channel 32 w + l % 32.
#pragma unroll
            for (int e = 0; e < 16; ++e)
                hist_rot[(8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * OS + 32 * wave + (lane & 31)] = rotated[e];
        }
        __syncthreads();
        if (part_active) {
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const float4 x = *reinterpret_cast<const float4*>(&hist_rot[r * OS + 16 * part + 4 * c4]);
                acc[4 * c4] = x.x * l;
                acc[4 * c4 + 1] = x.y * l;
                acc[4 * c4 + 2] = x.z * l;
                acc[4 * c4 + 3] = x.w * l;
            }
        }
    }

    // 3. Live tokens.
    float q[16];
    widen_bf16(qw[0], q);
    widen_bf16(qw[1], q + 8);
    if (!p.causal) {
        // The row's own token.
        float k[16], v[16];
        widen_bf16(kw[0], k);
        widen_bf16(kw[1], k + 8);
        widen_bf16(vw[0], v);
        widen_bf16(vw[1], v + 8);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) dot = fmaf(q[i], k[i], dot);
        const float score = row8_sum(dot) * scale - shift;
        const float total_max = fmaxf(m, score);
        const float hist_weight = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - total_max);
        const float live = __builtin_amdgcn_exp2f(score - total_max);
        l = fmaf(l, hist_weight, live);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = fmaf(live, v[i], acc[i] * hist_weight);
    } else {
        // The request's new tokens 0 .. row0 + r, in chunks of 32 shared by the tile's rows.
        if (part_active) {
            uint4* dst = reinterpret_cast<uint4*>(&q_tile[r * FS + 16 * part]);
            dst[0] = qw[0];
            dst[1] = qw[1];
        }
        const int live_end = n < row0 + 32 ? n : row0 + 32;
        for (int c0 = 0; c0 < live_end; c0 += 32) {
            __syncthreads();  // the previous chunk's reads are done
            if (part_active) {
                // Thread (r, part) stages the part's channels of live token c0 + r.
                const int j = c0 + r;
                uint4 kx[2] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)}, vx[2] = {kx[0], kx[1]};
                if (j < n) {
                    load_halves16(p.key + ((int64_t)first + j) * p.key_stride + channels, k_vec, kx);
                    load_halves16(p.value + ((int64_t)first + j) * p.value_stride + channels, v_vec, vx);
                }
                uint4* kd = reinterpret_cast<uint4*>(&k_tile[r * FS + 16 * part]);
                uint4* vd = reinterpret_cast<uint4*>(&v_tile[r * FS + 16 * part]);
                kd[0] = kx[0];
                kd[1] = kx[1];
                vd[0] = vx[0];
                vd[1] = vx[1];
            }
            __syncthreads();
            // Scores of row r against tokens c0 + 4 part .. + 3.
            float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
            for (int d = 0; d < D; d += 8) {
                float qd[8];
                widen_bf16(*reinterpret_cast<const uint4*>(&q_tile[r * FS + d]), qd);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float kd[8];
                    widen_bf16(*reinterpret_cast<const uint4*>(&k_tile[(4 * part + i) * FS + d]), kd);
#pragma unroll
                    for (int e = 0; e < 8; ++e) s[i] = fmaf(qd[e], kd[e], s[i]);
                }
            }
            float chunk_max = -__builtin_inff();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = c0 + 4 * part + i;
                s[i] = (valid && j <= row0 + r && j < n) ? s[i] * scale - shift : -__builtin_inff();
                chunk_max = fmaxf(chunk_max, s[i]);
            }
            const float new_max = fmaxf(m, row8_max(chunk_max));
            const float base = new_max == -__builtin_inff() ? 0.f : new_max;
            const float rescale = __builtin_amdgcn_exp2f(m - base);
            m = new_max;
            float chunk_sum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float w = __builtin_amdgcn_exp2f(s[i] - base);
                probs[r * 33 + 4 * part + i] = w;
                chunk_sum += w;
            }
            l = fmaf(l, rescale, row8_sum(chunk_sum));
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] *= rescale;
            wave_sync();  // row r's probabilities come from lanes of this wave
            if (part_active) {
#pragma unroll 4
                for (int jj = 0; jj < 32; ++jj) {
                    const float w = probs[r * 33 + jj];
                    float vd[16];
                    widen_bf16(*reinterpret_cast<const uint4*>(&v_tile[jj * FS + 16 * part]), vd);
                    widen_bf16(*reinterpret_cast<const uint4*>(&v_tile[jj * FS + 16 * part + 8]), vd + 8);
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[i] = fmaf(w, vd[i], acc[i]);
                }
            }
        }
    }

    // 4. Output.
    if (valid && part_active) {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = bf16_rn(acc[2 * i] / l) | (bf16_rn(acc[2 * i + 1] / l) << 16);
        uint16_t* out = p.output + row * p.output_stride + channels;
        if (aligned_rows(p.output, p.output_stride)) {
            reinterpret_cast<uint4*>(out)[0] = make_uint4(w[0], w[1], w[2], w[3]);
            reinterpret_cast<uint4*>(out)[1] = make_uint4(w[4], w[5], w[6], w[7]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                out[2 * i] = (uint16_t)(w[i] & 0xffffu);
                out[2 * i + 1] = (uint16_t)(w[i] >> 16);
            }
        }
    }
}

// Rows per stream tile: 16 when the call's requests average 16 rows or
// fewer (and the grid's z extent allows it), else 32.  The finish kernel
// always takes 32-row tiles (the partials are per row).
int stream_tile_rows(const MultiRowParams& p) {
    const int64_t tiles16 = (p.rows + 15) / 16;
    return (p.rows <= 16 * p.requests && (int64_t)p.splits * tiles16 <= 65535) ? 16 : 32;
}

template <int TR>
dim3 stream_grid(const MultiRowParams& p) {
    return dim3((unsigned)p.requests, (unsigned)p.heads, (unsigned)(p.splits * ((p.rows + TR - 1) / TR)));
}

// The launch parameters with stream_priority set: whether the grid's active
// workgroups, about requests x heads x splits x the average request's row
// tiles (the others exit at once), fit the device at once.
template <int TR>
MultiRowParams with_priority(const MultiRowParams& params, int per_cu) {
    MultiRowParams p = params;
    const int64_t average_rows = p.requests > 0 ? p.rows / p.requests : p.rows;
    const int64_t average_tiles = average_rows > TR ? (average_rows + TR - 1) / TR : 1;
    const int64_t active = p.requests * p.heads * p.splits * average_tiles;
    p.stream_priority = active <= (int64_t)per_cu * p.compute_units ? 1 : 0;
    return p;
}

template <int D, int PT, int TR, bool HasL, int BA, int GA, int BL, int GL>
void launch_one(const MultiRowParams& p, hipStream_t stream) {
    const auto kernel = multirow_stream_kernel<D, PT, TR, HasL, BA, GA, BL, GL>;
    static const int per_cu = resident_per_cu(reinterpret_cast<const void*>(kernel), kThreads);
    hipLaunchKernelGGL(kernel, stream_grid<TR>(p), dim3(kThreads), 0, stream, with_priority<TR>(p, per_cu));
}

template <int D, int PT, int TR, int Links>
void launch_chain(const MultiRowParams& p, hipStream_t stream) {
    const auto kernel = multirow_chain_kernel<D, PT, TR, Links>;
    static const int per_cu = resident_per_cu(reinterpret_cast<const void*>(kernel), kThreads);
    hipLaunchKernelGGL(kernel, stream_grid<TR>(p), dim3(kThreads), 0, stream, with_priority<TR>(p, per_cu));
}

template <int D, int PT, int TR, int BA, int GA, int BL>
void launch_residual_group(const MultiRowParams& p, hipStream_t stream) {
    if (p.residual.group == 32)
        launch_one<D, PT, TR, true, BA, GA, BL, 32>(p, stream);
    else
        launch_one<D, PT, TR, true, BA, GA, BL, 16>(p, stream);
}

template <int D, int PT, int TR, int BA, int GA>
void launch_anchor(const MultiRowParams& p, hipStream_t stream) {
    if (!p.has_residual)
        launch_one<D, PT, TR, false, BA, GA, 2, 32>(p, stream);
    else if (p.residual.bits == 2)
        launch_residual_group<D, PT, TR, BA, GA, 2>(p, stream);
    else
        launch_residual_group<D, PT, TR, BA, GA, 4>(p, stream);
}

template <int D, int PT, int TR, int BA>
void launch_anchor_group(const MultiRowParams& p, hipStream_t stream) {
    if (p.anchor.group == 32)
        launch_anchor<D, PT, TR, BA, 32>(p, stream);
    else
        launch_anchor<D, PT, TR, BA, 16>(p, stream);
}

template <int D, int PT, int TR>
bool launch_tr(const MultiRowParams& p, hipStream_t stream) {
    if (p.chain_length > 1) {
        switch (p.chain_length) {
            case 2: launch_chain<D, PT, TR, 2>(p, stream); return true;
            case 3: launch_chain<D, PT, TR, 3>(p, stream); return true;
            case 4: launch_chain<D, PT, TR, 4>(p, stream); return true;
            default: return false;
        }
    }
    if (p.anchor.bits == 4)
        launch_anchor_group<D, PT, TR, 4>(p, stream);
    else
        launch_anchor_group<D, PT, TR, 2>(p, stream);
    return true;
}

template <int D, int PT>
bool launch_pt(const MultiRowParams& p, hipStream_t stream) {
    return stream_tile_rows(p) == 16 ? launch_tr<D, PT, 16>(p, stream) : launch_tr<D, PT, 32>(p, stream);
}

template <int D>
bool launch_d(const MultiRowParams& p, hipStream_t stream) {
    bool launched = false;
    if (p.page_tokens == 16)
        launched = launch_pt<D, 16>(p, stream);
    else if (p.page_tokens == 32)
        launched = launch_pt<D, 32>(p, stream);
    if (!launched) return false;
    hipLaunchKernelGGL(multirow_finish_kernel<D>, dim3((unsigned)p.requests, (unsigned)p.heads, (unsigned)p.row_tiles),
                       dim3(kThreads), 0, stream, p);
    return true;
}

}  // namespace

hipError_t launch_multirow(const MultiRowParams& p, hipStream_t stream) {
    if (p.rows == 0 || p.requests == 0) return hipSuccess;
    bool launched = false;
    if (p.head_dim == 128)
        launched = launch_d<128>(p, stream);
    else if (p.head_dim == 96)
        launched = launch_d<96>(p, stream);
    if (!launched) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace rq
