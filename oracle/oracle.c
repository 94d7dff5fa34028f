/*
 * CPU oracle for the quantized matrix-multiply path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker, never by
 * the product. See oracle.h for the contract and the reference lines each function follows.
 *
 * Floating-point expressions keep the reference's evaluation order operation by operation;
 * the file is built with -ffp-contract=off (and the pragma below) so no multiply-add is fused,
 * as in backends/cpu/CMakeLists.txt:14-16 and src/tensor/quant.cpp:18-20.
 */

#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

enum {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q2_K = 10, T_Q3_K = 11,
    T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ4_NL = 20, T_IQ3_S = 21, T_IQ4_XS = 23, T_BF16 = 30
};

/* ---- fp16 ------------------------------------------------------------------------------ */

/* include/halo/tensor/fp16.h:19-37. Written as an explicit case split on the exponent field:
 * normal numbers rebias the exponent (15 -> 127), subnormals are m * 2^-24 (exact in fp32),
 * inf keeps its sign, NaN keeps sign and payload with the quiet bit set (what the reference's
 * scaling multiply produces on a signalling NaN). */
float oracle_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (m << 13) | (m != 0 ? 0x00400000u : 0u);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        const float v = (float)m * 0x1p-24f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float f16_at(const uint8_t* p) { return oracle_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---- geometry (src/tensor/dtype.cpp:19-51) ---------------------------------------------- */

uint32_t oracle_block_elems(uint32_t type) {
    switch (type) {
        case T_F32: case T_F16: case T_BF16: return 1;
        case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_IQ4_NL: return 32;
        case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_IQ4_XS: case T_IQ3_S: return 256;
        default: return 0;
    }
}

uint32_t oracle_block_bytes(uint32_t type) {
    switch (type) {
        case T_F32: return 4;
        case T_F16: case T_BF16: return 2;
        case T_Q4_0: case T_IQ4_NL: return 18;
        case T_Q4_1: return 20;
        case T_Q5_0: return 22;
        case T_Q5_1: return 24;
        case T_Q2_K: return 84;
        case T_Q3_K: case T_IQ3_S: return 110;
        case T_Q8_0: return 34;
        case T_Q4_K: return 144;
        case T_Q5_K: return 176;
        case T_Q6_K: return 210;
        case T_IQ4_XS: return 136;
        default: return 0;
    }
}

/* src/tensor/quant.cpp:411-428 (checked_blocks + row_bytes). */
uint64_t oracle_row_bytes(uint32_t type, int64_t n, int* err) {
    const uint32_t be = oracle_block_elems(type);
    *err = ORACLE_OK;
    if (be == 0) { *err = ORACLE_EUNSUPPORTED; return 0; }
    if (n < 0 || (uint64_t)n % be != 0) { *err = ORACLE_EMODEL; return 0; }
    const uint64_t nb = (uint64_t)n / be;
    if (nb > (uint64_t)INT64_MAX / oracle_block_bytes(type)) { *err = ORACLE_EMODEL; return 0; }
    return nb * oracle_block_bytes(type);
}

/* ---- per-block dequantizers ------------------------------------------------------------- */

/* quant.cpp:79-90. Element j < 16 is the low nibble of qs[j], element j + 16 the high one;
 * value fl(q - 8) * d. */
static void deq_q4_0(const uint8_t* blk, float* y) {
    const float d = f16_at(blk);
    for (int e = 0; e < 32; ++e) {
        const uint8_t byte = blk[2 + (e & 15)];
        const int q = (e < 16 ? (byte & 0x0F) : (byte >> 4)) - 8;
        y[e] = (float)q * d;
    }
}

/* quant.cpp:72-74 and fp16.h:61-63: the 16 bits are the top half of the fp32 pattern. */
static float bf16_at(const uint8_t* p) {
    const uint32_t bits = (uint32_t)(p[0] | (p[1] << 8)) << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* quant.cpp:93-105. Header d, m (fp16); nibbles in Q4_0's order, unsigned; value fl(q) * d + m,
 * the product rounded before the add. b (when asked) is -m, so that a - b is the value. */
static void deq_q4_1(const uint8_t* blk, float* y, float* a, float* b) {
    const float d = f16_at(blk), m = f16_at(blk + 2);
    for (int e = 0; e < 32; ++e) {
        const uint8_t byte = blk[4 + (e & 15)];
        const float t = (float)(e < 16 ? (byte & 0x0F) : (byte >> 4)) * d;
        if (y) y[e] = t + m;
        if (a) { a[e] = t; b[e] = -m; }
    }
}

/* The fifth bit of element e of a Q5_0 / Q5_1 block: bit e of the little-endian 32-bit qh.
 * (The reference moves bit j to bit 4 for j < 16 and bit j + 16 for the high half,
 * quant.cpp:114-115 and :132-133; both are bit e.) */
static int q5_high(const uint8_t* qh, int e) { return (qh[e / 8] >> (e % 8)) & 1; }

/* quant.cpp:108-122: d; qh at +2; qs at +6; value fl(code - 16) * d. */
static void deq_q5_0(const uint8_t* blk, float* y) {
    const float d = f16_at(blk);
    for (int e = 0; e < 32; ++e) {
        const uint8_t byte = blk[6 + (e & 15)];
        const int code = (e < 16 ? (byte & 0x0F) : (byte >> 4)) | (q5_high(blk + 2, e) << 4);
        y[e] = (float)(code - 16) * d;
    }
}

/* quant.cpp:125-140: d, m; qh at +4; qs at +8; value fl(code) * d + m. b (when asked) is -m. */
static void deq_q5_1(const uint8_t* blk, float* y, float* a, float* b) {
    const float d = f16_at(blk), m = f16_at(blk + 2);
    for (int e = 0; e < 32; ++e) {
        const uint8_t byte = blk[8 + (e & 15)];
        const int code = (e < 16 ? (byte & 0x0F) : (byte >> 4)) | (q5_high(blk + 4, e) << 4);
        const float t = (float)code * d;
        if (y) y[e] = t + m;
        if (a) { a[e] = t; b[e] = -m; }
    }
}

/* quant.cpp:168-193: scales[16], qs[64] at +16, d at +80, dmin at +82. Element
 * e = 128 n + 32 j + 16 h + l (the reference's loops: half n, shift 2 j, run h, lane l) takes
 * code bits 2 j, 2 j + 1 of qs[32 n + 16 h + l] and scale byte sc = scales[8 n + 2 j + h];
 * dl = d * fl(sc & 15), ml = dmin * fl(sc >> 4); value dl * fl(code) - ml. b (when asked) = ml. */
static void deq_q2_k(const uint8_t* blk, float* y, float* a, float* b) {
    const float d = f16_at(blk + 80), dmin = f16_at(blk + 82);
    for (int e = 0; e < 256; ++e) {
        const int n = e / 128, j = (e % 128) / 32, h = (e % 32) / 16, l = e % 16;
        const uint8_t sc = blk[8 * n + 2 * j + h];
        const float dl = d * (float)(sc & 0x0F), ml = dmin * (float)(sc >> 4);
        const float t = dl * (float)((blk[16 + 32 * n + 16 * h + l] >> (2 * j)) & 3);
        if (y) y[e] = t - ml;
        if (a) { a[e] = t; b[e] = ml; }
    }
}

/* quant.cpp:143-151: fl(int8 q) * d. */
static void deq_q8_0(const uint8_t* blk, float* y) {
    const float d = f16_at(blk);
    for (int e = 0; e < 32; ++e) y[e] = (float)(int8_t)blk[2 + e] * d;
}

/* quant.cpp:236-244 (ggml get_scale_min_k4), restated from the 12-byte packing: bytes 0-3
 * carry sc[0..3] in their low 6 bits and the top 2 bits of sc[4..7]; bytes 4-7 carry m[0..3]
 * and the top bits of m[4..7]; bytes 8-11 carry the low nibbles of sc[4..7] (low half) and
 * m[4..7] (high half). */
static void k4_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *m = s[j + 4] & 0x3F;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* quant.cpp:247-269. Element e: group g = e / 64 of 32 quant bytes; within it, e % 64 < 32
 * takes the low nibble of byte e % 32 with sub-block 2g, else the high nibble with 2g + 1.
 * value (d * sc) * q - dmin * m. */
static void deq_q4_k(const uint8_t* blk, float* y, float* a, float* b) {
    const float d = f16_at(blk);
    const float dmin = f16_at(blk + 2);
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int e = 0; e < 256; ++e) {
        const int g = e / 64, hi = (e % 64) / 32, l = e % 32;
        int sc, m;
        k4_scale_min(scales, 2 * g + hi, &sc, &m);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        const uint8_t byte = qs[32 * g + l];
        const int q = hi ? (byte >> 4) : (byte & 0x0F);
        const float t = d1 * (float)q;
        if (y) y[e] = t - m1;
        if (a) { a[e] = t; b[e] = m1; }
    }
}

/* quant.cpp:271-299. As Q4_K (the quants start at byte 48), with a fifth bit: bit 2g + hi of
 * qh[l] (qh holds 32 bytes and is not advanced per group, only the tested bit moves). value
 * (d * sc) * q - dmin * m. */
static void deq_q5_k(const uint8_t* blk, float* y, float* a, float* b) {
    const float d = f16_at(blk);
    const float dmin = f16_at(blk + 2);
    const uint8_t* scales = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    for (int e = 0; e < 256; ++e) {
        const int g = e / 64, hi = (e % 64) / 32, l = e % 32, j = 2 * g + hi;
        int sc, m;
        k4_scale_min(scales, j, &sc, &m);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        const uint8_t byte = qs[32 * g + l];
        const int q = (hi ? (byte >> 4) : (byte & 0x0F)) + (((qh[l] >> j) & 1) ? 16 : 0);
        const float t = d1 * (float)q;
        if (y) y[e] = t - m1;
        if (a) { a[e] = t; b[e] = m1; }
    }
}

/* The IQ4_NL value table of the GGUF format (ggml's kvalues_iq4nl; the reference's copy is
 * src/tensor/ggml_tables.h:94-96). */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* quant.cpp:330-347. Sub-block ib of 32: 6-bit scale ls = (nibble ib of scales_l) | (bits
 * 2ib..2ib+1 of scales_h) << 4, multiplier dl = d * fl(ls - 32); element j < 16 is the low
 * nibble of qs[16 ib + j], j + 16 the high one, value dl * fl(table[nibble]). */
static void deq_iq4_xs(const uint8_t* blk, float* y, float* a, float* off) {
    const float d = f16_at(blk);
    const unsigned sh = (unsigned)blk[2] | ((unsigned)blk[3] << 8);
    const uint8_t* sl = blk + 4;
    const uint8_t* qs = blk + 8;
    for (int ib = 0; ib < 8; ++ib) {
        const int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0x0F) | (int)(((sh >> (2 * ib)) & 3u) << 4);
        const float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; ++j) {
            const uint8_t byte = qs[16 * ib + j];
            const float lo = dl * (float)kIq4nl[byte & 0x0F], hi = dl * (float)kIq4nl[byte >> 4];
            if (y) { y[32 * ib + j] = lo; y[32 * ib + j + 16] = hi; }
            if (a) {
                a[32 * ib + j] = lo;
                a[32 * ib + j + 16] = hi;
                off[32 * ib + j] = off[32 * ib + j + 16] = 128.0f * dl;
            }
        }
    }
}

/* quant.cpp:302-327. Element e: half n = e / 128; r = e % 128; quarter k = r / 32; l = r % 32.
 * Low 4 bits: ql[64n + l + 32 (k & 1)], low nibble for k < 2 else high; top 2 bits: bits
 * 2k..2k+1 of qh[32n + l]; scale: int8 sc[8n + l / 16 + 2k]; value (d * sc) * (q - 32). */
static void deq_q6_k(const uint8_t* blk, float* y, float* a, float* off) {
    const float d = f16_at(blk + 208);
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int e = 0; e < 256; ++e) {
        const int n = e / 128, r = e % 128, k = r / 32, l = r % 32;
        const uint8_t lb = ql[64 * n + l + 32 * (k & 1)];
        const int lo4 = k < 2 ? (lb & 0x0F) : (lb >> 4);
        const int hi2 = (qh[32 * n + l] >> (2 * k)) & 3;
        const int q = (lo4 | (hi2 << 4)) - 32;
        const float ds = d * (float)sc[8 * n + l / 16 + 2 * k];
        const float v = ds * (float)q;
        if (y) y[e] = v;
        if (a) { a[e] = v; off[e] = ds * 32.0f; }
    }
}

/* quant.cpp:154-165. As Q4_0's nibble order (element j < 16: low nibble of qs[j]; j + 16:
 * the high one), value d * fl(table[nibble]). */
static void deq_iq4_nl(const uint8_t* blk, float* y, float* a, float* off) {
    const float d = f16_at(blk);
    for (int e = 0; e < 32; ++e) {
        const uint8_t byte = blk[2 + (e & 15)];
        const float v = d * (float)kIq4nl[e < 16 ? (byte & 0x0F) : (byte >> 4)];
        if (y) y[e] = v;
        if (a) { a[e] = v; off[e] = 128.0f * d; }
    }
}

/* quant.cpp:196-233. Sixteen 6-bit scales packed in bytes 96..107: scale i takes nibble i / 8
 * of byte i % 8 as its low 4 bits and bits 2 (i / 4) .. 2 (i / 4) + 1 of byte 8 + i % 4 as its
 * top 2 (the reference's aux/kmask shuffle, written per index). Element e: half n = e / 128,
 * shift pair j = (e % 128) / 32, l = e % 32; q = ((qs[32 n + l] >> 2 j) & 3) - 4 unless bit
 * 4 n + j of hmask[l] is set; scale index 8 n + 2 j + l / 16; value (d * fl(sc - 32)) * fl(q). */
static int q3k_scale(const uint8_t* sb, int i) {
    return ((sb[i % 8] >> (4 * (i / 8))) & 0x0F) | (((sb[8 + i % 4] >> (2 * (i / 4))) & 3) << 4);
}

static void deq_q3_k(const uint8_t* blk, float* y, float* a, float* off) {
    const float d_all = f16_at(blk + 108);
    const uint8_t* hm = blk;
    const uint8_t* qs = blk + 32;
    const uint8_t* sb = blk + 96;
    for (int e = 0; e < 256; ++e) {
        const int n = e / 128, j = (e % 128) / 32, l = e % 32;
        const int q = ((qs[32 * n + l] >> (2 * j)) & 3) - (((hm[l] >> (4 * n + j)) & 1) ? 0 : 4);
        const float dl = d_all * (float)(q3k_scale(sb, 8 * n + 2 * j + l / 16) - 32);
        const float v = dl * (float)q;
        if (y) y[e] = v;
        if (a) { a[e] = v; off[e] = 4.0f * dl; }
    }
}

/* The IQ3_S codebook of the GGUF format (ggml's iq3s_grid; the reference's copy is
 * src/tensor/ggml_tables.h:27-92), pinned against the reference's values by the tests. */
static const uint32_t kIq3sGrid[512] = {
#include "../halo_amd/csrc/iq3s_grid.inc"
};

/* quant.cpp:350-384. Sub-block b = e / 32 of 32 elements: multiplier db = d * fl(1 + 2 s) with s
 * nibble b % 2 of scales[b / 2]; group k = (e % 32) / 4 of 4 elements takes codebook entry
 * qs[8 b + k] | (bit k of qh[b]) << 8, element e its byte e % 4; the sign is bit e % 8 of
 * signs[4 b + (e % 32) / 8] (set: -1). value (db * fl(byte)) * sign. */
static void deq_iq3_s(const uint8_t* blk, float* y, float* a, float* off) {
    const float d = f16_at(blk);
    const uint8_t* qs = blk + 2;
    const uint8_t* qh = blk + 66;
    const uint8_t* signs = blk + 74;
    const uint8_t* scales = blk + 106;
    for (int e = 0; e < 256; ++e) {
        const int b = e / 32, k = (e % 32) / 4;
        const float db = d * (float)(1 + 2 * ((scales[b / 2] >> (4 * (b % 2))) & 0x0F));
        const unsigned idx = qs[8 * b + k] | (((qh[b] >> k) & 1u) << 8);
        const float g = (float)((kIq3sGrid[idx] >> (8 * (e % 4))) & 0xFFu);
        const float sgn = ((signs[4 * b + (e % 32) / 8] >> (e % 8)) & 1) ? -1.0f : 1.0f;
        const float v = db * g * sgn;
        if (y) y[e] = v;
        if (a) { a[e] = v; off[e] = 16.0f * db; }
    }
}

static int dequant_blocks(uint32_t type, const uint8_t* src, float* dst, uint64_t nb) {
    const uint32_t bb = oracle_block_bytes(type), be = oracle_block_elems(type);
    for (uint64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = src + i * bb;
        float* y = dst + i * be;
        switch (type) {
            case T_F32: memcpy(y, blk, 4); break;
            case T_F16: y[0] = f16_at(blk); break;
            case T_BF16: y[0] = bf16_at(blk); break;
            case T_Q4_0: deq_q4_0(blk, y); break;
            case T_Q4_1: deq_q4_1(blk, y, NULL, NULL); break;
            case T_Q5_0: deq_q5_0(blk, y); break;
            case T_Q5_1: deq_q5_1(blk, y, NULL, NULL); break;
            case T_Q2_K: deq_q2_k(blk, y, NULL, NULL); break;
            case T_IQ4_NL: deq_iq4_nl(blk, y, NULL, NULL); break;
            case T_Q3_K: deq_q3_k(blk, y, NULL, NULL); break;
            case T_IQ3_S: deq_iq3_s(blk, y, NULL, NULL); break;
            case T_Q8_0: deq_q8_0(blk, y); break;
            case T_Q4_K: deq_q4_k(blk, y, NULL, NULL); break;
            case T_Q5_K: deq_q5_k(blk, y, NULL, NULL); break;
            case T_Q6_K: deq_q6_k(blk, y, NULL, NULL); break;
            case T_IQ4_XS: deq_iq4_xs(blk, y, NULL, NULL); break;
            default: return ORACLE_EUNSUPPORTED;
        }
    }
    return ORACLE_OK;
}

/* quant.cpp:430-435. */
int oracle_dequantize_row(uint32_t type, const uint8_t* src, float* dst, int64_t n) {
    int err;
    (void)oracle_row_bytes(type, n, &err);
    if (err) return err;
    return dequant_blocks(type, src, dst, (uint64_t)n / oracle_block_elems(type));
}

int oracle_dequant_terms(uint32_t type, const uint8_t* src, float* a, float* b, float* off, int64_t n) {
    int err;
    (void)oracle_row_bytes(type, n, &err);
    if (err) return err;
    const uint32_t bb = oracle_block_bytes(type), be = oracle_block_elems(type);
    const uint64_t nb = (uint64_t)n / be;
    for (uint64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = src + i * bb;
        float* ab = a + i * be;
        float* bbv = b + i * be;
        float* ob = off + i * be;
        switch (type) {
            case T_Q4_0: {
                const float d = f16_at(blk);
                deq_q4_0(blk, ab);
                for (uint32_t e = 0; e < be; ++e) { bbv[e] = 0.0f; ob[e] = 8.0f * d; }
                break;
            }
            case T_Q8_0: {
                const float d = f16_at(blk);
                deq_q8_0(blk, ab);
                for (uint32_t e = 0; e < be; ++e) { bbv[e] = 0.0f; ob[e] = 128.0f * d; }
                break;
            }
            case T_Q4_K:
                deq_q4_k(blk, NULL, ab, bbv);
                for (uint32_t e = 0; e < be; ++e) ob[e] = 0.0f;
                break;
            case T_Q5_K:
                deq_q5_k(blk, NULL, ab, bbv);
                for (uint32_t e = 0; e < be; ++e) ob[e] = 0.0f;
                break;
            case T_IQ4_XS:
                deq_iq4_xs(blk, NULL, ab, ob);
                for (uint32_t e = 0; e < be; ++e) bbv[e] = 0.0f;
                break;
            case T_Q6_K:
                deq_q6_k(blk, NULL, ab, ob);
                for (uint32_t e = 0; e < be; ++e) bbv[e] = 0.0f;
                break;
            case T_IQ4_NL:
                deq_iq4_nl(blk, NULL, ab, ob);
                for (uint32_t e = 0; e < be; ++e) bbv[e] = 0.0f;
                break;
            case T_Q3_K:
                deq_q3_k(blk, NULL, ab, ob);
                for (uint32_t e = 0; e < be; ++e) bbv[e] = 0.0f;
                break;
            case T_IQ3_S:
                deq_iq3_s(blk, NULL, ab, ob);
                for (uint32_t e = 0; e < be; ++e) bbv[e] = 0.0f;
                break;
            /* GGUF-layout-only types: the value split as a - b where the reference rounds an add
             * (Q4_1, Q5_1: b = -m; Q2_K: b = ml); off = 0, no kernel takes a code bias out */
            case T_Q4_1:
                deq_q4_1(blk, NULL, ab, bbv);
                for (uint32_t e = 0; e < be; ++e) ob[e] = 0.0f;
                break;
            case T_Q5_1:
                deq_q5_1(blk, NULL, ab, bbv);
                for (uint32_t e = 0; e < be; ++e) ob[e] = 0.0f;
                break;
            case T_Q2_K:
                deq_q2_k(blk, NULL, ab, bbv);
                for (uint32_t e = 0; e < be; ++e) ob[e] = 0.0f;
                break;
            case T_BF16: case T_Q5_0:
                dequant_blocks(type, blk, ab, 1);
                for (uint32_t e = 0; e < be; ++e) { bbv[e] = 0.0f; ob[e] = 0.0f; }
                break;
            default: return ORACLE_EUNSUPPORTED;
        }
    }
    return ORACLE_OK;
}

/* ---- dot products ----------------------------------------------------------------------- */

/* backends/cpu/kernel_common.h:16-27: partial sum j accumulates the products of indices
 * i = j (mod 8) over the full groups of 8, in increasing i; the partials combine as
 * ((p0+p4)+(p1+p5))+((p2+p6)+(p3+p7)); the remaining n % 8 products are summed sequentially
 * into a separate tail that is added last. */
float oracle_dot(const float* a, const float* b, size_t n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const size_t full = n - n % 8;
    for (size_t i = 0; i < full; ++i) {
        const float prod = a[i] * b[i];
        p[i % 8] = p[i % 8] + prod;
    }
    float tail = 0.0f;
    for (size_t i = full; i < n; ++i) {
        const float prod = a[i] * b[i];
        tail = tail + prod;
    }
    const float left = (p[0] + p[4]) + (p[1] + p[5]);
    const float right = (p[2] + p[6]) + (p[3] + p[7]);
    return (left + right) + tail;
}

/* quant.cpp:447-466: double accumulation of the dequantized row times x. */
int oracle_vec_dot_row(uint32_t type, const uint8_t* row, const float* x, int64_t n, float* out) {
    int err;
    (void)oracle_row_bytes(type, n, &err);
    if (err) return err;
    const uint32_t be = oracle_block_elems(type), bb = oracle_block_bytes(type);
    float buf[256];
    double acc = 0.0;
    for (int64_t base = 0; base < n; base += be) {
        dequant_blocks(type, row + (uint64_t)(base / be) * bb, buf, 1);
        for (uint32_t i = 0; i < be; ++i) acc += (double)buf[i] * (double)x[base + i];
    }
    *out = (float)acc;
    return ORACLE_OK;
}

/* ---- static-partition thread pool (thread_pool.h:58-76, :103-113) ----------------------- */

void oracle_partition_range(size_t n, size_t parts, size_t i, size_t* begin, size_t* end) {
    const size_t base = n / parts, extra = n % parts;
    *begin = i * base + (i < extra ? i : extra);
    *end = *begin + base + (i < extra ? 1 : 0);
}

uint32_t oracle_default_threads(void) {
    const long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (uint32_t)n : 1u;
}

typedef void (*range_fn)(void* ctx, size_t b0, size_t b1);

typedef struct {
    range_fn fn;
    void* ctx;
    size_t b0, b1;
} part_t;

static void* run_part(void* p) {
    part_t* pt = (part_t*)p;
    pt->fn(pt->ctx, pt->b0, pt->b1);
    return NULL;
}

/* parallel_for: range 0 runs on the caller, ranges 1.. on their own threads. */
static void parallel_for(uint32_t threads, size_t n, range_fn fn, void* ctx) {
    if (n == 0) return;
    size_t parts = threads < 1 ? 1 : threads;
    if (parts > n) parts = n;
    if (parts == 1) { fn(ctx, 0, n); return; }
    part_t* pts = (part_t*)calloc(parts, sizeof(part_t));
    pthread_t* th = (pthread_t*)calloc(parts, sizeof(pthread_t));
    for (size_t i = 0; i < parts; ++i) {
        pts[i].fn = fn;
        pts[i].ctx = ctx;
        oracle_partition_range(n, parts, i, &pts[i].b0, &pts[i].b1);
    }
    for (size_t i = 1; i < parts; ++i) pthread_create(&th[i], NULL, run_part, &pts[i]);
    run_part(&pts[0]);
    for (size_t i = 1; i < parts; ++i) pthread_join(th[i], NULL);
    free(pts);
    free(th);
}

/* ---- matmul (backends/cpu/matmul.cpp:17, :37-59) ----------------------------------------- */

enum { kRowBlock = 16 };

typedef struct {
    uint32_t type;
    const uint8_t* w;
    uint64_t w_stride, rb;
    uint32_t rows, cols, n_vec;
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
} mm_ctx;

/* One range of 16-row blocks: each block is dequantized once into a scratch buffer (the
 * WeightMatrix::row_block materialization, weight_matrix.h:54-64; rows one at a time when
 * the stride is padded, cpu_backend.cpp:199-209) and dotted with every x row. */
static void mm_range(void* p, size_t b0, size_t b1) {
    const mm_ctx* c = (const mm_ctx*)p;
    float* scratch = (float*)malloc((size_t)kRowBlock * c->cols * sizeof(float));
    for (size_t blk = b0; blk < b1; ++blk) {
        const size_t n0 = blk * kRowBlock;
        const size_t nn = c->rows - n0 < kRowBlock ? c->rows - n0 : kRowBlock;
        if (c->type == T_F32) {
            for (size_t r = 0; r < nn; ++r) memcpy(scratch + r * c->cols, c->w + (n0 + r) * c->w_stride, (size_t)c->cols * 4);
        } else if (c->w_stride == c->rb) {
            dequant_blocks(c->type, c->w + n0 * c->rb, scratch, nn * c->cols / oracle_block_elems(c->type));
        } else {
            for (size_t r = 0; r < nn; ++r)
                dequant_blocks(c->type, c->w + (n0 + r) * c->w_stride, scratch + r * c->cols,
                               c->cols / oracle_block_elems(c->type));
        }
        for (size_t t = 0; t < c->n_vec; ++t) {
            const float* xt = c->x + t * c->x_stride;
            float* yt = c->y + t * c->y_stride + n0;
            for (size_t n = 0; n < nn; ++n) yt[n] = oracle_dot(xt, scratch + n * c->cols, c->cols);
        }
    }
    free(scratch);
}

int oracle_matmul(uint32_t type, const uint8_t* w, uint64_t w_stride, uint32_t rows, uint32_t cols,
                  const float* x, uint64_t x_stride, uint32_t n_vec, float* y, uint64_t y_stride,
                  uint32_t threads) {
    int err;
    const uint64_t rb = oracle_row_bytes(type, cols, &err);
    if (err) return err;
    mm_ctx c;
    c.type = type;
    c.w = w;
    c.rb = rb;
    c.w_stride = w_stride ? w_stride : rb;
    if (rows > 1 && c.w_stride < rb) return ORACLE_EKERNEL;
    c.rows = rows;
    c.cols = cols;
    c.n_vec = n_vec;
    c.x = x;
    c.x_stride = x_stride ? x_stride : cols;
    c.y = y;
    c.y_stride = y_stride ? y_stride : rows;
    if (n_vec > 1 && (c.x_stride < cols || c.y_stride < rows)) return ORACLE_EKERNEL;
    const size_t n_blocks = (rows + kRowBlock - 1) / kRowBlock;
    parallel_for(threads, n_blocks, mm_range, &c);
    return ORACLE_OK;
}

/* ---- swiglu (ops_basic.cpp:165-167, kernel_common.h:32) ---------------------------------- */

static float silu(float v) { return v / (1.0f + expf(-v)); }

void oracle_swiglu(const float* g, const float* u, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = silu(g[i]) * u[i];
}

/* backends/cpu/ops_basic.cpp:18-33. */
void oracle_rms_norm(const float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride,
                     uint32_t rows, uint32_t cols, float eps) {
    if (x_stride == 0) x_stride = cols;
    if (out_stride == 0) out_stride = cols;
    for (uint32_t r = 0; r < rows; ++r) {
        const float* xr = x + (uint64_t)r * x_stride;
        float* yr = out + (uint64_t)r * out_stride;
        const float mean = oracle_dot(xr, xr, cols) / (float)cols;
        const float inv = 1.0f / sqrtf(mean + eps);
        for (uint32_t i = 0; i < cols; ++i) {
            const float t = xr[i] * inv;
            yr[i] = t * w[i];
        }
    }
}

/* src/models/qwen35.cpp:789-805: gemv(gate) -> gemv(up) -> swiglu. */
int oracle_gate_up_swiglu(uint32_t type, const uint8_t* wg, const uint8_t* wu, uint64_t w_stride,
                          uint32_t rows, uint32_t cols, const float* x, uint32_t n_vec, float* out,
                          uint32_t threads) {
    const size_t n = (size_t)n_vec * rows;
    float* g = (float*)malloc(n * sizeof(float));
    float* u = (float*)malloc(n * sizeof(float));
    int err = oracle_matmul(type, wg, w_stride, rows, cols, x, 0, n_vec, g, 0, threads);
    if (!err) err = oracle_matmul(type, wu, w_stride, rows, cols, x, 0, n_vec, u, 0, threads);
    if (!err) oracle_swiglu(g, u, out, n);
    free(g);
    free(u);
    return err;
}

/* ---- LM head: matmul + fused argmax (src/backend/cpu_backend.cpp:669-770) ----------------- */

/*
 * One pass over the head matrix in slabs of 8192 rows (:724-726): each slab's logits by
 * cpu::matmul (:729-730); per vector and row, a NaN logit poisons the vector (:734-737);
 * otherwise rows below the argmax limit rank by value, a row replacing the best only when
 * strictly greater, so ties go to the lowest index (:738-739). valid_rows = 0 means all rows
 * (:721). A poisoned vector reports {-1, quiet NaN} (:745-747); the result words are {index,
 * value bits, poisoned} (:825-833), with TopKEntry's default {-1, 0.0f} (ops.h:351-355) when
 * no row ranks. logits (optional) receive every row's value (:740).
 */
int oracle_lm_head(uint32_t type, const uint8_t* w, uint64_t w_stride, uint32_t rows, uint32_t cols, const float* x,
                   uint32_t n_vec, uint32_t valid_rows, float* logits, uint32_t* result, uint32_t threads) {
    int err;
    const uint64_t rb = oracle_row_bytes(type, cols, &err);
    if (err) return err;
    if (w_stride == 0) w_stride = rb;
    if (n_vec == 0) return ORACLE_OK;
    const size_t kSlab = 8192;
    const size_t slab = rows < kSlab ? rows : kSlab;
    const size_t limit = valid_rows > 0 && valid_rows < rows ? valid_rows : rows;
    float* buf = (float*)malloc((size_t)n_vec * (slab ? slab : 1) * sizeof(float));
    int32_t* bi = (int32_t*)malloc(n_vec * sizeof(int32_t));
    float* bv = (float*)malloc(n_vec * sizeof(float));
    uint8_t* poisoned = (uint8_t*)calloc(n_vec, 1);
    if (!buf || !bi || !bv || !poisoned) {
        free(buf), free(bi), free(bv), free(poisoned);
        return ORACLE_EKERNEL;
    }
    for (uint32_t i = 0; i < n_vec; ++i) bi[i] = -1, bv[i] = 0.0f;
    for (size_t n0 = 0; n0 < rows && !err; n0 += slab) {
        const size_t ns = rows - n0 < slab ? rows - n0 : slab;
        err = oracle_matmul(type, w + n0 * w_stride, w_stride, (uint32_t)ns, cols, x, 0, n_vec, buf, slab, threads);
        for (uint32_t i = 0; i < n_vec && !err; ++i) {
            const float* row = buf + (size_t)i * slab;
            for (size_t c = 0; c < ns; ++c) {
                if (isnan(row[c])) {
                    poisoned[i] = 1;
                    continue;
                }
                if (!poisoned[i] && n0 + c < limit && (bi[i] < 0 || row[c] > bv[i])) bi[i] = (int32_t)(n0 + c), bv[i] = row[c];
            }
            if (logits) memcpy(logits + (size_t)i * rows + n0, row, ns * sizeof(float));
        }
    }
    for (uint32_t i = 0; i < n_vec && !err; ++i) {
        float v = bv[i];
        int32_t idx = bi[i];
        if (poisoned[i]) idx = -1, v = nanf("");
        uint32_t vb;
        memcpy(&vb, &v, 4);
        result[3 * i] = (uint32_t)idx;
        result[3 * i + 1] = vb;
        result[3 * i + 2] = poisoned[i] ? 1u : 0u;
    }
    free(buf), free(bi), free(bv), free(poisoned);
    return err;
}

void oracle_argmax_words(const float* logits, uint32_t n, uint32_t n_vec, uint32_t* result) {
    for (uint32_t i = 0; i < n_vec; ++i) {
        const float* row = logits + (size_t)i * n;
        uint32_t best = 0, nan = 0;
        for (uint32_t c = 0; c < n; ++c) {
            if (isnan(row[c])) nan = 1;
            else if (!isnan(row[best]) ? row[c] > row[best] : 1) best = c;
        }
        float v = nan ? nanf("") : row[best];
        uint32_t vb;
        memcpy(&vb, &v, 4);
        result[3 * i] = nan ? 0xFFFFFFFFu : best;
        result[3 * i + 1] = vb;
        result[3 * i + 2] = nan;
    }
}
