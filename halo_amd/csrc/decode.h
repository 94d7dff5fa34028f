// Device-side unpacking of GGUF blocks and SLAB slot records. Every weight value these
// helpers produce is bit-identical to the reference dequantizer (src/tensor/quant.cpp:68-74,
// :79-140, :143-151, :154-165, :168-193, :196-233, :236-269, :271-299, :302-327, :330-347,
// :350-384): each expression is evaluated in the reference's order with contraction off, so
// every rounding step (a product, then Q4_1's and Q5_1's `+ m`, Q2_K's `- ml`, Q4_K's and
// Q5_K's `- dmin * m`) is the same one.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "slab_layout.h"

namespace halo_mi::dev {

// fp16 -> fp32 with v_cvt_f32_f16 (exact, fp16 denormals kept: the library is built without
// denormal flushing; a test forces a subnormal scale in every row).
__device__ __forceinline__ float h2f(uint32_t h16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h16)));
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// ---- Q4_K 6-bit scale/min of sub-block j from the 12 packed bytes (held as 3 dwords) -------
// s0 = bytes 0..3, s1 = bytes 4..7, s2 = bytes 8..11 of the scales field.
// j < 4: sc = b[j] & 63, m = b[j+4] & 63; j >= 4: sc = (b[j+4] & 15) | (b[j-4] >> 6) << 4,
// m = (b[j+4] >> 4) | (b[j] >> 6) << 4 (ggml get_scale_min_k4, quant.cpp:236-244).
__device__ __forceinline__ void q4k_sc_m(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j, uint32_t& sc,
                                         uint32_t& m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const uint32_t jj = j - 4;
        const uint32_t b8 = (s2 >> (8 * jj)) & 0xFFu;
        sc = (b8 & 15u) | (((s0 >> (8 * jj + 6)) & 3u) << 4);
        m = (b8 >> 4) | (((s1 >> (8 * jj + 6)) & 3u) << 4);
    }
}

// d1 = d * sc and m1 = dmin * m for sub-block j of a Q4_K header (16 B as uint4).
__device__ __forceinline__ void q4k_scales(const uint4& hdr, uint32_t j, float& d1, float& m1) {
    uint32_t sc, m;
    q4k_sc_m(hdr.y, hdr.z, hdr.w, j, sc, m);
    d1 = h2f(hdr.x & 0xFFFFu) * (float)sc;
    m1 = h2f(hdr.x >> 16) * (float)m;
}

// ---- Q6_K slot record -> 6-bit unsigned quants, 4 per dword (byte lanes) --------------------
// ql: the 16-byte low-nibble record; qh: the 8-byte top-bit record (see q6_qh_byte).
// Output dword i (0..3) holds elements 4i..4i+3 (lo[i]) and 16+4i..16+4i+3 (hi[i]).
__device__ __forceinline__ void q6_slot_bytes(const uint4& ql, const uint2& qh, uint32_t lo[4], uint32_t hi[4]) {
    const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w};
    const uint32_t H[2] = {qh.x, qh.y};
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const uint32_t a = L[2 * w], b = L[2 * w + 1], h = H[w];
        lo[2 * w] = (a & 0x0F0F0F0Fu) | (h & 0x30303030u);
        hi[2 * w] = ((a >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
        lo[2 * w + 1] = (b & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
        hi[2 * w + 1] = ((b >> 4) & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    }
}

// ---- IQ4_XS ---------------------------------------------------------------------------------
// The IQ4_NL value table of the GGUF format (ggml's kvalues_iq4nl; the reference's copy is at
// src/tensor/ggml_tables.h:94-96), four int8 values per dword.
constexpr uint32_t kIq4Tab[4] = {0xBFAD9881u, 0xF6EADDCFu, 0x26190D01u, 0x71594535u};
// The same values plus 128 (1 .. 241): unsigned bytes for the paths that bias codes.
constexpr uint32_t kIq4TabB[4] = {0x3F2D1801u, 0x766A5D4Fu, 0xA6998D81u, 0xF1D9C5B5u};

__device__ __forceinline__ int iq4_value(uint32_t nib) {
    const uint32_t w = nib < 8 ? (nib < 4 ? kIq4Tab[0] : kIq4Tab[1]) : (nib < 12 ? kIq4Tab[2] : kIq4Tab[3]);
    return (int)(int8_t)((w >> (8 * (nib & 3u))) & 0xFFu);
}
// 6-bit scale of sub-block j (quant.cpp:336): ls = (scales_l nibble j) | (scales_h bits 2j..2j+1) << 4;
// the sub-block's multiplier is d * (ls - 32). sh = scales_h (16 bits), sl = scales_l (4 bytes).
__device__ __forceinline__ int iq4xs_ls(uint32_t sh, uint32_t sl, uint32_t j) {
    return (int)(((sl >> (4 * j)) & 15u) | (((sh >> (2 * j)) & 3u) << 4)) - 32;
}
// Four 4-bit codes in the low nibbles of q's bytes (the high nibbles are ignored) -> the
// table's biased values (kIq4TabB) as bytes: a byte-permute over each table half with the
// code's low 3 bits, then a third one that takes byte k from the half that bit 3 names.
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t q) {
    const uint32_t sel = q & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4TabB[1], kIq4TabB[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4TabB[3], kIq4TabB[2], sel);
    return __builtin_amdgcn_perm(hi, lo, ((q >> 1) & 0x04040404u) | 0x03020100u);
}

// ---- IQ3_S ----------------------------------------------------------------------------------
// The GGUF IQ3_S codebook (ggml's iq3s_grid): entry g holds four magnitudes, byte j for
// element j of a 4-element group.
__device__ const uint32_t kIq3sGrid[512] = {
#include "iq3s_grid.inc"
};

// Q3_K's 16 six-bit scales from the 12 packed bytes sb: scale i = nibble i / 8 of byte i % 8,
// with bits 2 (i / 4) .. + 1 of byte 8 + i % 4 on top (quant.cpp:203-212's shuffle, per index).
__device__ __forceinline__ int q3k_scale(const uint8_t* sb, uint32_t i) {
    return (int)(((sb[i % 8] >> (4 * (i / 8))) & 15u) | (((sb[8 + i % 4] >> (2 * (i / 4))) & 3u) << 4));
}

// ---- per-element decode of a GGUF row (the reference variant; byte loads) -------------------
// Same expressions as quant.cpp; contraction is off in every caller.
__device__ __forceinline__ float gguf_elem(uint32_t type, const uint8_t* row, uint32_t i) {
#pragma clang fp contract(off)
    switch (type) {
        case kF32: {
            uint32_t u = (uint32_t)row[4 * i] | ((uint32_t)row[4 * i + 1] << 8) | ((uint32_t)row[4 * i + 2] << 16) |
                         ((uint32_t)row[4 * i + 3] << 24);
            return __uint_as_float(u);
        }
        case kQ4_0: {
            const uint8_t* blk = row + (i / 32) * 18;
            const uint32_t e = i % 32;
            const float d = h2f(ld_u16(blk));
            const uint8_t b = blk[2 + (e & 15)];
            const int q = (int)(e < 16 ? (b & 15) : (b >> 4)) - 8;
            return (float)q * d;
        }
        case kQ8_0: {
            const uint8_t* blk = row + (i / 32) * 34;
            const float d = h2f(ld_u16(blk));
            return (float)(int8_t)blk[2 + i % 32] * d;
        }
        case kQ4_K: {
            const uint8_t* blk = row + (i / 256) * 144;
            const uint32_t e = i % 256, g = e / 64, hi = (e % 64) / 32, l = e % 32;
            const float d = h2f(ld_u16(blk)), dmin = h2f(ld_u16(blk + 2));
            const uint8_t* s = blk + 4;
            const uint32_t j = 2 * g + hi;
            uint32_t sc, m;
            if (j < 4) {
                sc = s[j] & 63;
                m = s[j + 4] & 63;
            } else {
                sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
                m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
            }
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            const uint8_t qb = blk[16 + 32 * g + l];
            const uint32_t q = hi ? (qb >> 4) : (qb & 15);
            return d1 * (float)q - m1;
        }
        case kQ5_K: {
            const uint8_t* blk = row + (i / 256) * 176;
            const uint32_t e = i % 256, g = e / 64, hi = (e % 64) / 32, l = e % 32;
            const float d = h2f(ld_u16(blk)), dmin = h2f(ld_u16(blk + 2));
            const uint8_t* s = blk + 4;
            const uint32_t j = 2 * g + hi;
            uint32_t sc, m;
            if (j < 4) {
                sc = s[j] & 63;
                m = s[j + 4] & 63;
            } else {
                sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
                m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
            }
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            const uint8_t qb = blk[48 + 32 * g + l];
            const uint32_t q = (hi ? (qb >> 4) : (qb & 15)) + (((blk[16 + l] >> j) & 1u) ? 16u : 0u);
            return d1 * (float)q - m1;
        }
        case kIQ4_XS: {
            const uint8_t* blk = row + (i / 256) * 136;
            const uint32_t e = i % 256, ib = e / 32, el = e % 32;
            const float d = h2f(ld_u16(blk));
            const uint32_t sl = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) | ((uint32_t)blk[7] << 24);
            const float dl = d * (float)iq4xs_ls(ld_u16(blk + 2), sl, ib);
            const uint8_t qb = blk[8 + 16 * ib + (el & 15)];
            return dl * (float)iq4_value(el < 16 ? (qb & 15u) : (qb >> 4));
        }
        case kQ6_K: {
            const uint8_t* blk = row + (i / 256) * 210;
            const uint32_t e = i % 256, n = e / 128, r = e % 128, k = r / 32, l = r % 32;
            const float d = h2f(ld_u16(blk + 208));
            const uint8_t lb = blk[64 * n + l + 32 * (k & 1)];
            const uint32_t lo4 = k < 2 ? (lb & 15) : (lb >> 4);
            const uint32_t hi2 = (blk[128 + 32 * n + l] >> (2 * k)) & 3;
            const int q = (int)(lo4 | (hi2 << 4)) - 32;
            const float sc = (float)(int8_t)blk[192 + 8 * n + l / 16 + 2 * k];
            return d * sc * (float)q;
        }
        case kF16:
            return h2f(ld_u16(row + 2 * (uint64_t)i));
        case kBF16:
            return __uint_as_float(ld_u16(row + 2 * (uint64_t)i) << 16);
        case kQ4_1: {
            // d, m; element e < 16 the low nibble of qs[e], e + 16 the high one: fl(q) * d + m
            const uint8_t* blk = row + (i / 32) * 20;
            const uint32_t e = i % 32;
            const float d = h2f(ld_u16(blk)), m = h2f(ld_u16(blk + 2));
            const uint8_t b = blk[4 + (e & 15)];
            const float t = (float)(e < 16 ? (b & 15) : (b >> 4)) * d;
            return t + m;
        }
        case kQ5_0:
        case kQ5_1: {
            // the nibble as Q4_0 / Q4_1, with bit e of the 32-bit qh as its fifth bit (quant.cpp's
            // xh_0 = bit j << 4 for e = j < 16, xh_1 = bit j + 16 << 4 for e = j + 16)
            const bool one = type == kQ5_1;
            const uint8_t* blk = row + (i / 32) * (one ? 24 : 22);
            const uint32_t e = i % 32;
            const uint8_t* qhp = blk + (one ? 4 : 2);
            const uint32_t qh = ld_u16(qhp) | (ld_u16(qhp + 2) << 16);
            const uint8_t b = qhp[4 + (e & 15)];
            const uint32_t code = (e < 16 ? (b & 15u) : (b >> 4)) | (((qh >> e) & 1u) << 4);
            const float d = h2f(ld_u16(blk));
            if (!one) return (float)((int)code - 16) * d;
            const float t = (float)code * d;
            return t + h2f(ld_u16(blk + 2));
        }
        case kQ2_K: {
            // element e = 128 n + 32 j + 16 h + l: code bits 2j..2j+1 of qs[32 n + 16 h + l]; scale
            // byte 8 n + 2 j + h gives dl = d * fl(low nibble), ml = dmin * fl(high nibble)
            const uint8_t* blk = row + (i / 256) * 84;
            const uint32_t e = i % 256, n = e / 128, j = (e % 128) / 32, hl = (e % 32) / 16, l = e % 16;
            const float d = h2f(ld_u16(blk + 80)), dmin = h2f(ld_u16(blk + 82));
            const uint32_t sc = blk[8 * n + 2 * j + hl];
            const float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
            const uint32_t q = (blk[16 + 32 * n + 16 * hl + l] >> (2 * j)) & 3u;
            const float t = dl * (float)q;
            return t - ml;
        }
        case kIQ4_NL: {
            const uint8_t* blk = row + (i / 32) * 18;
            const uint32_t e = i % 32;
            const float d = h2f(ld_u16(blk));
            const uint8_t qb = blk[2 + (e & 15)];
            return d * (float)iq4_value(e < 16 ? (qb & 15u) : (qb >> 4));
        }
        case kQ3_K: {
            // element e = 128 n + 32 j + l: code bits 2j..2j+1 of qs[32n + l] minus 4 unless bit
            // 4n + j of hmask[l] is set; scale 8n + 2j + l / 16
            const uint8_t* blk = row + (i / 256) * 110;
            const uint32_t e = i % 256, n = e / 128, j = (e % 128) / 32, l = e % 32;
            const float d_all = h2f(ld_u16(blk + 108));
            const int q = (int)((blk[32 + 32 * n + l] >> (2 * j)) & 3u) - (((blk[l] >> (4 * n + j)) & 1u) ? 0 : 4);
            const float dl = d_all * (float)(q3k_scale(blk + 96, 8 * n + 2 * j + l / 16) - 32);
            return dl * (float)q;
        }
        case kIQ3_S: {
            // sub-block b = e / 32: db = d (1 + 2 s); group k = (e % 32) / 4 takes codebook entry
            // qs[8b + k] | (bit k of qh[b]) << 8; sign bit e % 8 of signs[4b + (e % 32) / 8]
            const uint8_t* blk = row + (i / 256) * 110;
            const uint32_t e = i % 256, b = e / 32, k = (e % 32) / 4;
            const float d = h2f(ld_u16(blk));
            const float db = d * (float)(1 + 2 * ((blk[106 + b / 2] >> (4 * (b % 2))) & 15u));
            const uint32_t idx = blk[2 + 8 * b + k] | (((blk[66 + b] >> k) & 1u) << 8);
            const float g = (float)((kIq3sGrid[idx] >> (8 * (e % 4))) & 0xFFu);
            const float sgn = ((blk[74 + 4 * b + (e % 32) / 8] >> (e % 8)) & 1u) ? -1.0f : 1.0f;
            return db * g * sgn;
        }
        default:
            return 0.0f;
    }
}

}  // namespace halo_mi::dev
