// Block geometry and the SLAB weight layout, shared by the host repack and the device kernels.
//
// GGUF block formats (ggml ids; geometry as src/tensor/dtype.cpp:20-44 of the reference):
//   F16      1 weight  / 2 B
//   Q4_0    32 weights / 18 B   { f16 d; u8 qs[16] }
//   IQ4_NL  32 weights / 18 B   { f16 d; u8 qs[16] }            (codes index the IQ4_NL table)
//   Q8_0    32 weights / 34 B   { f16 d; i8 qs[32] }
//   Q4_K   256 weights / 144 B  { f16 d; f16 dmin; u8 scales[12]; u8 qs[128] }
//   Q5_K   256 weights / 176 B  { f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128] }
//   Q6_K   256 weights / 210 B  { u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d }
//   IQ4_XS 256 weights / 136 B  { f16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128] }
//   Q3_K   256 weights / 110 B  { u8 hmask[32]; u8 qs[64]; u8 scales[12]; f16 d }
//   IQ3_S  256 weights / 110 B  { f16 d; u8 qs[64]; u8 qh[8]; u8 signs[32]; u8 scales[4] }
//
// SLAB layout. Rows are grouped by 64 (one wave64, one row per lane). A row of K weights is
// cut into S = K / 32 "slots" of 32 consecutive weights. Inside a slab every plane is stored
// slot-major, row-minor, so the 64 lanes of a wave reading slot s of their rows touch one
// contiguous run of bytes. A slab holds exactly 64 * row_bytes bytes (no padding), so the
// SLAB image of a matrix is row_bytes * round_up(rows, 64) bytes.
//
// Per-slot 4-bit quant record (16 B): byte t (0..15) holds slot element t in its low nibble
// and slot element t + 16 in its high nibble. Q4_0 blocks already have this order; Q4_K
// sub-blocks are regrouped into it (one slot = one 32-weight sub-block).
//
//   Q4_0  [ q  S x 64 x 16 ][ d  S x 64 x 2 ]
//   Q8_0  [ q  S x 2 x 64 x 16 (the two 16-byte halves of a block, each row-minor) ]
//         [ d  S x 64 x 2 ]
//   Q4_K  [ q  S x 64 x 16 ][ hdr  nb x 64 x 16 : the block's bytes 0..15 (d, dmin, scales) ]
//   Q5_K  [ q  S x 64 x 16 : low 4 bits, as Q4_K ][ qh S x 64 x 4 : top bits, see q5_qh_word() ]
//         [ hdr nb x 64 x 16 : the block's bytes 0..15 ]
//   IQ4_XS [ q  S x 64 x 16 : the block's qs (already in slot order) ]
//          [ hdr nb x 64 x 8 : the block's bytes 0..7 (d, scales_h, scales_l) ]
//   Q6_K  [ ql S x 64 x 16 : low 4 bits, nibble order as above ]
//         [ qh S x 64 x 8  : top 2 bits, see q6_qh_byte() ]
//         [ sc nb x 64 x 16 : the block's int8 scales (bytes 192..207) ]
//         [ d  nb x 64 x 2  : the block's f16 d (bytes 208..209) ]
// with nb = K / 256 super-blocks. Slot j of a Q6_K super-block covers block elements
// 32j .. 32j+31 and uses scales sc[2j] (elements 0..15 of the slot) and sc[2j+1] (16..31).
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define HALO_HD __host__ __device__
#else
#define HALO_HD
#endif

namespace halo_mi {

inline constexpr uint32_t kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ2_K = 10,
                          kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kIQ4_NL = 20, kIQ3_S = 21, kIQ4_XS = 23,
                          kBF16 = 30;
inline constexpr uint32_t kSlabRows = 64;
inline constexpr uint32_t kSlot = 32;  // weights per slot

// Every type of the reference's HIP GEMV test matrix (tests/unit/hip/test_hip_gemv.cpp:217-218)
// plus the rest of its CPU dequantizer's dispatch (BF16, Q4_1, Q5_0, Q5_1, Q2_K; quant.cpp:386-407;
// geometry dtype.cpp:23-53): the GGUF layout takes all of them; is_quant() names those that also
// have a SLAB layout, is_hip_gemv_type() the reference HIP backend's eleven.
HALO_HD constexpr uint32_t block_elems(uint32_t t) {
    return (t == kF32 || t == kF16 || t == kBF16)                                               ? 1u
           : (t == kQ4_0 || t == kQ4_1 || t == kQ5_0 || t == kQ5_1 || t == kQ8_0 || t == kIQ4_NL) ? 32u
           : (t == kQ2_K || t == kQ3_K || t == kQ4_K || t == kQ5_K || t == kQ6_K || t == kIQ4_XS || t == kIQ3_S)
               ? 256u
               : 0u;
}
HALO_HD constexpr uint32_t block_bytes(uint32_t t) {
    return t == kF32                      ? 4u
           : (t == kF16 || t == kBF16)    ? 2u
           : (t == kQ4_0 || t == kIQ4_NL) ? 18u
           : t == kQ4_1                   ? 20u
           : t == kQ5_0                   ? 22u
           : t == kQ5_1                   ? 24u
           : t == kQ8_0                   ? 34u
           : t == kQ2_K                   ? 84u
           : (t == kQ3_K || t == kIQ3_S)  ? 110u
           : t == kQ4_K                   ? 144u
           : t == kQ5_K                   ? 176u
           : t == kQ6_K                   ? 210u
           : t == kIQ4_XS                 ? 136u
                                          : 0u;
}
// The types the reference's HIP GEMV and GET_ROWS take (backends/hip/src/ops.cpp:531-549).
HALO_HD constexpr bool is_hip_gemv_type(uint32_t t) {
    return t == kF32 || t == kF16 || t == kQ4_0 || t == kQ8_0 || t == kQ3_K || t == kQ4_K || t == kQ5_K || t == kQ6_K ||
           t == kIQ3_S || t == kIQ4_NL || t == kIQ4_XS;
}
HALO_HD constexpr bool is_quant(uint32_t t) {
    return t == kQ4_0 || t == kQ8_0 || t == kQ4_K || t == kQ5_K || t == kQ6_K || t == kIQ4_XS;
}

// Byte offsets of the planes inside one slab, for K = cols.
struct SlabGeom {
    uint64_t slab_bytes;
    uint64_t q_off;    // 4-bit quants (ql for Q6_K), or int8 quants for Q8_0
    uint64_t aux_off;  // Q4_0/Q8_0: d plane; Q4_K, IQ4_XS: header plane; Q5_K, Q6_K: qh plane
    uint64_t sc_off;   // Q6_K scale plane; Q5_K header plane
    uint64_t d_off;    // Q6_K d plane
};

HALO_HD inline SlabGeom slab_geom(uint32_t t, uint32_t cols) {
    const uint64_t S = cols / kSlot, nb = cols / 256u;
    SlabGeom g{};
    g.q_off = 0;
    switch (t) {
        case kQ4_0:
            g.aux_off = S * 64 * 16;
            g.slab_bytes = S * 64 * 18;
            break;
        case kQ8_0:
            g.aux_off = S * 64 * 32;
            g.slab_bytes = S * 64 * 34;
            break;
        case kQ4_K:
            g.aux_off = S * 64 * 16;
            g.slab_bytes = nb * 64 * 144;
            break;
        case kQ5_K:
            g.aux_off = S * 64 * 16;
            g.sc_off = g.aux_off + S * 64 * 4;
            g.slab_bytes = nb * 64 * 176;
            break;
        case kQ6_K:
            g.aux_off = S * 64 * 16;
            g.sc_off = g.aux_off + S * 64 * 8;
            g.d_off = g.sc_off + nb * 64 * 16;
            g.slab_bytes = nb * 64 * 210;
            break;
        case kIQ4_XS:
            g.aux_off = S * 64 * 16;
            g.slab_bytes = nb * 64 * 136;
            break;
        default:
            g.slab_bytes = 0;
    }
    return g;
}

HALO_HD inline uint32_t nib(uint8_t b, int hi) { return hi ? (b >> 4) : (b & 0x0Fu); }

// Q6_K slot element t (0..31) of slot j inside the 210-byte block `blk`:
// low 4 bits and top 2 bits, following the block format (quant.cpp:302-327 of the reference).
HALO_HD inline uint32_t q6_lo4(const uint8_t* blk, uint32_t j, uint32_t t) {
    const uint32_t n = j / 4, k = j % 4;
    return nib(blk[64 * n + t + 32 * (k & 1)], k >= 2);
}
HALO_HD inline uint32_t q6_hi2(const uint8_t* blk, uint32_t j, uint32_t t) {
    const uint32_t n = j / 4, k = j % 4;
    return (blk[128 + 32 * n + t] >> (2 * k)) & 3u;
}

// Byte `b` (0..3) of qh dword `w` (0..1) of a Q6_K slot record, from the slot's top-2-bit
// values h[0..31]. The record is arranged so the kernel can OR the bits straight into the
// byte lanes of the 4-bit quant dwords:
//   bits 5:4 -> element 8w+b      (low nibble of ql dword 2w, byte b)
//   bits 7:6 -> element 8w+b+16   (high nibble of ql dword 2w)
//   bits 1:0 -> element 8w+4+b    (low nibble of ql dword 2w+1)
//   bits 3:2 -> element 8w+4+b+16 (high nibble of ql dword 2w+1)
HALO_HD inline uint8_t q6_qh_byte(const uint32_t* h, uint32_t w, uint32_t b) {
    return static_cast<uint8_t>(h[8 * w + 4 + b] | (h[8 * w + 4 + b + 16] << 2) | (h[8 * w + b] << 4) |
                                (h[8 * w + b + 16] << 6));
}

// Q5_K slot record top bits: h[e] (0 or 1) is the fifth bit of slot element e. Bit i + 8 b of
// the word is element 4 i + b's (i < 4) and bit 4 + i + 8 b is element 16 + 4 i + b's, so that
// for dword i of the 4-bit record (elements 4 i .. 4 i + 3 in its low nibbles and 16 + 4 i ..
// in its high nibbles) one shift and the mask 0x10101010 put each bit at bit 4 of its byte:
//   low  codes: (q & 0x0F0F0F0F) | ((word << (4 - i)) & 0x10101010)
//   high codes: ((q >> 4) & 0x0F0F0F0F) | ((word >> i) & 0x10101010)
HALO_HD inline uint32_t q5_qh_word(const uint32_t* h) {
    uint32_t w = 0;
    for (uint32_t i = 0; i < 4; ++i)
        for (uint32_t b = 0; b < 4; ++b)
            w |= (h[4 * i + b] << (i + 8 * b)) | (h[16 + 4 * i + b] << (4 + i + 8 * b));
    return w;
}
// Its inverse for one element.
HALO_HD inline uint32_t q5_qh_bit(uint32_t w, uint32_t e) {
    const uint32_t up = e >> 4, i = (e & 15) >> 2, b = e & 3;
    return (w >> ((up ? 4 + i : i) + 8 * b)) & 1u;
}

// Repack GGUF block `blk` (block index `b` of a row) of the row at lane `r` of a slab.
HALO_HD inline void slab_pack_block(uint32_t t, const uint8_t* blk, uint8_t* slab, const SlabGeom& g,
                                    uint32_t S, uint32_t r, uint32_t b) {
    switch (t) {
        case kQ4_0: {
            uint8_t* q = slab + g.q_off + ((uint64_t)b * 64 + r) * 16;
            for (int i = 0; i < 16; ++i) q[i] = blk[2 + i];
            uint8_t* d = slab + g.aux_off + ((uint64_t)b * 64 + r) * 2;
            d[0] = blk[0];
            d[1] = blk[1];
            break;
        }
        case kQ8_0: {
            for (uint32_t h = 0; h < 2; ++h) {
                uint8_t* q = slab + g.q_off + (((uint64_t)b * 2 + h) * 64 + r) * 16;
                for (int i = 0; i < 16; ++i) q[i] = blk[2 + 16 * h + i];
            }
            uint8_t* d = slab + g.aux_off + ((uint64_t)b * 64 + r) * 2;
            d[0] = blk[0];
            d[1] = blk[1];
            break;
        }
        case kQ4_K: {
            for (uint32_t j = 0; j < 8; ++j) {  // slot j = sub-block j
                const uint32_t grp = j / 2, hi = j % 2;
                uint8_t* q = slab + g.q_off + (((uint64_t)b * 8 + j) * 64 + r) * 16;
                for (uint32_t i = 0; i < 16; ++i) {
                    const uint32_t lo = nib(blk[16 + 32 * grp + i], hi);
                    const uint32_t up = nib(blk[16 + 32 * grp + i + 16], hi);
                    q[i] = static_cast<uint8_t>(lo | (up << 4));
                }
            }
            uint8_t* hdr = slab + g.aux_off + ((uint64_t)b * 64 + r) * 16;
            for (int i = 0; i < 16; ++i) hdr[i] = blk[i];
            break;
        }
        case kQ5_K: {
            // qs group grp (64 elements): low nibbles -> slot 2 grp, high -> slot 2 grp + 1;
            // qh[l] bit j is the top bit of element l of slot j (quant.cpp:271-299)
            for (uint32_t j = 0; j < 8; ++j) {
                const uint32_t grp = j / 2, hi = j % 2;
                uint8_t* q = slab + g.q_off + (((uint64_t)b * 8 + j) * 64 + r) * 16;
                for (uint32_t i = 0; i < 16; ++i) {
                    const uint32_t lo = nib(blk[48 + 32 * grp + i], hi);
                    const uint32_t up = nib(blk[48 + 32 * grp + i + 16], hi);
                    q[i] = static_cast<uint8_t>(lo | (up << 4));
                }
                uint32_t h[32];
                for (uint32_t e = 0; e < 32; ++e) h[e] = (blk[16 + e] >> j) & 1u;
                const uint32_t w = q5_qh_word(h);
                uint8_t* qh = slab + g.aux_off + (((uint64_t)b * 8 + j) * 64 + r) * 4;
                for (uint32_t k = 0; k < 4; ++k) qh[k] = static_cast<uint8_t>(w >> (8 * k));
            }
            uint8_t* hdr = slab + g.sc_off + ((uint64_t)b * 64 + r) * 16;
            for (int i = 0; i < 16; ++i) hdr[i] = blk[i];
            break;
        }
        case kIQ4_XS: {
            for (uint32_t j = 0; j < 8; ++j) {
                uint8_t* q = slab + g.q_off + (((uint64_t)b * 8 + j) * 64 + r) * 16;
                for (uint32_t i = 0; i < 16; ++i) q[i] = blk[8 + 16 * j + i];
            }
            uint8_t* hdr = slab + g.aux_off + ((uint64_t)b * 64 + r) * 8;
            for (int i = 0; i < 8; ++i) hdr[i] = blk[i];
            break;
        }
        case kQ6_K: {
            for (uint32_t j = 0; j < 8; ++j) {
                const uint64_t s = (uint64_t)b * 8 + j;
                uint8_t* ql = slab + g.q_off + (s * 64 + r) * 16;
                uint8_t* qh = slab + g.aux_off + (s * 64 + r) * 8;
                uint32_t h[32];
                for (uint32_t e = 0; e < 32; ++e) h[e] = q6_hi2(blk, j, e);
                for (uint32_t i = 0; i < 16; ++i)
                    ql[i] = static_cast<uint8_t>(q6_lo4(blk, j, i) | (q6_lo4(blk, j, i + 16) << 4));
                for (uint32_t w = 0; w < 2; ++w)
                    for (uint32_t bb = 0; bb < 4; ++bb) qh[4 * w + bb] = q6_qh_byte(h, w, bb);
            }
            uint8_t* sc = slab + g.sc_off + ((uint64_t)b * 64 + r) * 16;
            for (int i = 0; i < 16; ++i) sc[i] = blk[192 + i];
            uint8_t* d = slab + g.d_off + ((uint64_t)b * 64 + r) * 2;
            d[0] = blk[208];
            d[1] = blk[209];
            break;
        }
        default:
            break;
    }
    (void)S;
}

// Exact inverse of slab_pack_block: rebuild GGUF block `b` of lane `r` into `blk`.
HALO_HD inline void slab_unpack_block(uint32_t t, const uint8_t* slab, uint8_t* blk, const SlabGeom& g,
                                      uint32_t S, uint32_t r, uint32_t b) {
    switch (t) {
        case kQ4_0: {
            const uint8_t* q = slab + g.q_off + ((uint64_t)b * 64 + r) * 16;
            const uint8_t* d = slab + g.aux_off + ((uint64_t)b * 64 + r) * 2;
            blk[0] = d[0];
            blk[1] = d[1];
            for (int i = 0; i < 16; ++i) blk[2 + i] = q[i];
            break;
        }
        case kQ8_0: {
            const uint8_t* d = slab + g.aux_off + ((uint64_t)b * 64 + r) * 2;
            blk[0] = d[0];
            blk[1] = d[1];
            for (uint32_t h = 0; h < 2; ++h) {
                const uint8_t* q = slab + g.q_off + (((uint64_t)b * 2 + h) * 64 + r) * 16;
                for (int i = 0; i < 16; ++i) blk[2 + 16 * h + i] = q[i];
            }
            break;
        }
        case kQ4_K: {
            const uint8_t* hdr = slab + g.aux_off + ((uint64_t)b * 64 + r) * 16;
            for (int i = 0; i < 16; ++i) blk[i] = hdr[i];
            for (uint32_t grp = 0; grp < 4; ++grp) {
                const uint8_t* qa = slab + g.q_off + (((uint64_t)b * 8 + 2 * grp) * 64 + r) * 16;
                const uint8_t* qb = slab + g.q_off + (((uint64_t)b * 8 + 2 * grp + 1) * 64 + r) * 16;
                for (uint32_t i = 0; i < 16; ++i) {
                    blk[16 + 32 * grp + i] = static_cast<uint8_t>((qa[i] & 0x0F) | ((qb[i] & 0x0F) << 4));
                    blk[16 + 32 * grp + i + 16] = static_cast<uint8_t>((qa[i] >> 4) | (qb[i] & 0xF0));
                }
            }
            break;
        }
        case kQ5_K: {
            const uint8_t* hdr = slab + g.sc_off + ((uint64_t)b * 64 + r) * 16;
            for (int i = 0; i < 16; ++i) blk[i] = hdr[i];
            for (int i = 16; i < 48; ++i) blk[i] = 0;
            for (uint32_t grp = 0; grp < 4; ++grp) {
                const uint8_t* qa = slab + g.q_off + (((uint64_t)b * 8 + 2 * grp) * 64 + r) * 16;
                const uint8_t* qb = slab + g.q_off + (((uint64_t)b * 8 + 2 * grp + 1) * 64 + r) * 16;
                for (uint32_t i = 0; i < 16; ++i) {
                    blk[48 + 32 * grp + i] = static_cast<uint8_t>((qa[i] & 0x0F) | ((qb[i] & 0x0F) << 4));
                    blk[48 + 32 * grp + i + 16] = static_cast<uint8_t>((qa[i] >> 4) | (qb[i] & 0xF0));
                }
            }
            for (uint32_t j = 0; j < 8; ++j) {
                const uint8_t* qh = slab + g.aux_off + (((uint64_t)b * 8 + j) * 64 + r) * 4;
                const uint32_t w = (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) | ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
                for (uint32_t e = 0; e < 32; ++e) blk[16 + e] |= static_cast<uint8_t>(q5_qh_bit(w, e) << j);
            }
            break;
        }
        case kIQ4_XS: {
            const uint8_t* hdr = slab + g.aux_off + ((uint64_t)b * 64 + r) * 8;
            for (int i = 0; i < 8; ++i) blk[i] = hdr[i];
            for (uint32_t j = 0; j < 8; ++j) {
                const uint8_t* q = slab + g.q_off + (((uint64_t)b * 8 + j) * 64 + r) * 16;
                for (uint32_t i = 0; i < 16; ++i) blk[8 + 16 * j + i] = q[i];
            }
            break;
        }
        case kQ6_K: {
            for (int i = 0; i < 192; ++i) blk[i] = 0;
            for (uint32_t j = 0; j < 8; ++j) {
                const uint64_t s = (uint64_t)b * 8 + j;
                const uint8_t* ql = slab + g.q_off + (s * 64 + r) * 16;
                const uint8_t* qh = slab + g.aux_off + (s * 64 + r) * 8;
                const uint32_t n = j / 4, k = j % 4;
                for (uint32_t e = 0; e < 32; ++e) {
                    const uint32_t lo4 = e < 16 ? (ql[e] & 0x0F) : (ql[e - 16] >> 4);
                    // invert q6_qh_byte: find the byte and bit pair holding element e
                    const uint32_t base = e & 15, up = e >> 4;  // e = base + 16 * up
                    const uint32_t w = base / 8, rem = base % 8;
                    const uint32_t bb = rem % 4, second = rem / 4;  // second: element 8w+4+b
                    const uint32_t shift = second ? (up ? 2 : 0) : (up ? 6 : 4);
                    const uint32_t hi2 = (qh[4 * w + bb] >> shift) & 3u;
                    blk[64 * n + e + 32 * (k & 1)] |= static_cast<uint8_t>(k >= 2 ? (lo4 << 4) : lo4);
                    blk[128 + 32 * n + e] |= static_cast<uint8_t>(hi2 << (2 * k));
                }
            }
            const uint8_t* sc = slab + g.sc_off + ((uint64_t)b * 64 + r) * 16;
            const uint8_t* d = slab + g.d_off + ((uint64_t)b * 64 + r) * 2;
            for (int i = 0; i < 16; ++i) blk[192 + i] = sc[i];
            blk[208] = d[0];
            blk[209] = d[1];
            break;
        }
        default:
            break;
    }
    (void)S;
}

}  // namespace halo_mi
