// gfx950 exact-product small-M GEMM: k_gemm_sx<T, PAIR, NP> for 1..8 rows of x.
//
// The slab GEMV's arithmetic (exact products, fp32 sums) on v_mfma_f32_32x32x16_bf16 tiles:
//   - B: the weights' integer codes themselves as bf16 bit patterns (a code c < 256 in the low
//     bits of a bf16 is exactly c 2^-133), unpacked with masks only;
//   - A: x scaled by a power of two per 256-weight group and split exactly into three bf16
//     pieces, one A row per piece (vector v's pieces are rows of the same lane, so its dot is
//     the sum of three of the lane's accumulators);
//   - the per-slot scales, mins and code offsets are applied per lane after each slot's two
//     MFMAs, as the reference's expressions factor them, and each group's sum is brought back
//     with ldexp.
// Rows and the arithmetic are those of the slab GEMV (same bound), but a workgroup streams two
// units (256 W rows) x one K chunk, one 64-row slab per wave, and no wave dequantizes: per slot
// and row block a lane unpacks 16 codes with about 10 masks and folds its vectors' sums,
// instead of converting and rounding 16 weights. Each lane loads its row's whole 16-byte slot
// record (one 1 KB load instruction per wave and slot: half the load instructions of 8-byte
// loads, which is what lets the stream run at the plain-read rate) and v_permlane32_swap hands
// each lane half the bytes of the MFMA B layout. x enters LDS once per workgroup; the chunks'
// partials go to the workspace and k_sx_reduce adds them in chunk order. The K split is the one
// planned for 8 vectors whatever n_vec is, so a row's sums do not depend on the other vectors of
// the batch: MFMA output element (i, j) takes only A row i and B column j, and nothing else in a
// row's arithmetic looks at another vector. (A split planned per vector count, and a form with
// two waves per slab taking alternate super-blocks, measured slower at every vector count on
// the 17408 x 5120 and 5120 x 17408 shapes.)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "device.h"
#include "launch.h"

namespace halo_mi {
namespace {

using namespace dev;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kSxOob = 0x80000000u;  // buffer offset past every resource: the load returns 0
constexpr int kSxDepth = 8;               // slots of weight records in flight per wave (8 KB)
constexpr uint32_t kSxLdsMax = 52 * 1024;  // x pieces, sums and exponents of one K chunk
constexpr uint32_t kSxPairs = 10;          // (vector, group) pairs of x per wave of a four-wave fill
constexpr uint32_t kSxWgsPerCu = 1;        // workgroups per CU the K split aims for

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sx_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
// Weight records, read once per launch: nontemporal loads (cache policy 2; measured on MI355X
// against the default: Q4_K gate/up M = 4 30.6 -> 28.6 us, 17408 x 5120 M = 4 18.5 -> 17.9)
__device__ __forceinline__ uint4 sx_ld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
    return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ uint2 sx_ld64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 2);
    return uint2{v[0], v[1]};
}
__device__ __forceinline__ uint32_t sx_ld32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 2);
}
__device__ __forceinline__ uint32_t sx_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 2);
}

template <int CTRL>
__device__ __forceinline__ float sx_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t sx_dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;

__device__ __forceinline__ uint32_t sx_wave_max(uint32_t v) {
    v = max(v, sx_dpp_u<kXor1>(v));
    v = max(v, sx_dpp_u<kXor2>(v));
    v = max(v, sx_dpp_u<kHalfMirror>(v));
    v = max(v, sx_dpp_u<kMirror>(v));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}

__device__ __forceinline__ uint32_t sx_pack(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
}
// (a, b) -> three bf16 pairs whose sums are exactly a and b (each residual is exact in fp32 and
// has at most 16, then 8 significant bits, so the third piece is the residual itself)
__device__ __forceinline__ void sx_split3(float a, float b, uint32_t (&p)[3]) {
    p[0] = sx_pack(a, b);
    const float ra = a - __uint_as_float(p[0] << 16), rb = b - __uint_as_float(p[0] & 0xFFFF0000u);
    p[1] = sx_pack(ra, rb);
    p[2] = sx_pack(ra - __uint_as_float(p[1] << 16), rb - __uint_as_float(p[1] & 0xFFFF0000u));
}

// Byte codes (e0, e1, e2, e3) of one dword -> the two bf16 pairs (e0, e2), (e1, e3).
__device__ __forceinline__ uint32_t sx_b02(uint32_t L) { return L & 0x00FF00FFu; }
__device__ __forceinline__ uint32_t sx_b13(uint32_t L) { return __builtin_amdgcn_perm(0u, L, 0x0C030C01u); }

struct SxArgs {
    const uint8_t* w0;  // gate (PAIR) or the matrix
    const uint8_t* w1;  // up (PAIR) or null
    const float* x;
    uint64_t x_stride;
    float* partials;  // kchunks > 1: [unit][chunk][32 rows][128 columns], rows < n_vec written
    uint32_t rows, cols, n_vec, kchunks;
    float* y;  // kchunks == 1: the result (SiLU(gate) * up for the pair), n_vec rows y_stride apart
    uint64_t y_stride;
};

// One lane's records of one slot: lane l loads row l's whole 16-byte code record (a wave reads
// the slab's 1 KB slot record in one 16-byte load per lane) and the side words that go with it;
// and of one super-block, the header fields of row l. Offsets as the SLAB layout.
template <uint32_t T>
struct SxQ {
    uint4 q;    // the code record (Q8_0: its first 16 bytes)
    uint4 q2;   // Q8_0: the second 16 bytes
    uint2 aux;  // Q5_K: .x the top-bit word; Q6_K: the two halves' top-bit words; Q4_0 / Q8_0: .x the f16 d
};
template <uint32_t T>
struct SxH {
    uint4 hdr;  // Q4_K / Q5_K: bytes 0..15; IQ4_XS: bytes 0..7; Q6_K: the 16 scales
    uint32_t d;  // Q6_K: the f16 d
};
// What lane (r, h) = (l % 32, l / 32) needs of one 32-row block b of the slab: half h of row
// 32 b + r's record (the B operand layout of v_mfma_f32_32x32x16_bf16) and that row's side words.
struct SxV {
    uint32_t q0, q1;  // the 8 code bytes (Q8_0: of the first 16 bytes)
    uint32_t r0, r1;  // Q8_0: of the second 16 bytes
    uint32_t aux;
};

// v_permlane32_swap: {a, b} -> {a with its upper 32 lanes replaced by b's lower 32, b with its
// lower 32 lanes replaced by a's upper 32}. With a = bytes 0..7 and b = bytes 8..15 of each
// lane's own row, the first result is half h of row r (block 0) and the second half h of row
// r + 32 (block 1); with a = b = a per-row word, the row r and row r + 32 words.
__device__ __forceinline__ uint2 sx_swap(uint32_t a, uint32_t b) {
    const auto v = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    return uint2{v[0], v[1]};
}

template <uint32_t T>
__device__ __forceinline__ void sx_views(const SxQ<T>& R, SxV (&V)[2]) {
    uint2 t = sx_swap(R.q.x, R.q.z);
    V[0].q0 = t.x, V[1].q0 = t.y;
    t = sx_swap(R.q.y, R.q.w);
    V[0].q1 = t.x, V[1].q1 = t.y;
    if constexpr (T == kQ8_0) {
        t = sx_swap(R.q2.x, R.q2.z);
        V[0].r0 = t.x, V[1].r0 = t.y;
        t = sx_swap(R.q2.y, R.q2.w);
        V[0].r1 = t.x, V[1].r1 = t.y;
    }
    if constexpr (T == kQ6_K) {
        t = sx_swap(R.aux.x, R.aux.y);  // half h's word of rows r and r + 32
        V[0].aux = t.x, V[1].aux = t.y;
    } else if constexpr (T == kQ5_K || T == kQ4_0 || T == kQ8_0) {
        t = sx_swap(R.aux.x, R.aux.x);
        V[0].aux = t.x, V[1].aux = t.y;
    }
}
template <uint32_t T>
__device__ __forceinline__ void sx_hviews(const SxH<T>& H, SxH<T> (&V)[2]) {
    uint2 t = sx_swap(H.hdr.x, H.hdr.x);
    V[0].hdr.x = t.x, V[1].hdr.x = t.y;
    t = sx_swap(H.hdr.y, H.hdr.y);
    V[0].hdr.y = t.x, V[1].hdr.y = t.y;
    if constexpr (T != kIQ4_XS) {
        t = sx_swap(H.hdr.z, H.hdr.z);
        V[0].hdr.z = t.x, V[1].hdr.z = t.y;
        t = sx_swap(H.hdr.w, H.hdr.w);
        V[0].hdr.w = t.x, V[1].hdr.w = t.y;
    }
    if constexpr (T == kQ6_K) {
        t = sx_swap(H.d, H.d);
        V[0].d = t.x, V[1].d = t.y;
    }
}

template <uint32_t T>
__device__ __forceinline__ void sx_load_q(SxQ<T>& R, __amdgpu_buffer_rsrc_t w, const SlabGeom& g, uint32_t lane, uint32_t s,
                                          bool live) {
    auto so = [&](uint64_t x) { return live ? (uint32_t)x : kSxOob; };
    if constexpr (T == kQ8_0) {
        R.q = sx_ld128(w, lane * 16, so(g.q_off + s * 2048));
        R.q2 = sx_ld128(w, lane * 16, so(g.q_off + s * 2048 + 1024));
    } else {
        R.q = sx_ld128(w, lane * 16, so(g.q_off + s * 1024));
    }
    if constexpr (T == kQ5_K) R.aux.x = sx_ld32(w, lane * 4, so(g.aux_off + s * 256));
    if constexpr (T == kQ6_K) R.aux = sx_ld64(w, lane * 8, so(g.aux_off + s * 512));
    if constexpr (T == kQ4_0 || T == kQ8_0) R.aux.x = sx_ld16(w, lane * 2, so(g.aux_off + s * 128));
}

template <uint32_t T>
__device__ __forceinline__ void sx_load_h(SxH<T>& H, __amdgpu_buffer_rsrc_t w, const SlabGeom& g, uint32_t lane, uint32_t sb,
                                          bool live) {
    auto so = [&](uint64_t x) { return live ? (uint32_t)x : kSxOob; };
    if constexpr (T == kQ4_K) H.hdr = sx_ld128(w, lane * 16, so(g.aux_off + sb * 1024));
    if constexpr (T == kQ5_K) H.hdr = sx_ld128(w, lane * 16, so(g.sc_off + sb * 1024));
    if constexpr (T == kIQ4_XS) {
        const uint2 v = sx_ld64(w, lane * 8, so(g.aux_off + sb * 512));
        H.hdr = uint4{v.x, v.y, 0u, 0u};
    }
    if constexpr (T == kQ6_K) {
        H.hdr = sx_ld128(w, lane * 16, so(g.sc_off + sb * 1024));
        H.d = sx_ld16(w, lane * 2, so(g.d_off + sb * 128));
    }
}

// The two B operands of one slot for one row block: K half 0 (record elements 8h + (0, 2, 1, 3,
// 4, 6, 5, 7)) and K half 1 (16 + the same). Q4_K / Q4_0 deliver K half 1 as 16 q (the A side
// divides x by 16).
template <uint32_t T>
__device__ __forceinline__ void sx_codes(const SxV& R, uint32_t h, u32x4_t& b0, u32x4_t& b1) {
    const uint32_t Q0 = R.q0, Q1 = R.q1;
    if constexpr (T == kQ4_K || T == kQ4_0) {
        const uint32_t S0 = Q0 >> 8, S1 = Q1 >> 8;
        b0 = u32x4_t{Q0 & 0x000F000Fu, S0 & 0x000F000Fu, Q1 & 0x000F000Fu, S1 & 0x000F000Fu};
        b1 = u32x4_t{Q0 & 0x00F000F0u, S0 & 0x00F000F0u, Q1 & 0x00F000F0u, S1 & 0x00F000F0u};
    } else {
        uint32_t lo[2], hi[2];
        if constexpr (T == kQ5_K) {
            // record dword i = 2 h + w: fifth bits at (qh << (4 - i)) and (qh >> i), bit 4 of each byte
            const uint32_t hq = R.aux >> (2 * h);
            const uint32_t Q[2] = {Q0, Q1};
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                lo[w] = (Q[w] & 0x0F0F0F0Fu) | ((hq << (4 - w)) & 0x10101010u);
                hi[w] = ((Q[w] >> 4) & 0x0F0F0F0Fu) | ((hq >> w) & 0x10101010u);
            }
        } else if constexpr (T == kIQ4_XS) {
            lo[0] = iq4_lookup4(Q0);
            lo[1] = iq4_lookup4(Q1);
            hi[0] = iq4_lookup4(Q0 >> 4);
            hi[1] = iq4_lookup4(Q1 >> 4);
        } else if constexpr (T == kQ6_K) {
            const uint32_t hq = R.aux;
            lo[0] = (Q0 & 0x0F0F0F0Fu) | (hq & 0x30303030u);
            lo[1] = (Q1 & 0x0F0F0F0Fu) | ((hq << 4) & 0x30303030u);
            hi[0] = ((Q0 >> 4) & 0x0F0F0F0Fu) | ((hq >> 2) & 0x30303030u);
            hi[1] = ((Q1 >> 4) & 0x0F0F0F0Fu) | ((hq << 2) & 0x30303030u);
        } else {  // Q8_0: q + 128 as unsigned bytes
            lo[0] = Q0 ^ 0x80808080u;
            lo[1] = Q1 ^ 0x80808080u;
            hi[0] = R.r0 ^ 0x80808080u;
            hi[1] = R.r1 ^ 0x80808080u;
        }
        b0 = u32x4_t{sx_b02(lo[0]), sx_b13(lo[0]), sx_b02(lo[1]), sx_b13(lo[1])};
        b1 = u32x4_t{sx_b02(hi[0]), sx_b13(hi[0]), sx_b02(hi[1]), sx_b13(hi[1])};
    }
}

// A row of the 32x32 tile that holds piece c of vector v: vector v lives in the lane half v & 1
// of the accumulator layout (rows 8 i + 4 (v & 1) + j), at accumulator index k = 3 (v >> 1) + c.
__host__ __device__ constexpr uint32_t sx_row(uint32_t v, uint32_t c) {
    const uint32_t k = 3 * (v >> 1) + c;
    return 8 * (k >> 2) + 4 * (v & 1) + (k & 3);
}
// A rows stored in LDS per (slot, K half, lane half): every row a vector's piece uses.
__host__ __device__ constexpr uint32_t sx_rows(int np) { return np <= 2 ? 16u : 32u; }
// LDS bytes per slot of the chunk: the pieces, then per K half and vector the x sum.
__host__ __device__ constexpr uint32_t sx_slot_bytes(int np) { return 64u * sx_rows(np) + 2u * 8u * 4u; }

template <uint32_t T, bool PAIR, int NP>
__global__ __launch_bounds__(256, 3) void k_gemm_sx(SxArgs a) {
    extern __shared__ uint4 sxl[];
    constexpr uint32_t RS = sx_rows(NP);
    constexpr bool kHi16 = T == kQ4_K || T == kQ4_0;  // K half 1's codes arrive as 16 q
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t S = a.cols / kSlot;
    const SlabGeom g = slab_geom(T, a.cols);
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    const uint32_t units = PAIR ? slabs : (slabs + 1) / 2;
    const uint32_t chunk = blockIdx.x % a.kchunks;
    const uint32_t ng = S / 8, base = ng / a.kchunks, extra = ng % a.kchunks;
    const uint32_t g0 = chunk * base + min(chunk, extra);
    const uint32_t ngc = base + (chunk < extra ? 1u : 0u);  // super-blocks of this chunk
    const uint32_t s_begin = 8 * g0, s_end = 8 * (g0 + ngc);
    const uint32_t ns = s_end - s_begin;
    // wave w: unit 2 (blockIdx / kchunks) + w / 2, matrix w % 2 (PAIR: gate / up; else the
    // unit's two slabs), all 64 rows of that slab
    const uint32_t unit = 2 * (blockIdx.x / a.kchunks) + ((wave >> 1) & 1u), mat = wave & 1u;
    const bool live_unit = unit < units;  // an odd unit count leaves the last workgroup's second unit empty
    const uint32_t lu = min(unit, units - 1);
    const uint32_t r = lane & 31u, h = lane >> 5;
    const uint8_t* slab_ptr;
    if constexpr (PAIR) {
        slab_ptr = (mat ? a.w1 : a.w0) + (uint64_t)lu * g.slab_bytes;
    } else {
        // a missing second slab reads the last one again: its outputs are never stored
        slab_ptr = a.w0 + (uint64_t)min(2 * lu + mat, slabs - 1) * g.slab_bytes;
    }
    const __amdgpu_buffer_rsrc_t wres = sx_rsrc(slab_ptr, (uint32_t)g.slab_bytes);
    // LDS: pieces [slot][K half][lane half][RS rows] x 16 B, then x sums [slot][K half][8 vectors],
    // then the groups' exponents [group][8 vectors]
    uint8_t* lds = reinterpret_cast<uint8_t*>(sxl);
    float* xsum = reinterpret_cast<float*>(lds + (size_t)ns * 64 * RS);
    int* expo = reinterpret_cast<int*>(xsum + (size_t)ns * 16);

    // ---- x of the chunk into LDS: one wave per (vector, group) pair. The x loads are issued
    // first, then the weight stream's first loads, then the split (which waits only for x).
    constexpr uint32_t kWaves = 4;
    constexpr int kPairs = (int)((4 * kSxPairs + kWaves - 1) / kWaves);
    const uint32_t npairs = a.n_vec * ngc;
    float4 xv[kPairs];
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const uint32_t pi = wave + kWaves * i;
        xv[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (pi < npairs) {  // four dword loads: x rows need only 4-byte alignment
            const uint32_t v = pi % a.n_vec, gg = pi / a.n_vec;
            const float* xp = a.x + (uint64_t)v * a.x_stride + 256 * (g0 + gg) + 4 * lane;
            xv[i] = float4{xp[0], xp[1], xp[2], xp[3]};
        }
    }
    SxQ<T> R[kSxDepth];
    SxH<T> H[2];
    auto load_q = [&](int q, uint32_t s) { sx_load_q<T>(R[q], wres, g, lane, s, s < s_end); };
    auto load_h = [&](int i, uint32_t sb) { sx_load_h<T>(H[i], wres, g, lane, sb, 8 * sb < s_end); };
    const uint32_t sb0 = s_begin / 8;  // the chunk's first super-block
    load_h(0, sb0);
    load_h(1, sb0 + 1);
#pragma unroll
    for (int q = 0; q < kSxDepth; ++q) load_q(q, 8 * sb0 + q);
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
        const uint32_t pi = wave + kWaves * i;
        if (pi >= npairs) break;  // wave-uniform
        const uint32_t v = pi % a.n_vec, gg = pi / a.n_vec;
        const float xr[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        uint32_t mb = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) mb = max(mb, __float_as_uint(xr[k]) & 0x7FFFFFFFu);
        mb = sx_wave_max(mb);
        const int e = min(max((int)(mb >> 23) - 127, -100), 127);
        const int sxp = 100 - e;  // the largest |x| * 2^sxp is about 2^100
        if (lane == 0) expo[gg * 8 + v] = 33 + e;  // 133 - sxp: the group's sums back to fp32 units
        // lane: slot 8 gg + lane / 8, K half kh = bit 2 of lane, lane half hb = bit 1, and
        // within the 8 elements the first or second four (bit 0)
        const uint32_t ls = 8 * gg + (lane >> 3), kh = (lane >> 2) & 1u, hb = (lane >> 1) & 1u;
        const int sh = sxp - ((kHi16 && kh) ? 4 : 0);
        uint32_t p02[3], p13[3];
        sx_split3(ldexpf(xr[0], sh), ldexpf(xr[2], sh), p02);
        sx_split3(ldexpf(xr[1], sh), ldexpf(xr[3], sh), p13);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const uint32_t m = sx_row(v, c);
            *reinterpret_cast<uint2*>(lds + (((ls * 2 + kh) * 2 + hb) * RS + m) * 16 + 8 * (lane & 1u)) =
                uint2{p02[c], p13[c]};
        }
        float sm = (xr[0] + xr[1]) + (xr[2] + xr[3]);
        sm += sx_dpp<kXor1>(sm);
        sm += sx_dpp<kXor2>(sm);
        if ((lane & 3u) == 0) xsum[(ls * 2 + kh) * 8 + v] = ldexpf(sm, sxp - 133);
    }
    __syncthreads();

    // ---- the slots: per row block, two MFMAs into a fresh tile, then the fold into each
    // vector's sums
    const uint32_t hd = h;  // the accumulator layout's lane half: vectors hd, hd + 2, ...
    const uint32_t arow = min(r, RS - 1);  // this lane's A row (rows past RS hold no piece)
    const uint8_t* abase = lds + (h * RS + arow) * 16;
    const uint32_t nv_lane = (a.n_vec + 1 - hd) / 2;  // vectors of this lane half
    float acc[2][NP];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[b][p] = 0.0f;
    float sa[2][NP], sb[2][NP];
    SxH<T> HV[2];  // the current super-block's header words of rows r and r + 32
    auto group_begin = [&](int hi) {
        sx_hviews<T>(H[hi], HV);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int p = 0; p < NP; ++p) sa[b][p] = sb[b][p] = 0.0f;
    };
    auto slot = [&](int q, uint32_t s) {
        const int qr = q & (kSxDepth - 1);
        const uint32_t ls = s - s_begin, j = (uint32_t)(q & 7);
        SxV V[2];
        sx_views<T>(R[qr], V);
        const uint4 a0 = *reinterpret_cast<const uint4*>(abase + (ls * 2 + 0) * 2 * RS * 16);
        const uint4 a1 = *reinterpret_cast<const uint4*>(abase + (ls * 2 + 1) * 2 * RS * 16);
        const float* xs = xsum + ls * 16 + hd;  // [K half][vector], vector 2 p + hd
        load_q(qr, s + 8);  // the next super-block
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            u32x4_t b0, b1;
            sx_codes<T>(V[b], h, b0, b1);
            floatx16 D0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a0), __builtin_bit_cast(bf16x8, b0),
                                                                  floatx16{}, 0, 0, 0);
            if constexpr (T == kQ6_K) {
                // the two halves have their own scales
                const floatx16 D1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a1),
                                                                            __builtin_bit_cast(bf16x8, b1), floatx16{}, 0, 0, 0);
                const SxH<T>& Hs = HV[b];
                const uint32_t w = (j >> 1) == 0 ? Hs.hdr.x : (j >> 1) == 1 ? Hs.hdr.y : (j >> 1) == 2 ? Hs.hdr.z : Hs.hdr.w;
                const float sA = sbyte(w, 2 * (j & 1)), sB = sbyte(w, 2 * (j & 1) + 1);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const float dlo = (D0[3 * p] + D0[3 * p + 1]) + D0[3 * p + 2];
                    const float dhi = (D1[3 * p] + D1[3 * p + 1]) + D1[3 * p + 2];
                    sa[b][p] = fmaf(sA, fmaf(-32.0f, xs[2 * p], dlo), sa[b][p]);
                    sa[b][p] = fmaf(sB, fmaf(-32.0f, xs[8 + 2 * p], dhi), sa[b][p]);
                }
            } else {
                D0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a1), __builtin_bit_cast(bf16x8, b1), D0, 0,
                                                             0, 0);
                float dot[NP], xss[NP];
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    dot[p] = (D0[3 * p] + D0[3 * p + 1]) + D0[3 * p + 2];
                    xss[p] = xs[2 * p] + xs[8 + 2 * p];
                }
                if constexpr (T == kQ4_K || T == kQ5_K) {
                    const SxH<T>& Hs = HV[b];
                    uint32_t sc, m;
                    q4k_sc_m(Hs.hdr.y, Hs.hdr.z, Hs.hdr.w, j, sc, m);
                    const float fsc = (float)sc, fm = (float)m;
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        sa[b][p] = fmaf(fsc, dot[p], sa[b][p]);
                        sb[b][p] = fmaf(fm, xss[p], sb[b][p]);
                    }
                } else if constexpr (T == kIQ4_XS) {
                    const SxH<T>& Hs = HV[b];
                    const float fl = (float)iq4xs_ls(Hs.hdr.x >> 16, Hs.hdr.y, j);
#pragma unroll
                    for (int p = 0; p < NP; ++p) sa[b][p] = fmaf(fl, fmaf(-128.0f, xss[p], dot[p]), sa[b][p]);
                } else {  // Q4_0, Q8_0: the slot's own d
                    const float d = h2f(V[b].aux);
                    constexpr float off = T == kQ4_0 ? -8.0f : -128.0f;
#pragma unroll
                    for (int p = 0; p < NP; ++p) sa[b][p] = fmaf(d, fmaf(off, xss[p], dot[p]), sa[b][p]);
                }
            }
        }
    };
    auto group_end = [&](uint32_t gg) {
        const int* ex = expo + gg * 8 + hd;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float d = 1.0f, dmin = 0.0f;
            if constexpr (T == kQ4_K || T == kQ5_K) {
                d = h2f(HV[b].hdr.x & 0xFFFFu);
                dmin = h2f(HV[b].hdr.x >> 16);
            } else if constexpr (T == kIQ4_XS) {
                d = h2f(HV[b].hdr.x & 0xFFFFu);
            } else if constexpr (T == kQ6_K) {
                d = h2f(HV[b].d);
            }
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                float grp;
                if constexpr (T == kQ4_K || T == kQ5_K) grp = fmaf(d, sa[b][p], -(dmin * sb[b][p]));
                else if constexpr (T == kQ4_0 || T == kQ8_0) grp = sa[b][p];
                else grp = d * sa[b][p];
                acc[b][p] += ldexpf(grp, ex[2 * p]);
            }
        }
    };
    // the chunk's super-blocks: H[0] serves the first of each pair, H[1] the second, each
    // reloaded with the super-block two ahead once its own is done
    for (uint32_t i0 = 8 * sb0; i0 < s_end; i0 += 16) {
        group_begin(0);
#pragma unroll
        for (int q = 0; q < 8; ++q) slot(q, i0 + q);
        group_end((i0 - s_begin) / 8);
        load_h(0, i0 / 8 + 2);
        if (i0 + 8 >= s_end) break;
        group_begin(1);
#pragma unroll
        for (int q = 0; q < 8; ++q) slot(q, i0 + 8 + q);
        group_end((i0 - s_begin) / 8 + 1);
        load_h(1, i0 / 8 + 3);
    }
    if (!live_unit) return;
    if (a.kchunks > 1) {
        // the chunks' sums go to the workspace; k_sx_reduce adds them in chunk order
        float* P = a.partials + ((uint64_t)unit * a.kchunks + chunk) * 32 * 128 + 64 * mat + r;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int p = 0; p < NP; ++p)
                if ((uint32_t)p < nv_lane) P[(2 * p + hd) * 128 + 32 * b] = acc[b][p];
        return;
    }
    // one K chunk: y directly; row 32 b + r of the wave's slab, vectors 2 p + hd
    if constexpr (PAIR) {
        // gate (mat 0) and up (mat 1) of a unit are two waves: up goes through LDS (the x pieces
        // are dead once every wave of the workgroup is past the loop)
        __syncthreads();
        float* ex = reinterpret_cast<float*>(lds) + ((wave >> 1) & 1u) * (2 * NP * 64) + lane;
        if (mat == 1) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int p = 0; p < NP; ++p) ex[(b * NP + p) * 64] = acc[b][p];
        }
        __syncthreads();
        if (mat == 1) return;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint32_t row = unit * kSlabRows + 32 * b + r;
#pragma unroll
            for (int p = 0; p < NP; ++p)
                if ((uint32_t)p < nv_lane && row < a.rows)
                    a.y[(uint64_t)(2 * p + hd) * a.y_stride + row] = silu_f(acc[b][p]) * ex[(b * NP + p) * 64];
        }
    } else {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint32_t row = 2 * unit * kSlabRows + 64 * mat + 32 * b + r;
#pragma unroll
            for (int p = 0; p < NP; ++p)
                if ((uint32_t)p < nv_lane && row < a.rows) a.y[(uint64_t)(2 * p + hd) * a.y_stride + row] = acc[b][p];
        }
    }
}

// The chunks' sums in chunk order, 0 + c0 + c1 + ..., and the epilogue (SiLU(gate) * up for the
// pair, the IEEE SiLU of the slab GEMV pair). One thread per (unit, vector, output column): the
// loads of 8 chunks are in flight together, so a launch of up to 8 chunks is one memory round trip.
template <bool PAIR>
__global__ __launch_bounds__(256) void k_sx_reduce(const float* __restrict__ partials, float* __restrict__ y,
                                                   uint64_t y_stride, uint32_t rows, uint32_t units, uint32_t n_vec,
                                                   uint32_t kc) {
    constexpr uint32_t NC = PAIR ? 64 : 128;  // output columns of a unit
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)units * n_vec * NC) return;
    const uint32_t u = (uint32_t)(idx / (n_vec * NC)), e = (uint32_t)(idx % (n_vec * NC));
    const uint32_t v = e / NC, n = e % NC;
    const uint32_t row = PAIR ? u * kSlabRows + n : 2 * u * kSlabRows + n;
    if (row >= rows) return;
    const float* P = partials + (uint64_t)u * kc * 32 * 128 + v * 128 + n;
    constexpr uint64_t CS = 32 * 128;  // floats per chunk
    float s0 = 0.0f, s1 = 0.0f;
    for (uint32_t c0 = 0; c0 < kc; c0 += 8) {
        float q0[8], q1[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint64_t off = (uint64_t)min(c0 + i, kc - 1) * CS;
            q0[i] = P[off];
            if constexpr (PAIR) q1[i] = P[off + 64];
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            if (c0 + i >= kc) break;
            s0 += q0[i];
            if constexpr (PAIR) s1 += q1[i];
        }
    }
    y[(uint64_t)v * y_stride + row] = PAIR ? silu_f(s0) * s1 : s0;
}

template <bool PAIR, int NP>
void launch_sx_np(uint32_t type, const SxArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL((k_gemm_sx<kQ4_0, PAIR, NP>), grid, dim3(256), lds, st, a); break;
        case kQ8_0: hipLaunchKernelGGL((k_gemm_sx<kQ8_0, PAIR, NP>), grid, dim3(256), lds, st, a); break;
        case kQ4_K: hipLaunchKernelGGL((k_gemm_sx<kQ4_K, PAIR, NP>), grid, dim3(256), lds, st, a); break;
        case kQ5_K: hipLaunchKernelGGL((k_gemm_sx<kQ5_K, PAIR, NP>), grid, dim3(256), lds, st, a); break;
        case kIQ4_XS: hipLaunchKernelGGL((k_gemm_sx<kIQ4_XS, PAIR, NP>), grid, dim3(256), lds, st, a); break;
        default: hipLaunchKernelGGL((k_gemm_sx<kQ6_K, PAIR, NP>), grid, dim3(256), lds, st, a); break;
    }
}

uint32_t sx_cu_count() {
    static const uint32_t cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return (uint32_t)std::max(n, 1);
    }();
    return cus;
}

}  // namespace

bool gemm_sx_plan(uint32_t units, uint32_t cols, uint32_t n_vec, uint32_t* kc, size_t* lds) {
    const uint32_t S = cols / kSlot;
    if (n_vec < 1 || n_vec > kGemmSxMaxRows || cols % 256 != 0 || S == 0 || units == 0) return false;
    // the K split is planned for the most vectors a launch takes, so that every n_vec gets the
    // same chunks (and the same sums)
    const uint32_t pv = kGemmSxMaxRows;
    // with the fused norm the launch normalizes all n_vec rows into the workspace's norm buffer
    // at once; the plan refuses shapes past it with or without the norm, so that the auto choice
    // stays a function of the shape only
    if ((uint64_t)pv * cols > kNormFloats) return false;
    const uint32_t ng = S / 8;
    const auto group_bytes = [](uint32_t nv) { return 8 * sx_slot_bytes((int)(nv + 1) / 2) + 8 * 4; };
    // a chunk's (vector, group) pairs: at most 4 kSxPairs per workgroup (the fill's registers;
    // the two-wave form spreads them over eight waves)
    const uint32_t max_groups = std::min<uint32_t>(kSxLdsMax / group_bytes(pv), 4 * kSxPairs / pv);
    const uint32_t kc_min = (ng + max_groups - 1) / max_groups;
    const uint32_t wgs = (units + 1) / 2;  // a workgroup streams two units
    uint32_t k = std::clamp<uint32_t>((kSxWgsPerCu * sx_cu_count() + wgs - 1) / wgs, kc_min, ng);
    while (k > kc_min && (uint64_t)units * k * 32 * 128 > kPartialFloats) --k;
    if ((uint64_t)units * k * 32 * 128 > kPartialFloats) return false;
    *kc = k;
    *lds = (size_t)((ng + k - 1) / k) * group_bytes(n_vec);
    return true;
}

int launch_gemm_sx(uint32_t type, bool pair, const GemmArgs& g, Workspace* ws, uint32_t units, hipStream_t st) {
    if (g.tiles == kGemmTilesSxFixed && g.n_vec > kGemmSxMaxRows) {
        // passes of kGemmSxMaxRows vectors, each planned alike: rows stay independent of n_vec
        for (uint32_t t0 = 0; t0 < g.n_vec; t0 += kGemmSxMaxRows) {
            GemmArgs p = g;
            p.x = g.x + (uint64_t)t0 * g.x_stride;
            p.y = g.y + (uint64_t)t0 * g.y_stride;
            p.n_vec = std::min(kGemmSxMaxRows, g.n_vec - t0);
            if (int rc = launch_gemm_sx(type, pair, p, ws, units, st)) return rc;
        }
        return HALO_MI_OK;
    }
    uint32_t kc = 0;
    size_t lds = 0;
    if (!gemm_sx_plan(units, g.cols, g.n_vec, &kc, &lds))
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: the exact small-M kernel takes 1..%u rows of x and cols a multiple "
                                                "of 256 within the workspace", kGemmSxMaxRows);
    const float* x = g.x;
    uint64_t xs = g.x_stride;
    if (g.norm_w) {  // rms_norm first (bitwise cpu::rms_norm), as every variant
        if (int rc = launch_rms_norm(g.x, g.x_stride, g.norm_w, ws->xn, g.cols, g.n_vec, g.cols, g.norm_eps, st)) return rc;
        x = ws->xn;
        xs = g.cols;
    }
    const SxArgs a{g.w0, g.w1, x, xs, ws->partials, g.rows, g.cols, g.n_vec, kc, g.y, g.y_stride};
    const dim3 grid(((units + 1) / 2) * kc);
    const int np = (int)(g.n_vec + 1) / 2;
    switch (np) {
        case 1:
            pair ? launch_sx_np<true, 1>(type, a, grid, lds, st) : launch_sx_np<false, 1>(type, a, grid, lds, st);
            break;
        case 2:
            pair ? launch_sx_np<true, 2>(type, a, grid, lds, st) : launch_sx_np<false, 2>(type, a, grid, lds, st);
            break;
        case 3:
            pair ? launch_sx_np<true, 3>(type, a, grid, lds, st) : launch_sx_np<false, 3>(type, a, grid, lds, st);
            break;
        default:
            pair ? launch_sx_np<true, 4>(type, a, grid, lds, st) : launch_sx_np<false, 4>(type, a, grid, lds, st);
            break;
    }
    if (int rc = hip_status(hipGetLastError(), "gemm_sx launch")) return rc;
    if (kc == 1) return HALO_MI_OK;
    const uint64_t threads = (uint64_t)units * g.n_vec * (pair ? 64 : 128);
    const dim3 rgrid((uint32_t)((threads + 255) / 256));
    if (pair)
        hipLaunchKernelGGL(k_sx_reduce<true>, rgrid, dim3(256), 0, st, ws->partials, g.y, g.y_stride, g.rows, units, g.n_vec, kc);
    else
        hipLaunchKernelGGL(k_sx_reduce<false>, rgrid, dim3(256), 0, st, ws->partials, g.y, g.y_stride, g.rows, units, g.n_vec, kc);
    return hip_status(hipGetLastError(), "gemm_sx reduce launch");
}

}  // namespace halo_mi
