// Device code of the slab GEMV kernels (k_gemv.hip: the plain launches; k_gemv_group.hip: the
// grouped launch over several matrices that share x). Each including file gets its own copy
// (an anonymous namespace), so the two are compiled in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "device.h"
#include "launch.h"
#include "norm_device.h"

namespace halo_mi {
namespace {

using namespace dev;

// ==========================================================================================
// Reference-order GEMV over GGUF rows (bitwise equal to cpu::matmul)
// ==========================================================================================

// Block of 256 threads = 32 groups of 8 lanes; group -> one W row, every x vector.
__global__ __launch_bounds__(256) void k_gemv_gguf_ref(uint32_t type, const uint8_t* __restrict__ w, uint64_t w_stride,
                                                       const float* __restrict__ x, uint64_t x_stride,
                                                       float* __restrict__ y, uint64_t y_stride, uint32_t rows,
                                                       uint32_t cols, uint32_t n_vec) {
#pragma clang fp contract(off)
    const uint32_t j = threadIdx.x & 7u;
    const uint32_t n = blockIdx.x * 32u + (threadIdx.x >> 3);
    const bool live = n < rows;
    const uint8_t* row = w + (uint64_t)(live ? n : 0) * w_stride;
    const uint32_t full = cols - cols % 8u;
    for (uint32_t t = 0; t < n_vec; ++t) {
        const float* xt = x + (uint64_t)t * x_stride;
        float p = 0.0f;
        if (live)
            for (uint32_t i = j; i < full; i += 8) {
                const float prod = xt[i] * gguf_elem(type, row, i);
                p = p + prod;
            }
        // ((p0+p4)+(p1+p5)) + ((p2+p6)+(p3+p7)), then + tail, exactly as the CPU dot.
        const float q = p + __shfl_down(p, 4, 8);   // lanes 0..3: p_j + p_{j+4}
        const float r = q + __shfl_down(q, 1, 8);   // lane 0: left, lane 2: right
        const float s = r + __shfl_down(r, 2, 8);   // lane 0: left + right
        if (j == 0 && live) {
            float tail = 0.0f;
            for (uint32_t i = full; i < cols; ++i) {
                const float prod = xt[i] * gguf_elem(type, row, i);
                tail = tail + prod;
            }
            y[(uint64_t)t * y_stride + n] = s + tail;
        }
    }
}

// ==========================================================================================
// SLAB GEMV: one row per lane; a one-wave workgroup owns a (slab, K chunk) unit
// ==========================================================================================
//
// The grid is slabs x ks units (ks K chunks per slab, chosen so the chip gets many more
// units than CUs). A unit first issues the loads of its first slot group (8 slots = 256
// weights per row: eight contiguous 1 KB wave loads plus the group's scale records), then
// stages its slice of x in LDS while they are in flight, and streams the remaining groups
// with the next group's loads issued before the current group is computed. With ks > 1 the
// per-row partials go to a workspace; the unit that finishes last for a slab (an atomic
// counter per slab) adds the ks partials in chunk order and writes y, so the result does
// not depend on scheduling.



// Q6_K slot record -> 6-bit quants as bytes, like q6_slot_bytes (decode.h), for the GEMV.
__device__ __forceinline__ void q6_slot_bytes_gemv(const uint4& ql, const uint2& qh, uint32_t lo[4], uint32_t hi[4]) {
    const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w};
    const uint32_t H[2] = {qh.x, qh.y};
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const uint32_t a = L[2 * w], b = L[2 * w + 1], h = H[w];
        lo[2 * w] = and_or_opaque(a, 0x0F0F0F0Fu, h & 0x30303030u);
        hi[2 * w] = and_or_opaque(a >> 4, 0x0F0F0F0Fu, (h >> 2) & 0x30303030u);
        lo[2 * w + 1] = and_or_opaque(b, 0x0F0F0F0Fu, (h << 4) & 0x30303030u);
        hi[2 * w + 1] = and_or_opaque(b >> 4, 0x0F0F0F0Fu, (h << 2) & 0x30303030u);
    }
}

template <uint32_t T>
struct SlotGroup;

template <>
struct SlotGroup<kQ4_K> {
    uint4 q[8];
    uint4 hdr;
};
template <>
struct SlotGroup<kQ6_K> {
    uint4 ql[8];
    uint2 qh[8];
    uint4 sc;
    uint32_t d;
};
template <>
struct SlotGroup<kQ5_K> {
    uint4 q[8];
    uint32_t qh[8];
    uint4 hdr;
};
template <>
struct SlotGroup<kIQ4_XS> {
    uint4 q[8];
    uint2 hdr;
};
template <>
struct SlotGroup<kQ4_0> {
    uint4 q[8];
    uint32_t d[8];
};
template <>
struct SlotGroup<kQ8_0> {
    uint4 qa[8], qb[8];
    uint32_t d[8];
};

// The weight records are read once per launch: nontemporal loads, so the stream does not
// displace reusable lines (x, partials) from the caches.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_nt16(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_nt8(const uint8_t* p) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_nt2(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

// SPLIT (Q6_K): the eight ql records, then the eight qh records (two sequential streams), then
// the group's scales, instead of the scales first and each slot's pair in turn. Measured on
// MI355X for the one-group form (5120 x 17408, against the pairs: M = 2 24.9 -> 24.2 us, M = 4
// 28.2 -> 26.2; the scales last: M = 1 19.3 -> 19.05, M = 2 24.1 -> 24.8); the form with several
// groups per wave (the 151936-row head 114.5 -> 115.5) and Q5_K's qh words (14.52 -> 14.83) keep
// the pairs, and Q4_0 / Q8_0 measured slower with their scales first or last.
template <uint32_t T, bool SPLIT = false>
__device__ __forceinline__ void load_group(SlotGroup<T>& G, const uint8_t* __restrict__ slab, const SlabGeom& g,
                                           uint32_t lane, uint32_t grp, uint32_t S) {
    const uint32_t sb = grp * 8;
    // the quants in slot order with the scales first (loads complete in order, so slot j can be
    // used as soon as its own record has arrived), except Q4_K's header after its quants (measured
    // on MI355X, 17408 x 5120 M = 1: 11.95 -> 11.84 us; IQ4_XS's header last: 14.19 -> 14.69)
    if constexpr (T == kQ4_K) {
#pragma unroll
        for (int j = 0; j < 8; ++j) G.q[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
        G.hdr = ld_nt16(slab + g.aux_off + ((uint64_t)grp * 64 + lane) * 16);
    } else if constexpr (T == kQ5_K) {
        G.hdr = ld_nt16(slab + g.sc_off + ((uint64_t)grp * 64 + lane) * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            G.q[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
            G.qh[j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(slab + g.aux_off + ((uint64_t)(sb + j) * 64 + lane) * 4));
        }
    } else if constexpr (T == kIQ4_XS) {
        G.hdr = ld_nt8(slab + g.aux_off + ((uint64_t)grp * 64 + lane) * 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) G.q[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
    } else if constexpr (T == kQ6_K) {
        if constexpr (SPLIT) {
#pragma unroll
            for (int j = 0; j < 8; ++j) G.ql[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
#pragma unroll
            for (int j = 0; j < 8; ++j) G.qh[j] = ld_nt8(slab + g.aux_off + ((uint64_t)(sb + j) * 64 + lane) * 8);
            G.sc = ld_nt16(slab + g.sc_off + ((uint64_t)grp * 64 + lane) * 16);
            G.d = ld_nt2(slab + g.d_off + ((uint64_t)grp * 64 + lane) * 2);
        } else {
            G.d = ld_nt2(slab + g.d_off + ((uint64_t)grp * 64 + lane) * 2);
            G.sc = ld_nt16(slab + g.sc_off + ((uint64_t)grp * 64 + lane) * 16);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                G.ql[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
                G.qh[j] = ld_nt8(slab + g.aux_off + ((uint64_t)(sb + j) * 64 + lane) * 8);
            }
        }
    } else if constexpr (T == kQ4_0) {
        const uint32_t n = min(8u, S - sb);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if ((uint32_t)j < n) {
                G.q[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
                G.d[j] = ld_nt2(slab + g.aux_off + ((uint64_t)(sb + j) * 64 + lane) * 2);
            }
    } else {
        const uint32_t n = min(8u, S - sb);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if ((uint32_t)j < n) {
                G.qa[j] = ld_nt16(slab + g.q_off + (((uint64_t)(sb + j) * 2) * 64 + lane) * 16);
                G.qb[j] = ld_nt16(slab + g.q_off + (((uint64_t)(sb + j) * 2 + 1) * 64 + lane) * 16);
                G.d[j] = ld_nt2(slab + g.aux_off + ((uint64_t)(sb + j) * 64 + lane) * 2);
            }
    }
}

// x through the constant address space: wave-uniform loads become scalar loads, so x is
// read through the scalar cache into SGPRs and fed to the FMAs as scalar operands.
typedef __attribute__((address_space(4))) const float cfloat;
typedef __attribute__((address_space(4))) const float4 cfloat4;

// 4-bit slot record against x (SGPR): lo = sum x[t] q[t] (t < 16), hi = sum x[16 + t] q[16 + t],
// in units of fp8_unit().
__device__ __forceinline__ void dot_nibbles_s(const uint4& q, cfloat* xs, float& lo, float& hi) {
    const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = Q[i] & 0x0F0F0F0Fu, b = (Q[i] >> 4) & 0x0F0F0F0Fu;
        const float2v a01 = __builtin_amdgcn_cvt_pk_f32_fp8(a, false), a23 = __builtin_amdgcn_cvt_pk_f32_fp8(a, true);
        const float2v b01 = __builtin_amdgcn_cvt_pk_f32_fp8(b, false), b23 = __builtin_amdgcn_cvt_pk_f32_fp8(b, true);
        lo = fmaf(xs[4 * i + 0], a01[0], lo);
        lo = fmaf(xs[4 * i + 1], a01[1], lo);
        lo = fmaf(xs[4 * i + 2], a23[0], lo);
        lo = fmaf(xs[4 * i + 3], a23[1], lo);
        hi = fmaf(xs[16 + 4 * i + 0], b01[0], hi);
        hi = fmaf(xs[16 + 4 * i + 1], b01[1], hi);
        hi = fmaf(xs[16 + 4 * i + 2], b23[0], hi);
        hi = fmaf(xs[16 + 4 * i + 3], b23[1], hi);
    }
}

__device__ __forceinline__ void dot_bytes_s(const uint32_t A[4], const uint32_t B[4], cfloat* xs, float& lo, float& hi) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            lo = fmaf(xs[4 * i + k], ubyte(A[i], k), lo);
            hi = fmaf(xs[16 + 4 * i + k], ubyte(B[i], k), hi);
        }
}

// Half-slot sums (16 x values each) of the up-to-4 slot groups starting at group gb, held one
// per lane: lane 16 i + h has half-slot h of group gb + i. Read back with xsum_at (readlane),
// so the main loop never waits on memory for them.
__device__ __forceinline__ float wave_xsums(const float* __restrict__ x, uint32_t gb, uint32_t S, uint32_t lane) {
    const uint32_t e = gb * 256 + lane * 16;  // this lane's 16 elements
    float s = 0.0f;
    if (e < S * 32) {
#pragma unroll
        for (int k = 0; k < 16; k += 4) s += (x[e + k] + x[e + k + 1]) + (x[e + k + 2] + x[e + k + 3]);
    }
    return s;
}
__device__ __forceinline__ float xsum_at(float xsv, uint32_t idx) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xsv), idx));
}

// One loaded group against NV vectors; x of vector v at x + v * x_stride (SGPR loads),
// X[v][h] the group's half-slot sums.
template <uint32_t T, int NV>
__device__ __forceinline__ void compute_group(const SlotGroup<T>& G, uint32_t grp, uint32_t gi, uint32_t S, cfloat* x,
                                              uint64_t x_stride, const float (&xsv)[NV], float inv_unit,
                                              float acc[NV]) {
    const uint32_t sbase = grp * 8, hb = gi * 16;  // this group's half-slot sums: lanes hb .. hb + 15
    if constexpr (T == kQ4_K) {
        // d is scaled by 1 / fp8_unit (a power of two: exact) to undo the fp8 conversion
        const float d = h2f(G.hdr.x & 0xFFFFu) * inv_unit, dmin = h2f(G.hdr.x >> 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, m;
            q4k_sc_m(G.hdr.y, G.hdr.z, G.hdr.w, j, sc, m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float lo = 0.0f, hi = 0.0f;
                dot_nibbles_s(G.q[j], x + v * x_stride + (uint64_t)(sbase + j) * 32, lo, hi);
                acc[v] = fmaf(d1, lo + hi, acc[v]);
                acc[v] = fmaf(-m1, xsum_at(xsv[v], hb + 2 * j) + xsum_at(xsv[v], hb + 2 * j + 1), acc[v]);
            }
        }
    } else if constexpr (T == kQ6_K) {
        const float d = h2f(G.d);
        const uint32_t SC[4] = {G.sc.x, G.sc.y, G.sc.z, G.sc.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float dA = d * sbyte(SC[j >> 1], 2 * (j & 1)), dB = d * sbyte(SC[j >> 1], 2 * (j & 1) + 1);
            uint32_t lo6[4], hi6[4];
            q6_slot_bytes_gemv(G.ql[j], G.qh[j], lo6, hi6);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float lo = 0.0f, hi = 0.0f;
                dot_bytes_s(lo6, hi6, x + v * x_stride + (uint64_t)(sbase + j) * 32, lo, hi);
                acc[v] = fmaf(dA, fmaf(-32.0f, xsum_at(xsv[v], hb + 2 * j), lo), acc[v]);
                acc[v] = fmaf(dB, fmaf(-32.0f, xsum_at(xsv[v], hb + 2 * j + 1), hi), acc[v]);
            }
        }
    } else if constexpr (T == kQ4_0) {
        const uint32_t n = min(8u, S - sbase);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if ((uint32_t)j >= n) break;
            const float d = h2f(G.d[j]);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float lo = 0.0f, hi = 0.0f;
                dot_nibbles_s(G.q[j], x + v * x_stride + (uint64_t)(sbase + j) * 32, lo, hi);
                const float t = fmaf(-8.0f, xsum_at(xsv[v], hb + 2 * j) + xsum_at(xsv[v], hb + 2 * j + 1), (lo + hi) * inv_unit);
                acc[v] = fmaf(d, t, acc[v]);
            }
        }
    } else {  // Q8_0
        const uint32_t n = min(8u, S - sbase);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if ((uint32_t)j >= n) break;
            const float d = h2f(G.d[j]);
            // int8 q -> q + 128 as an unsigned byte; the 128 is taken back with the x sums
            const uint32_t A[4] = {xor_opaque<0x80808080u>(G.qa[j].x), xor_opaque<0x80808080u>(G.qa[j].y),
                                   xor_opaque<0x80808080u>(G.qa[j].z), xor_opaque<0x80808080u>(G.qa[j].w)};
            const uint32_t B[4] = {xor_opaque<0x80808080u>(G.qb[j].x), xor_opaque<0x80808080u>(G.qb[j].y),
                                   xor_opaque<0x80808080u>(G.qb[j].z), xor_opaque<0x80808080u>(G.qb[j].w)};
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float lo = 0.0f, hi = 0.0f;
                dot_bytes_s(A, B, x + v * x_stride + (uint64_t)(sbase + j) * 32, lo, hi);
                acc[v] = fmaf(d, fmaf(-128.0f, xsum_at(xsv[v], hb + 2 * j) + xsum_at(xsv[v], hb + 2 * j + 1), lo + hi), acc[v]);
            }
        }
    }
}

// Split-K: the workgroup's start ticket for its slab, taken when it starts and used only at its
// end, so the device-scope round trip overlaps the weight stream. A slab's counter holds the
// arrivals of the running launch in its low kTicketBits bits and the slab's launch generation
// above them (kept across launches: the reducer moves it on by one and clears the arrivals).
__device__ __forceinline__ uint32_t gemv_ticket(const GemvSlabArgs& a, uint32_t slab, uint32_t nch) {
    uint32_t t = 0;
    if (nch > 1 && threadIdx.x == 0)
        t = __hip_atomic_fetch_add(&a.counters[a.slab0 + slab], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return t;
}

// Cross-lane moves within rows of 16 lanes (DPP): lane ^ 1, lane ^ 2 (quad permutes), the
// mirror inside 8 lanes (pairs the two quads) and inside 16 lanes (pairs the two halves).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the wave, wave-uniform, in a fixed order: DPP inside each row of 16 lanes (pairs,
// quads, halves of 8, halves of 16), then (row 0 + row 1) + (row 2 + row 3).
__device__ __forceinline__ float wave_sum(float s) {
    s += dpp_f<kDppXor1>(s);
    s += dpp_f<kDppXor2>(s);
    s += dpp_f<kDppHalfMirror>(s);
    s += dpp_f<kDppMirror>(s);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 48));
    return (r0 + r1) + (r2 + r3);
}

// Split-K meeting of one slab's pieces (the workgroups, or segments of workgroups, that summed
// parts of its K range) in the workspace words, without cache maintenance and without a round
// trip at the end of most pieces. The piece with the slab's last start ticket is the reducer:
// every other piece of the slab started before it, so they are all running. The others store
// their partials as 64-bit words (fp32 bits and this launch's tag: one atomic access carries the
// value and its mark) and finish. The reducer loads those words, re-reads (bounded, with a pause)
// any not yet ready, adds the pieces in piece order (deterministic), and clears the words and
// the arrivals for the next launch.
// c: this piece of nch, holding acc0; ticket: its start ticket (the calling wave's first lane).
// Pieces [0, n0) are the gate rows of a pair (or all), [n0, nch) the up rows. gs: the slab's
// index among the launch's slabs (a grouped launch covers several matrices); stride: the pieces
// the workspace holds per slab. Returns false for a piece that stored its partial, true for the
// reducer, which then holds the slab's sums in acc0 and acc1. SLAB_NORM: the in-kernel norm's
// published words are per slab (the reducer clears the slab's), not per workgroup.
template <int NV, bool SLAB_NORM = true>
__device__ __forceinline__ bool splitk_meet(const GemvSlabArgs& a, float (&acc0)[NV], float (&acc1)[NV], uint32_t lane,
                                            uint32_t gs, uint32_t c, uint32_t nch, uint32_t n0, uint32_t stride,
                                            uint32_t ticket) {
    uint64_t* P = a.slots + (uint64_t)gs * stride * NV * 64;
    // A word is ready when its high half holds this launch's tag (the slab's generation, never
    // 0): a word left over from an earlier launch (one that arrived after its reducer gave up
    // waiting) is never taken for this launch's.
    const uint32_t tk = __builtin_amdgcn_readfirstlane(ticket);
    const uint32_t gen = tk >> kTicketBits;
    const uint64_t tag = (uint64_t)((gen & kTagMask) | (kTagMask + 1)) << 32;
    if ((tk & kArrivalMask) != nch - 1) {
#pragma unroll
        for (int v = 0; v < NV; ++v)
            __hip_atomic_store(P + ((uint64_t)c * NV + v) * 64 + lane, (uint64_t)__float_as_uint(acc0[v]) | tag,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    float own[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        own[v] = acc0[v];
        acc0[v] = 0.0f;
    }
    // The loads of 8 pieces are issued before any is used (one memory round trip per 8 pieces);
    // past the last piece the address is clamped and the value dropped.
    constexpr uint32_t KB = 8;
    // The other pieces are running, so a word is a few microseconds away at most. A wait that
    // gives up marks the stream's status word (the host reports it as a device error at its next
    // check) and leaves NaN in the output.
    constexpr uint32_t kSpinLimit = 1u << 20;
    const uint32_t spin_limit = a.spin_limit ? a.spin_limit : kSpinLimit;
    const uint64_t want = tag ^ a.tag_flip;  // tag_flip: the host's forced-timeout test only
    for (uint32_t k0 = 0; k0 < nch; k0 += KB) {
        uint64_t q[KB][NV];
#pragma unroll
        for (uint32_t kk = 0; kk < KB; ++kk) {
            const uint64_t* Q = P + (uint64_t)min(k0 + kk, nch - 1) * NV * 64;
#pragma unroll
            for (int v = 0; v < NV; ++v)
                q[kk][v] = __hip_atomic_load(Q + v * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (uint32_t kk = 0; kk < KB; ++kk) {
            const uint32_t k = k0 + kk;
            if (k >= nch) break;
            float val[NV];
            if (k == c) {
#pragma unroll
                for (int v = 0; v < NV; ++v) val[v] = own[v];
            } else {
                // while a word of this piece is not ready, the piece's words not ready are loaded
                // again together (one round trip per retry, not one per word)
                for (uint32_t spin = 0;; ++spin) {
                    bool all = true;
#pragma unroll
                    for (int v = 0; v < NV; ++v) all = all && (q[kk][v] & ~0xFFFFFFFFull) == want;
                    if (all || spin >= spin_limit) break;
                    __builtin_amdgcn_s_sleep(2);
#pragma unroll
                    for (int v = 0; v < NV; ++v)
                        if ((q[kk][v] & ~0xFFFFFFFFull) != want)
                            q[kk][v] = __hip_atomic_load(P + ((uint64_t)k * NV + v) * 64 + lane, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    if ((q[kk][v] & ~0xFFFFFFFFull) == want) {
                        val[v] = __uint_as_float((uint32_t)q[kk][v]);
                    } else {  // gave up: the stream's status word, NaN in y
                        if (a.status)
                            __hip_atomic_fetch_or(a.status, kStatusSplitKTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        val[v] = __builtin_nanf("");
                    }
                }
            }
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (k < n0) acc0[v] += val[v];
                else acc1[v] += val[v];
            }
        }
    }
    for (uint32_t k = 0; k < nch; ++k)
        if (k != c) {
#pragma unroll
            for (int v = 0; v < NV; ++v)
                __hip_atomic_store(P + ((uint64_t)k * NV + v) * 64 + lane, 0ull, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    if (lane == 0) {
        // the slab's published 1 / rms (in-kernel norm): every piece has read it
        if (SLAB_NORM && a.norm_words) __hip_atomic_store(a.norm_words + gs, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&a.counters[gs], (gen + 1) << kTicketBits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

// End of a slab: the LM head's argmax parts and y (SiLU(gate) * up for the pair), one row per
// lane of the calling wave (all 64 lanes).
template <int NV, bool PAIR>
__device__ __forceinline__ void gemv_store(const GemvSlabArgs& a, const float (&acc0)[NV], const float (&acc1)[NV],
                                           uint32_t slab, uint32_t lane) {
    const uint32_t row = slab * kSlabRows + lane;
    if constexpr (!PAIR) {
        // LM head: the slab's argmax per vector, over exactly the values written to y (rows past
        // the matrix take no part)
        if (a.parts) {
            const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
            const bool live = row < a.rows;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if ((uint32_t)v >= a.n_vec) break;
                const bool nan = live && acc0[v] != acc0[v];
                const bool rank = live && !nan && (a.valid_rows == 0 || row < a.valid_rows);
                float bv;
                uint32_t bi, any_nan;
                wave_argmax(acc0[v], row, rank, nan, bv, bi, any_nan);
                if (lane == 0) a.parts[(uint64_t)v * slabs + slab] = ArgPart{bv, bi, any_nan, 0u};
            }
        }
    }
    if (row >= a.rows || !a.y) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        if ((uint32_t)v >= a.n_vec) break;
        a.y[(uint64_t)v * a.y_stride + row] = PAIR ? silu_f(acc0[v]) * acc1[v] : acc0[v];
    }
}

// End of a chunked slab-GEMV workgroup: the waves' partial sums meet in LDS in wave order, then
// (split K) the workgroups of the slab meet in the workspace, and the reducer writes the slab.
// acc0 holds this wave's sums in fp32, rows = lanes.
template <int NV, bool PAIR>
__device__ __forceinline__ void gemv_finish(const GemvSlabArgs& a, float (&acc0)[NV], float* red, uint32_t wave,
                                            uint32_t nw, uint32_t lane, uint32_t slab, uint32_t c, uint32_t nch,
                                            uint32_t ticket) {
    // waves -> wave 0, in wave order
    if (nw > 1) {
#pragma unroll
        for (int v = 0; v < NV; ++v) red[(wave * NV + v) * 64 + lane] = acc0[v];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            float s = red[v * 64 + lane];
            for (uint32_t w = 1; w < nw; ++w) s += red[(w * NV + v) * 64 + lane];
            acc0[v] = s;
        }
    }
    float acc1[NV];  // the up sums (PAIR)
#pragma unroll
    for (int v = 0; v < NV; ++v) acc1[v] = 0.0f;
    if (nch > 1 && !splitk_meet<NV>(a, acc0, acc1, lane, a.slab0 + slab, c, nch, a.ks, nch, ticket)) return;
    gemv_store<NV, PAIR>(a, acc0, acc1, slab, lane);
}

// grid.x = slabs * ks * MATS; block = 64 * nw (nw waves). Dynamic LDS: the waves' partials
// [nw][NV][64]. With PAIR (MATS = 2) a workgroup streams one matrix only (chunks [0, ks) the
// gate rows, [ks, 2 ks) the up rows of the same slab) and the gate and up sums meet in the
// split-K fix-up, which applies SiLU: the pair costs no registers over a single GEMV.
template <uint32_t T, int NV, bool PAIR>
__global__ __launch_bounds__(1024, 4) void k_gemv_slab(GemvSlabArgs a) {
    extern __shared__ float smem[];
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint32_t S = a.cols / kSlot, ngrp = (S + 7) / 8;
    const uint32_t nch = a.ks * MATS;  // chunks per slab
    const uint32_t slab = blockIdx.x / nch, c = blockIdx.x % nch;
    const uint32_t mat = c / a.ks, cc = c % a.ks;
    // this workgroup's groups [g0, g1), then this wave's share [w0, w1)
    const uint32_t base = ngrp / a.ks, extra = ngrp % a.ks;
    const uint32_t g0 = cc * base + min(cc, extra), g1 = g0 + base + (cc < extra ? 1u : 0u);
    const uint32_t wb = (g1 - g0) / nw, we = (g1 - g0) % nw;
    const uint32_t w0 = g0 + wave * wb + min(wave, we), w1 = w0 + wb + (wave < we ? 1u : 0u);
    const SlabGeom geo = slab_geom(T, a.cols);
    const uint8_t* slab0 = (mat ? a.w1 : a.w0) + (uint64_t)slab * geo.slab_bytes;
    cfloat* xc = reinterpret_cast<cfloat*>(reinterpret_cast<uintptr_t>(a.x));
    float* red = smem;

    // 1 / fp8_unit, built from the exponent bits (exact for a power of two)
    const float inv_unit = __uint_as_float(0x7F000000u - __float_as_uint(fp8_unit()));
    float acc0[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc0[v] = 0.0f;
    SlotGroup<T> cur0;
    if (w0 < w1) load_group<T>(cur0, slab0, geo, lane, w0, S);
    const uint32_t ticket = gemv_ticket(a, slab, nch);
    float xsv[NV];  // half-slot sums of this wave's groups (at most 4), one per lane
#pragma unroll
    for (int v = 0; v < NV; ++v) xsv[v] = wave_xsums(a.x + (uint64_t)v * a.x_stride, w0, S, lane);
    for (uint32_t grp = w0; grp < w1; ++grp) {
        if constexpr (T == kQ8_0) {
            // a Q8_0 group is 72 registers: one buffer, the next group loaded after this one
            compute_group<T, NV>(cur0, grp, grp - w0, S, xc, a.x_stride, xsv, inv_unit, acc0);
            if (grp + 1 < w1) load_group<T>(cur0, slab0, geo, lane, grp + 1, S);
        } else {
            // Ping-pong between two register buffers: the next group is always in flight. The
            // prefetch is unconditional (past the last group it reloads the last one, an L2
            // hit) so the compiler can wait for exactly the older loads (vmcnt counts in order).
            SlotGroup<T> nxt;
            load_group<T>(nxt, slab0, geo, lane, min(grp + 1, w1 - 1), S);
            compute_group<T, NV>(cur0, grp, grp - w0, S, xc, a.x_stride, xsv, inv_unit, acc0);
            if (grp + 1 >= w1) break;
            ++grp;
            load_group<T>(cur0, slab0, geo, lane, min(grp + 1, w1 - 1), S);
            compute_group<T, NV>(nxt, grp, grp - w0, S, xc, a.x_stride, xsv, inv_unit, acc0);
        }
    }
    gemv_finish<NV, PAIR>(a, acc0, red, wave, nw, lane, slab, c, nch, ticket);
}

// ------------------------------------------------------------------------------------------
// MFMA GEMV: k_gemv_mx<T, NV, PAIR>
//
// Same work split and SLAB stream as k_gemv_slab (one row per lane, a wave streams slot groups
// of its 64 rows), but the multiply-adds run on v_mfma_f32_4x4x4_16b_bf16 instead of the VALU:
//   B (per lane, its own row): four weights of one "k-step" as raw bf16 bit patterns. A code c
//     in 0..255 held in the low bits of a bf16 is exactly c * 2^-133 (subnormal up to 127,
//     then the first normal binade, which continues the same scale), so the quants need only
//     masks: 4-bit records as (q & 0x000F000F), (q & 0x00F000F0) = 16 * the high nibble,
//     6-bit and biased 8-bit codes as byte pairs.
//   A (broadcast from one 4-lane block to all 16 with cbsz = 4): rows = x pieces. Per slot
//     group and vector, x is scaled by 2^S (S from the group's largest |x|, so the products
//     stay normal) and split exactly into three bf16 pieces b1 + b2 + b3 = x * 2^S. Row
//     3 v + p holds piece p of vector v; the high-nibble k-steps carry x / 16.
//   D (per lane, its own row): D[3 v + p] = sum_k piece_p(x_k) * q_k * 2^-133, exact products
//     accumulated in fp32. The three pieces added give x . q for the slot in units of
//     2^(S - 133); the slot scales (d * sc, dmin * m, offsets) are applied per row as in the
//     VALU kernel, and each group's sum is brought back to fp32 units with ldexp.
// The A operands of a group (8 slots x 8 k-steps x M row blocks of 4 x 4 bf16) are built by
// the wave itself in a private LDS table and read back as 4 M register pairs; one pair feeds
// 16 MFMAs through the broadcast block id.
// ------------------------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A-operand row blocks per k-step for NV vectors (3 pieces each, 4 rows per block)
template <int NV>
constexpr int mx_blocks() { return (3 * NV + 3) / 4; }
// LDS bytes of one wave's A table: 8 slots x 8 k-steps x M blocks x 32 B
template <int NV>
constexpr uint32_t mx_table_bytes() { return 64u * mx_blocks<NV>() * 32u; }

__device__ __forceinline__ f32x4 mfma4_bc(s16x4 a, s16x4 b, f32x4 c, uint32_t abid) {
    switch (abid & 15u) {
#define HALO_MI_BC(k) \
    case k: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 4, k, 0);
        HALO_MI_BC(0) HALO_MI_BC(1) HALO_MI_BC(2) HALO_MI_BC(3) HALO_MI_BC(4) HALO_MI_BC(5) HALO_MI_BC(6)
        HALO_MI_BC(7) HALO_MI_BC(8) HALO_MI_BC(9) HALO_MI_BC(10) HALO_MI_BC(11) HALO_MI_BC(12)
        HALO_MI_BC(13) HALO_MI_BC(14) HALO_MI_BC(15)
#undef HALO_MI_BC
    }
    return c;
}

__device__ __forceinline__ s16x4 as_b(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(s16x4, u32x2_t{lo, hi});
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
}
// (a, b) -> three bf16 pairs whose sums are exactly a and b: each residual is exact in fp32
// and has at most 16, then 8 significant bits, so the third piece is the residual itself.
__device__ __forceinline__ void split3(float a, float b, uint32_t (&p)[3]) {
    p[0] = pack_bf16(a, b);
    const float ra = a - __uint_as_float(p[0] << 16), rb = b - __uint_as_float(p[0] & 0xFFFF0000u);
    p[1] = pack_bf16(ra, rb);
    p[2] = pack_bf16(ra - __uint_as_float(p[1] << 16), rb - __uint_as_float(p[1] & 0xFFFF0000u));
}

// Maximum over the wave, wave-uniform (DPP inside rows, then the four row results).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u<kDppXor1>(v));
    v = max(v, dpp_u<kDppXor2>(v));
    v = max(v, dpp_u<kDppHalfMirror>(v));
    v = max(v, dpp_u<kDppMirror>(v));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}

// x of one slot group, lane = 8 s + r: x[slot 8 grp + s][4 r .. 4 r + 3] (zero past the end).
// Branch-free (the address is clamped, the value selected after): a load under a branch would
// make the compiler wait for it before the weight loads that follow are issued.
template <int NV>
__device__ __forceinline__ void mx_load_x(float (&xr)[NV][4], const float* __restrict__ x, uint64_t x_stride, uint32_t grp,
                                          uint32_t S, uint32_t lane) {
    const uint32_t slot = grp * 8 + (lane >> 3);
    const bool in = slot < S;
    const uint64_t e = (uint64_t)min(slot, S - 1) * 32 + 4 * (lane & 7);
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float t = x[(uint64_t)v * x_stride + e + i];
            xr[v][i] = in ? t : 0.0f;
        }
}

// Builds this wave's A table for one group from xr, reads it back as register pairs, and
// returns per vector the exponent that brings the group's sums to fp32 units (es) and the x
// sums in MFMA units (xs: lane 8 s holds slot s's sum, lane 8 s + 4 the high half's sum for
// Q6_K, whose low-half sum is then in lane 8 s).
// The k-step r of a slot (k-steps 0..3: slot elements 0..15, 4..7: 16..31) covers elements
// 4 r .. 4 r + 3 in the order (0, 2, 1, 3), the order the masks below produce them.
template <uint32_t T, int NV>
__device__ __forceinline__ void mx_build(const float (&xr)[NV][4], uint8_t* tab, uint32_t lane,
                                         s16x4 (&A)[4 * mx_blocks<NV>()], int (&es)[NV], float (&xs)[NV]) {
    constexpr int M = mx_blocks<NV>();
    constexpr int kHiShift = (T == kQ4_K || T == kQ4_0) ? 4 : 0;  // high nibbles arrive as 16 q
    const uint32_t s = lane >> 3, r = lane & 7;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        uint32_t mb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) mb = max(mb, __float_as_uint(xr[v][i]) & 0x7FFFFFFFu);
        mb = wave_max_u32(mb);
        const int e = min(max((int)(mb >> 23) - 127, -100), 127);
        const int sx = 100 - e;  // the largest |x| * 2^sx is about 2^100
        es[v] = 33 + e;          // 133 - sx
        const int sh = sx - (r >= 4 ? kHiShift : 0);
        uint32_t p01[3], p23[3];
        split3(ldexpf(xr[v][0], sh), ldexpf(xr[v][2], sh), p01);
        split3(ldexpf(xr[v][1], sh), ldexpf(xr[v][3], sh), p23);
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            const int rho = 3 * v + p, m = rho >> 2, row = rho & 3;
            const uint32_t lam = (s * 8 + r) * M + m;
            *reinterpret_cast<uint2*>(tab + (lam >> 4) * 512 + ((lam & 15) * 4 + row) * 8) = make_uint2(p01[p], p23[p]);
        }
        float h = (xr[v][0] + xr[v][1]) + (xr[v][2] + xr[v][3]);
        h += dpp_f<kDppXor1>(h);
        h += dpp_f<kDppXor2>(h);
        if constexpr (T != kQ6_K) h += dpp_f<kDppHalfMirror>(h);
        xs[v] = ldexpf(h, sx - 133);
    }
#pragma unroll
    for (int rho = 3 * NV; rho < 4 * M; ++rho) {  // unused A rows are zero
        const int m = rho >> 2, row = rho & 3;
        const uint32_t lam = (s * 8 + r) * M + m;
        *reinterpret_cast<uint2*>(tab + (lam >> 4) * 512 + ((lam & 15) * 4 + row) * 8) = make_uint2(0u, 0u);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < 4 * M; ++q) A[q] = *reinterpret_cast<const s16x4*>(tab + q * 512 + lane * 8);
}

// Sum of the three pieces of vector v from the D blocks. The last vector also adds the unused
// rows (their A rows are zero, so they hold exactly 0 and the sum is unchanged): every row an
// MFMA chain writes is then read after the chain. Otherwise the compiler may give a dead row's
// register to another value a few instructions after the chain's last MFMA issues, and on
// gfx950 a dependent MFMA (C from the previous one) can write back after that value is written
// (seen as wrong sums, different from run to run).
template <int NV>
__device__ __forceinline__ float mx_dot(const f32x4 (&D)[mx_blocks<NV>()], int v) {
    const int r0 = 3 * v, r1 = 3 * v + 1, r2 = 3 * v + 2;
    const float s = (D[r0 >> 2][r0 & 3] + D[r1 >> 2][r1 & 3]) + D[r2 >> 2][r2 & 3];
    if (v != NV - 1) return s;
    float z = 0.0f;
#pragma unroll
    for (int r = 3 * NV; r < 4 * mx_blocks<NV>(); ++r) z += D[r >> 2][r & 3];
    return s + z;
}

// The MFMAs of k-step r of slot j with B = b, into D (all row blocks)
template <int NV>
__device__ __forceinline__ void mx_kstep(const s16x4 (&A)[4 * mx_blocks<NV>()], s16x4 b, int j, int r,
                                         f32x4 (&D)[mx_blocks<NV>()]) {
    constexpr int M = mx_blocks<NV>();
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int lam = (j * 8 + r) * M + m;
        D[m] = mfma4_bc(A[lam >> 4], b, D[m], (uint32_t)(lam & 15));
    }
}

// One loaded group against the A table; acc in MFMA units of this group.
template <uint32_t T, int NV>
__device__ __forceinline__ void mx_group(const SlotGroup<T>& G, const s16x4 (&A)[4 * mx_blocks<NV>()],
                                         const float (&xs)[NV], uint32_t n, float (&acc)[NV]) {
    constexpr int M = mx_blocks<NV>();
    // Q4_K: sum_j d sc_j dot_j - dmin m_j xs_j = d sum_j sc_j dot_j - dmin sum_j m_j xs_j, the
    // block's d and dmin applied once per group; Q6_K likewise with d.
    float sa[NV], sb[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) sa[v] = sb[v] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if constexpr (T == kQ4_0 || T == kQ8_0)
            if ((uint32_t)j >= n) break;
        f32x4 D[M], Dh[M];
#pragma unroll
        for (int m = 0; m < M; ++m) D[m] = Dh[m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (T == kQ4_K || T == kQ4_0) {
            const uint32_t Q[4] = {G.q[j].x, G.q[j].y, G.q[j].z, G.q[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = Q[i], q8 = q >> 8;
                mx_kstep<NV>(A, as_b(q & 0x000F000Fu, q8 & 0x000F000Fu), j, i, D);
                mx_kstep<NV>(A, as_b(q & 0x00F000F0u, q8 & 0x00F000F0u), j, 4 + i, D);
            }
        } else if constexpr (T == kQ8_0) {
            const uint32_t Qa[4] = {G.qa[j].x, G.qa[j].y, G.qa[j].z, G.qa[j].w};
            const uint32_t Qb[4] = {G.qb[j].x, G.qb[j].y, G.qb[j].z, G.qb[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ua = Qa[i] ^ 0x80808080u, ub = Qb[i] ^ 0x80808080u;  // q + 128
                mx_kstep<NV>(A, as_b(ua & 0x00FF00FFu, __builtin_amdgcn_perm(0u, ua, 0x0C030C01u)), j, i, D);
                mx_kstep<NV>(A, as_b(ub & 0x00FF00FFu, __builtin_amdgcn_perm(0u, ub, 0x0C030C01u)), j, 4 + i, D);
            }
        } else if constexpr (T == kQ5_K || T == kIQ4_XS) {
            // byte codes: Q5_K's 5-bit quants (fifth bit from the qh word), IQ4_XS's table
            // values + 128
            const uint32_t Q[4] = {G.q[j].x, G.q[j].y, G.q[j].z, G.q[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t lo, hi;
                if constexpr (T == kQ5_K) {
                    lo = and_or_opaque(Q[i], 0x0F0F0F0Fu, (G.qh[j] << (4 - i)) & 0x10101010u);
                    hi = and_or_opaque(Q[i] >> 4, 0x0F0F0F0Fu, (G.qh[j] >> i) & 0x10101010u);
                } else {
                    lo = iq4_lookup4(Q[i]);
                    hi = iq4_lookup4(Q[i] >> 4);
                }
                mx_kstep<NV>(A, as_b(lo & 0x00FF00FFu, __builtin_amdgcn_perm(0u, lo, 0x0C030C01u)), j, i, D);
                mx_kstep<NV>(A, as_b(hi & 0x00FF00FFu, __builtin_amdgcn_perm(0u, hi, 0x0C030C01u)), j, 4 + i, D);
            }
        } else {  // Q6_K: the two halves have their own scales
            uint32_t lo6[4], hi6[4];
            q6_slot_bytes_gemv(G.ql[j], G.qh[j], lo6, hi6);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mx_kstep<NV>(A, as_b(lo6[i] & 0x00FF00FFu, __builtin_amdgcn_perm(0u, lo6[i], 0x0C030C01u)), j, i, D);
                mx_kstep<NV>(A, as_b(hi6[i] & 0x00FF00FFu, __builtin_amdgcn_perm(0u, hi6[i], 0x0C030C01u)), j, 4 + i, Dh);
            }
        }
        if constexpr (T == kQ4_K || T == kQ5_K) {
            uint32_t sc, m;
            q4k_sc_m(G.hdr.y, G.hdr.z, G.hdr.w, (uint32_t)j, sc, m);
            const float fsc = (float)sc, fm = (float)m;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                sa[v] = fmaf(fsc, mx_dot<NV>(D, v), sa[v]);
                sb[v] = fmaf(fm, xsum_at(xs[v], 8 * j), sb[v]);
            }
        } else if constexpr (T == kIQ4_XS) {
            // dl_j = d (ls_j - 32); the codes carry + 128, taken out with the slot's x sum
            const float fl = (float)iq4xs_ls(G.hdr.x >> 16, G.hdr.y, (uint32_t)j);
#pragma unroll
            for (int v = 0; v < NV; ++v) sa[v] = fmaf(fl, fmaf(-128.0f, xsum_at(xs[v], 8 * j), mx_dot<NV>(D, v)), sa[v]);
        } else if constexpr (T == kQ4_0 || T == kQ8_0) {
            const float d = h2f(G.d[j]);
            constexpr float off = T == kQ4_0 ? -8.0f : -128.0f;
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[v] = fmaf(d, fmaf(off, xsum_at(xs[v], 8 * j), mx_dot<NV>(D, v)), acc[v]);
        } else {
            const uint32_t SC[4] = {G.sc.x, G.sc.y, G.sc.z, G.sc.w};
            const float sA = sbyte(SC[j >> 1], 2 * (j & 1)), sB = sbyte(SC[j >> 1], 2 * (j & 1) + 1);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                sa[v] = fmaf(sA, fmaf(-32.0f, xsum_at(xs[v], 8 * j), mx_dot<NV>(D, v)), sa[v]);
                sa[v] = fmaf(sB, fmaf(-32.0f, xsum_at(xs[v], 8 * j + 4), mx_dot<NV>(Dh, v)), sa[v]);
            }
        }
    }
    if constexpr (T == kQ4_K || T == kQ5_K) {
        const float d = h2f(G.hdr.x & 0xFFFFu), dmin = h2f(G.hdr.x >> 16);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = fmaf(d, sa[v], -(dmin * sb[v]));
    } else if constexpr (T == kIQ4_XS) {
        const float d = h2f(G.hdr.x & 0xFFFFu);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = d * sa[v];
    } else if constexpr (T == kQ6_K) {
        const float d = h2f(G.d);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = d * sa[v];
    }
}

// ---- the fused RMS norm (NORM: one vector, GemvArgs::norm_w) ---------------------------------
// One dispatch, bitwise RMS_NORM then the unfused GEMV: every workgroup computes 1 / rms of the raw
// x row itself in cpu::rms_norm's order (norm_device.h: the same chains, combine and finish as the
// RMS_NORM kernel), then each wave normalizes its own slot group of x in registers, (x * inv) *
// norm_w rounded as the CPU rounds it, before the three-piece split: the values RMS_NORM writes.
// The row's x is loaded and its squares staged in LDS before the weight loads are issued (so its
// registers are free again), and the chains run while the weights are on their way, in wave 0 at
// raised wave priority: the chain is 640 dependent additions at 5120 columns, and at the default
// priority it shares its SIMD's issue slots with the other workgroups' waves.
constexpr uint32_t kNormPerThread = 16;  // x loads per thread: the host takes this form when the
                                         // row's first cols - cols % 8 floats need no more
constexpr uint32_t kNormMaxCols = 8192;  // the chain rows fit 33 KB of LDS

__device__ __forceinline__ void lds_sync() { __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The row's x into the chain rows as squares (sq: norm_lds_floats(full) floats of LDS): element
// tid + i nt of the first `full` (> 0) floats, addresses clamped, every load issued before the
// first square is written.
__device__ __forceinline__ void norm_x_squares(const float* __restrict__ x, uint32_t cols, float* sq, uint32_t tid,
                                               uint32_t nt) {
#pragma clang fp contract(off)
    const uint32_t full = cols - cols % 8u, stride = norm_chain_stride(full);
    float v[kNormPerThread];
#pragma unroll
    for (uint32_t i = 0; i < kNormPerThread; ++i) v[i] = x[min(tid + i * nt, full - 1)];
#pragma unroll
    for (uint32_t i = 0; i < kNormPerThread; ++i) {
        const uint32_t e = tid + i * nt;
        if (e < full) sq[(e % 8) * stride + e / 8] = v[i] * v[i];
    }
}

// After norm_x_squares: the chains in lanes 0..7 of wave 0 (wave priority raised for them), the
// combine and the tail: 1 / sqrt(mean + eps) for the whole workgroup.
constexpr int kNormChainBatch = 4;  // 16-byte LDS reads per batch of the chains (16 VGPRs)
constexpr uint32_t kNormPublishPerLane = 16;  // words per lane of the publishing wave (1024 at most)
__device__ __forceinline__ float norm_x_chains(const float* __restrict__ x, uint32_t cols, float eps, float* sq,
                                               uint32_t wave, uint32_t lane) {
    const uint32_t full = cols - cols % 8u, stride = norm_chain_stride(full);
    lds_sync();
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        float p = 0.0f;
        if (lane < 8) p = norm_chain<kNormChainBatch>(sq + lane * stride, full / 8, p);
        const float inv = norm_finish(p, x, full, cols, eps, lane);
        if (lane == 0) sq[8 * stride] = inv;
        __builtin_amdgcn_s_setprio(0);
    }
    lds_sync();
    return sq[8 * stride];
}

// The published 1 / rms for this workgroup's slab (a.norm_words): thread 0, which holds the slab's
// ticket (the generation), waits for the word with this launch's tag and hands it to the
// workgroup through LDS. A wait that gives up sets the stream's status word and yields NaN.
__device__ __forceinline__ float norm_x_wait(const GemvSlabArgs& a, uint32_t slab, uint32_t ticket, float* slot) {
    if (threadIdx.x == 0) {
        const uint32_t gen = ticket >> kTicketBits;
        const uint64_t want = ((uint64_t)((gen & kTagMask) | (kTagMask + 1)) << 32) ^ a.tag_flip;
        const uint64_t* word = a.norm_words + a.slab0 + slab;
        const uint32_t spin_limit = a.spin_limit ? a.spin_limit : (1u << 20);
        uint64_t v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (uint32_t spin = 0; (v & ~0xFFFFFFFFull) != want && spin < spin_limit; ++spin) {
            __builtin_amdgcn_s_sleep(2);
            v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        float inv = __uint_as_float((uint32_t)v);
        if ((v & ~0xFFFFFFFFull) != want) {
            if (a.status) __hip_atomic_fetch_or(a.status, kStatusSplitKTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            inv = __builtin_nanf("");
        }
        *slot = inv;
    }
    lds_sync();
    return *slot;
}

// The in-kernel norm's publishing workgroup, before it issues any weight load: a barrier behind
// the weight loads would wait for every wave's issue, which a launch's saturated memory queue holds
// back for microseconds. x's loads, then wave 0's loads of the tags' generations (counter_of(i) for
// word i < n_pub, i = lane + 64 j: all issued, the index clamped, so they are in flight
// together), the squares into LDS and a barrier; then wave 0 runs the chains, leaves 1 / rms in
// sq[8 stride] and publishes word_of(i) for every i while the other waves go on to their weight
// loads. They read 1 / rms after one more barrier (norm_leader_inv). n_pub <= 64 P.
template <uint32_t P, typename CounterOf, typename WordOf>
__device__ __forceinline__ void norm_leader_publish(const GemvSlabArgs& a, float* sq, uint32_t wave, uint32_t lane,
                                                    uint32_t n_pub, CounterOf counter_of, WordOf word_of) {
    const uint32_t full = a.cols - a.cols % 8u, stride = norm_chain_stride(full);
    float xv[kNormPerThread];
#pragma unroll
    for (uint32_t i = 0; i < kNormPerThread; ++i) xv[i] = a.x[min(threadIdx.x + i * blockDim.x, full - 1)];
    uint32_t gens[P];
    if (wave == 0) {
#pragma unroll
        for (uint32_t i = 0; i < P; ++i)
            gens[i] = __hip_atomic_load(&a.counters[counter_of(min(lane + 64 * i, n_pub - 1))], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    }
    {
#pragma clang fp contract(off)
#pragma unroll
        for (uint32_t i = 0; i < kNormPerThread; ++i) {
            const uint32_t e = threadIdx.x + i * blockDim.x;
            if (e < full) sq[(e % 8) * stride + e / 8] = xv[i] * xv[i];
        }
    }
    lds_sync();
    if (wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        float p = 0.0f;
        if (lane < 8) p = norm_chain_ahead<kNormChainBatch>(sq + lane * stride, full / 8, p);
        const float inv = __shfl(norm_finish(p, a.x, full, a.cols, a.norm_eps, lane), 0);
        if (lane == 0) sq[8 * stride] = inv;
#pragma unroll
        for (uint32_t i = 0; i < P; ++i) {
            const uint32_t w = lane + 64 * i;
            if (w < n_pub)
                __hip_atomic_store(word_of(w),
                                   (uint64_t)__float_as_uint(inv) |
                                       ((uint64_t)(((gens[i] >> kTicketBits) & kTagMask) | (kTagMask + 1)) << 32),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_setprio(0);
    }
}

// The publishing workgroup's waves: 1 / rms after norm_leader_publish (one barrier)
__device__ __forceinline__ float norm_leader_inv(uint32_t cols, const float* sq) {
    lds_sync();
    return sq[8 * norm_chain_stride(cols - cols % 8u)];
}

// LDS bytes of the chain rows and the result word for a row of cols floats
__host__ __device__ constexpr size_t norm_lds_bytes(uint32_t cols) { return (size_t)norm_lds_floats(cols - cols % 8u) * sizeof(float); }

// norm_w at this lane's x elements of group grp (lane = 8 s + r: slot 8 grp + s, elements
// 4 r .. 4 r + 3), the address clamped as mx_load_x's.
__device__ __forceinline__ void mx_load_nw(float (&wr)[4], const float* __restrict__ nw, uint32_t grp, uint32_t S, uint32_t lane) {
    const uint32_t slot = grp * 8 + (lane >> 3);
    const uint64_t e = (uint64_t)min(slot, S - 1) * 32 + 4 * (lane & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[i] = nw[e + i];
}

// xr (one vector, raw x of group grp) -> (x * inv) * norm_w, as cpu::rms_norm rounds it; zero
// past the row's end, as mx_load_x leaves it.
__device__ __forceinline__ void mx_norm_x(float (&xr)[1][4], const float (&wr)[4], float inv, uint32_t grp, uint32_t S,
                                          uint32_t lane) {
#pragma clang fp contract(off)
    const bool in = grp * 8 + (lane >> 3) < S;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float t = xr[0][i] * inv;
        const float n = t * wr[i];
        xr[0][i] = in ? n : 0.0f;
    }
}

// Dynamic LDS bytes of a k_gemv_mx workgroup of nw waves: the waves' partials and A tables.
template <int NV>
__host__ __device__ constexpr size_t mx_lds_bytes(uint32_t nw) {
    return (size_t)nw * (NV * 64 * sizeof(float) + mx_table_bytes<NV>());
}

// Dynamic LDS bytes of a k_gemv_mx_even workgroup: nu unit entries and nw waves' A tables.
template <int NV>
__host__ __device__ constexpr size_t even_lds_bytes(uint32_t nu, uint32_t nw) {
    return (size_t)nu * NV * 64 * sizeof(float) + (size_t)nw * mx_table_bytes<NV>();
}

// Workgroup size bound: single-vector kernels fit 128 VGPRs (16 waves per workgroup), except
// the Q8_0, Q6_K and Q5_K loops (two register groups); so do the one-group loops of the other
// formats at up to 4 vectors; the rest run at most 8 waves.
template <uint32_t T, int NV, bool ONE>
constexpr uint32_t mx_max_threads() {
    constexpr bool heavy = T == kQ8_0 || T == kQ6_K || T == kQ5_K;
    return ((ONE && !heavy) || (NV == 1 && (ONE || !heavy))) ? 1024u : 512u;
}

// grid, split and LDS as k_gemv_slab, plus one A table per wave after the partials. ONE: every
// wave has at most one slot group (no second register buffer, so more waves fit per SIMD).
// The body of workgroup `bid` of a k_gemv_mx launch over the matrix of `a` (also one segment of a
// grouped launch, k_gemv_mx_group).
template <uint32_t T, int NV, bool PAIR, bool ONE, bool NORM = false>
__device__ __forceinline__ void gemv_mx_body(const GemvSlabArgs& a, uint32_t bid) {
    static_assert(!NORM || NV == 1, "the in-kernel norm is the one-vector form");
    extern __shared__ float smem[];
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    constexpr int M = mx_blocks<NV>();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint32_t S = a.cols / kSlot, ngrp = (S + 7) / 8;
    const uint32_t nch = a.ks * MATS;
    float* sq = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(smem) + mx_lds_bytes<NV>(nw));
    // NORM with published words: only the first workgroup runs the chains, before its weight loads
    const bool leader = !NORM || a.norm_words == nullptr || bid == 0;
    if constexpr (NORM) {
        if (a.norm_words && bid == 0)
            norm_leader_publish<kNormPublishPerLane>(
                a, sq, wave, lane, a.norm_slabs, [&](uint32_t s) { return a.slab0 + s; },
                [&](uint32_t s) { return a.norm_words + a.slab0 + s; });
        else if (!a.norm_words)  // every workgroup runs the chains: the squares now, the chains after its loads
            norm_x_squares(a.x, a.cols, sq, threadIdx.x, blockDim.x);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t slab = bid / nch, c = bid % nch;
    const uint32_t mat = c / a.ks, cc = c % a.ks;
    const uint32_t base = ngrp / a.ks, extra = ngrp % a.ks;
    const uint32_t g0 = cc * base + min(cc, extra), g1 = g0 + base + (cc < extra ? 1u : 0u);
    const uint32_t wb = (g1 - g0) / nw, we = (g1 - g0) % nw;
    const uint32_t w0 = g0 + wave * wb + min(wave, we), w1 = w0 + wb + (wave < we ? 1u : 0u);
    const SlabGeom geo = slab_geom(T, a.cols);
    const uint8_t* slab0 = (mat ? a.w1 : a.w0) + (uint64_t)slab * geo.slab_bytes;
    float* red = smem;
    uint8_t* tab = reinterpret_cast<uint8_t*>(smem + nw * NV * 64) + wave * mx_table_bytes<NV>();

    float acc0[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc0[v] = 0.0f;
    float xr[NV][4];
    uint32_t ticket = 0;
    float wr[4];  // NORM: norm_w at this lane's x elements
    // NORM: 1 / rms for the workgroup: the published word, or what the publishing workgroup's wave
    // 0 computed, or (no words) the chains here, after this workgroup's weight loads
    auto norm_inv = [&]() {
        if (!leader) return norm_x_wait(a, bid / (a.ks * (PAIR ? 2u : 1u)), ticket, sq + 8 * norm_chain_stride(a.cols - a.cols % 8u));
        if (a.norm_words) return norm_leader_inv(a.cols, sq);
        return norm_x_chains(a.x, a.cols, a.norm_eps, sq, wave, lane);
    };
    if constexpr (ONE) {
        if (w0 < w1) {
            SlotGroup<T> G;
            // x first: the A table is built while the weights are on their way (loads are waited
            // for in issue order)
            mx_load_x<NV>(xr, a.x, a.x_stride, w0, S, lane);
            if constexpr (NORM) mx_load_nw(wr, a.norm_w, w0, S, lane);
            load_group<T, true>(G, slab0, geo, lane, w0, S);
            ticket = gemv_ticket(a, slab, nch);
            if constexpr (NORM) mx_norm_x(xr, wr, norm_inv(), w0, S, lane);
            s16x4 A[4 * M];
            int es[NV];
            float xs[NV];
            mx_build<T, NV>(xr, tab, lane, A, es, xs);
            mx_group<T, NV>(G, A, xs, min(8u, S - w0 * 8), acc0);
#pragma unroll
            for (int v = 0; v < NV; ++v) acc0[v] = ldexpf(acc0[v], es[v]);
        } else {
            ticket = gemv_ticket(a, slab, nch);
            if constexpr (NORM) (void)norm_inv();
        }
        gemv_finish<NV, PAIR>(a, acc0, red, wave, nw, lane, slab, c, nch, ticket);
        return;
    }
    SlotGroup<T> cur, nxt;
    // Wave w takes the chunk's groups g0 + w, g0 + w + nw, ... (sf to sl): at each step the
    // workgroup's waves read consecutive groups of the slab (measured on MI355X against contiguous
    // runs per wave: Q6_K 151936 x 5120 M = 1 115.7 -> 114.6 us, M = 4 185 -> 172)
    const uint32_t sf = g0 + wave;
    const uint32_t sl = sf < g1 ? sf + (g1 - 1 - sf) / nw * nw : sf;
    if (sf < g1) {  // x first: the A table is built while the weights are on their way
        mx_load_x<NV>(xr, a.x, a.x_stride, sf, S, lane);
        if constexpr (NORM) mx_load_nw(wr, a.norm_w, sf, S, lane);
        load_group<T>(cur, slab0, geo, lane, sf, S);
    }
    ticket = gemv_ticket(a, slab, nch);
    float inv = 1.0f;
    if constexpr (NORM) inv = norm_inv();
    // One group: build its A table from xr, prefetch x and the weights of the wave's next group
    // (past its last group: the last one again, an L2 hit, so the loop stays branch-free), multiply.
    auto step = [&](const SlotGroup<T>& G, SlotGroup<T>& next, uint32_t grp) {
        s16x4 A[4 * M];
        int es[NV];
        float xs[NV];
        if constexpr (NORM) mx_norm_x(xr, wr, inv, grp, S, lane);
        mx_build<T, NV>(xr, tab, lane, A, es, xs);
        const uint32_t gn = min(grp + nw, sl);
        mx_load_x<NV>(xr, a.x, a.x_stride, gn, S, lane);
        if constexpr (NORM) mx_load_nw(wr, a.norm_w, gn, S, lane);
        load_group<T>(next, slab0, geo, lane, gn, S);
        float accg[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) accg[v] = 0.0f;
        mx_group<T, NV>(G, A, xs, min(8u, S - grp * 8), accg);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc0[v] += ldexpf(accg[v], es[v]);
    };
    for (uint32_t grp = sf; grp < g1; grp += nw) {
        step(cur, nxt, grp);
        if (grp + nw >= g1) break;
        grp += nw;
        step(nxt, cur, grp);
    }
    gemv_finish<NV, PAIR>(a, acc0, red, wave, nw, lane, slab, c, nch, ticket);
}

template <uint32_t T, int NV, bool PAIR, bool ONE, bool NORM = false>
__global__ __launch_bounds__((mx_max_threads<T, NV, ONE>())) void k_gemv_mx(GemvSlabArgs a) {
    gemv_mx_body<T, NV, PAIR, ONE, NORM>(a, blockIdx.x);
}

// ------------------------------------------------------------------------------------------
// Even split: k_gemv_mx_even<T, NV, PAIR, NORM> (the one-group form of a large launch).
//
// A chunked split gives each workgroup one K chunk of one slab, so the workgroup count is slabs
// x chunks, and the CUs do not get equal work: 272 slabs x 4 chunks = 1088 workgroups put 5
// workgroups on 64 of the 256 CUs and 4 on the rest, and the last weights of the launch arrive
// on the 64 (measured with per-wave timestamps). Here the launch's W workgroups (a multiple of
// the CU count) take equal shares [b G / W, (b + 1) G / W) of the launch's G = slabs x matrices x
// groups slot groups ("units"), in (slab, matrix, group) order.
// Inside a workgroup, wave w takes the units w and w + nw of the share (one each when the share
// has at most nw units), and each unit's sum goes to its own LDS entry.
// The units of a (slab, matrix) in the share form a segment: one piece of its slab's split-K meeting, summed
// from the entries in unit order by the wave holding its first unit (which took the slab's
// ticket); the pieces of a slab are numbered by workgroup, the gate matrix's first. A slab that
// lies wholly inside one workgroup meets in LDS alone. The sums depend on W only: nw is chosen
// per vector count so that the launch's workgroups fit the CUs in one round.
// In-kernel norm: the first workgroup runs the chains and publishes 1 / rms to one word per
// workgroup, tagged with the generation of that workgroup's first slab (its wave 0 always holds
// a ticket for that slab: the slab's reducer, or the workgroup itself for a slab wholly inside
// it, moves the generation on); each workgroup clears its word when it has read it.
// ------------------------------------------------------------------------------------------
// The even split's workgroup count: 2 per CU of an MI355X
constexpr uint32_t kEvenW = 512;
// the even split's in-kernel norm: wave 0 of the first workgroup publishes for the other kEvenW - 1
constexpr uint32_t kEvenPublishPerLane = 8;
static_assert(kEvenW - 1 <= 64 * kEvenPublishPerLane, "one published word per workgroup");
// x / d for x, d < 2^22, given inv = 1.0f / d: the float quotient is within one of x / d (relative
// error below 2^-22), then corrected (a few instructions where an integer divide takes about 30)
__device__ __forceinline__ uint32_t udiv_inv(uint32_t x, uint32_t d, float inv) {
    const uint32_t q = (uint32_t)((float)x * inv);
    const int r = (int)(x - q * d);
    return r < 0 ? q - 1 : (r >= (int)d ? q + 1 : q);
}

// Units per wave at most: two where the kernel's registers leave fewer resident waves than the
// two workgroups of a CU need with one unit each (two vectors; every vector count of the formats
// with the heavier loops, whose 2- to 4-vector kernels also take at most 8 waves), else one (nw is
// then the share's size; a second unit's registers would spill in the 3- and 4-vector kernels of
// the others)
template <uint32_t T, int NV>
constexpr uint32_t even_units_per_wave() {
    constexpr bool heavy = T == kQ8_0 || T == kQ6_K || T == kQ5_K;
    return (NV == 2 || heavy) ? 2u : 1u;
}
// The workgroup whose share holds unit u (of G over kEvenW workgroups; inv_g = 1.0f / G)
__device__ __forceinline__ uint32_t even_wg(uint32_t u, uint32_t G, float inv_g) {
    return udiv_inv((u + 1) * kEvenW - 1, G, inv_g);
}

template <uint32_t T, int NV, bool PAIR, bool NORM>
__device__ __forceinline__ void gemv_mx_even_body(const GemvSlabArgs& a, uint32_t bid) {
    static_assert(!NORM || NV == 1, "the in-kernel norm is the one-vector form");
    extern __shared__ float smem[];
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    constexpr int M = mx_blocks<NV>();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint32_t S = a.cols / kSlot, ngrp = (S + 7) / 8, U = MATS * ngrp;
    const uint32_t G = ((a.rows + kSlabRows - 1) / kSlabRows) * U, W = kEvenW;
    const uint32_t L0 = bid * G / W, L1 = (bid + 1) * G / W;
    const uint32_t nu = (G + W - 1) / W;  // LDS entries: the largest share
    const SlabGeom geo = slab_geom(T, a.cols);
    float* red = smem;  // [nu][NV][64]
    uint8_t* tab = reinterpret_cast<uint8_t*>(smem + nu * NV * 64) + wave * mx_table_bytes<NV>();
    float* sq = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(smem) + even_lds_bytes<NV>(nu, nw));
    const bool words = NORM && a.norm_words != nullptr;
    const bool leader = !words || bid == 0;  // runs the norm's chains
    const uint32_t slot = 8 * norm_chain_stride(a.cols - a.cols % 8u);  // sq[slot]: 1 / rms for the workgroup
    if constexpr (NORM) {
        // the first workgroup publishes for workgroups 1 .. W - 1, tagged with the generation of
        // each one's first slab, before it issues any weight load
        if (words && bid == 0)
            norm_leader_publish<kEvenPublishPerLane>(
                a, sq, wave, lane, W - 1,
                [&](uint32_t i) { return udiv_inv((i + 1) * G / W, ngrp, a.even_inv_ngrp) / MATS; },
                [&](uint32_t i) { return a.norm_words + i + 1; });
        else if (!words)  // every workgroup runs the chains: the squares now, the chains after its loads
            norm_x_squares(a.x, a.cols, sq, threadIdx.x, blockDim.x);
        __builtin_amdgcn_sched_barrier(0);
    }
    // A unit u of the share: its segment (slab * MATS + matrix), the segment's first unit in the
    // share, whether its slab lies inside the share, and whether u leads a segment that takes a
    // ticket (every piece; with published words also the share's first unit, as above)
    auto seg_of = [&](uint32_t u) { return udiv_inv(u, ngrp, a.even_inv_ngrp); };
    auto seg_first = [&](uint32_t u) { return max(L0, seg_of(u) * ngrp); };
    auto whole_of = [&](uint32_t u) {
        const uint32_t s_lo = seg_of(u) / MATS * U;
        return s_lo >= L0 && s_lo + U <= L1;
    };
    auto ticketed = [&](uint32_t u) { return u == seg_first(u) && (!whole_of(u) || (words && u == L0)); };
    constexpr uint32_t KU = even_units_per_wave<T, NV>();
    uint32_t tickets[KU];
    // NORM (one unit per wave): 1 / rms for the workgroup, once by every wave (the barriers of the
    // wait, of the publishing workgroup, or of the chains when nothing is published)
    auto norm_inv = [&]() {
        if (!leader) {
            const float inv = norm_x_wait(a, bid, tickets[0], sq + slot);
            if (threadIdx.x == 0) __hip_atomic_store(a.norm_words + bid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return inv;
        }
        if (words) return norm_leader_inv(a.cols, sq);
        return norm_x_chains(a.x, a.cols, a.norm_eps, sq, wave, lane);
    };
#pragma unroll
    for (uint32_t k = 0; k < KU; ++k) {
        tickets[k] = 0;
        const uint32_t u = L0 + wave + k * nw;
        if (u >= L1) break;
        const uint32_t seg = seg_of(u), slab = seg / MATS, mat = seg - slab * MATS, grp = u - seg * ngrp;
        const uint8_t* wp = (mat ? a.w1 : a.w0) + (uint64_t)slab * geo.slab_bytes;
        float xr[NV][4];
        float wr[4];  // NORM: norm_w at this lane's x elements
        SlotGroup<T> Gr;
        // x first: the A table is built while the weights are on their way
        mx_load_x<NV>(xr, a.x, a.x_stride, grp, S, lane);
        if constexpr (NORM) mx_load_nw(wr, a.norm_w, grp, S, lane);
        load_group<T>(Gr, wp, geo, lane, grp, S);
        if (ticketed(u) && lane == 0)
            tickets[k] = __hip_atomic_fetch_add(&a.counters[slab], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (NORM) mx_norm_x(xr, wr, norm_inv(), grp, S, lane);
        s16x4 A[4 * M];
        int es[NV];
        float xs[NV];
        float acc[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
        mx_build<T, NV>(xr, tab, lane, A, es, xs);
        mx_group<T, NV>(Gr, A, xs, min(8u, S - grp * 8), acc);
#pragma unroll
        for (int v = 0; v < NV; ++v) red[((u - L0) * NV + v) * 64 + lane] = ldexpf(acc[v], es[v]);
        // the next unit's loads after this one's arithmetic (its registers are free again)
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NORM) {
        // a wave without a unit (the share is smaller than the workgroup) still takes part
        if (wave >= L1 - L0) (void)norm_inv();
    }
    __syncthreads();
    // the segments this wave leads: their units' entries in unit order, then the slab's meeting
#pragma unroll
    for (uint32_t k = 0; k < KU; ++k) {
        const uint32_t u = L0 + wave + k * nw;
        if (u >= L1) break;
        if (u != seg_first(u)) continue;
        const uint32_t seg = seg_of(u), slab = seg / MATS, mat = seg - slab * MATS;
        const uint32_t s_lo = slab * U, s_hi = s_lo + U;
        const bool whole = whole_of(u);
        if (PAIR && whole && mat == 1) continue;  // a whole slab's gate lead takes its up half
        const uint32_t seg_hi = min(L1, seg * ngrp + ngrp);
        float acc0[NV], acc1[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            float s = red[((u - L0) * NV + v) * 64 + lane];
            for (uint32_t e = u - L0 + 1; e < seg_hi - L0; ++e) s += red[(e * NV + v) * 64 + lane];
            acc0[v] = s;
            acc1[v] = 0.0f;
        }
        if (whole) {
            if constexpr (PAIR) {
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    float s = red[((s_lo + ngrp - L0) * NV + v) * 64 + lane];
                    for (uint32_t e = s_lo + ngrp - L0 + 1; e < s_hi - L0; ++e) s += red[(e * NV + v) * 64 + lane];
                    acc1[v] = s;
                }
            }
            if (ticketed(u) && lane == 0)  // no reducer: the generation moves on here
                __hip_atomic_store(&a.counters[slab], ((tickets[k] >> kTicketBits) + 1) << kTicketBits, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            gemv_store<NV, PAIR>(a, acc0, acc1, slab, lane);
            continue;
        }
        // this slab's pieces: the workgroups over its gate units, then those over its up units
        const float ig = a.even_inv_units;
        const uint32_t wa0 = even_wg(s_lo, G, ig), n0 = even_wg(s_lo + ngrp - 1, G, ig) - wa0 + 1;
        uint32_t nch = n0, c = bid - wa0;
        if constexpr (PAIR) {
            const uint32_t wa1 = even_wg(s_lo + ngrp, G, ig);
            nch += even_wg(s_hi - 1, G, ig) - wa1 + 1;
            if (mat) c = n0 + bid - wa1;
        }
        if (splitk_meet<NV, false>(a, acc0, acc1, lane, slab, c, nch, n0, a.even_stride, tickets[k]))
            gemv_store<NV, PAIR>(a, acc0, acc1, slab, lane);
    }
}

template <uint32_t T, int NV, bool PAIR, bool NORM = false>
__global__ __launch_bounds__((mx_max_threads<T, NV, true>())) void k_gemv_mx_even(GemvSlabArgs a) {
    gemv_mx_even_body<T, NV, PAIR, NORM>(a, blockIdx.x);
}

}  // namespace
}  // namespace halo_mi
