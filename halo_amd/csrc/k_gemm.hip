// gfx950 GEMM kernels of the halo_mi355x library (M >= 8), bf16 MFMA with exact dequantization:
//   k_gemm_pc  producer / consumer workgroups (M <= 256)
//   k_gemm_lm  512-row M tiles, every wave dequantizes and multiplies (M > 256)
// plus the fused SwiGLU epilogue and the standalone SWIGLU op.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "device.h"
#include "launch.h"

namespace halo_mi {
namespace {

using namespace dev;

// SiLU for the GEMM epilogues: v * rcp(1 + 2^(-v log2 e)) on v_exp_f32 and v_rcp_f32 (five
// instructions instead of the IEEE divide and expf). Relative error at most (1.5 |v| + 8) 2^-24:
// the rounded argument moves 2^(.) by at most 1.5 |v| 2^-24 relative, v_exp_f32 and v_rcp_f32
// are within 1 ulp, the add and multiplies round once each, and 1 / (1 + e) damps the error of
// e by e / (1 + e) <= 1. The bf16 GEMM's own error bound is larger by orders of magnitude; the
// GEMV pair (fp32 throughout) keeps the IEEE form.
__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.44269504088896341f));
}

// ==========================================================================================
// SWIGLU (backends/cpu/ops_basic.cpp:165-167): out = silu(g) * u, rows x cols
// ==========================================================================================

__global__ void k_swiglu(const float* __restrict__ g, uint64_t gs, const float* __restrict__ u, uint64_t us,
                         float* __restrict__ out, uint64_t os, uint32_t rows, uint32_t cols) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)rows * cols) return;
    const uint64_t r = idx / cols, c = idx % cols;
    out[r * os + c] = silu_f(g[r * gs + c]) * u[r * us + c];
}

// ==========================================================================================
// SLAB GEMM, producer / consumer workgroups on v_mfma_f32_32x32x16_bf16
// ==========================================================================================
//
// x is first rounded to bf16 (RNE) and stored in MFMA A-fragment order (k_x_to_frag). A
// workgroup owns a BM x 128 tile of the output: BM x rows times 128 W rows, which are gate rows
// [64 u, 64 u + 64) followed by the up rows of the same range (PAIR), or two consecutive slabs.
// It has 8 waves:
//   waves 0-3 (consumers) hold the tile in fp32 accumulators, load their x fragments straight
//     from the fragment-ordered buffer (a ring of kPcADepth stages in registers), read the W
//     fragments from LDS and run the MFMAs;
//   waves 4-7 (producers) keep kPcDepth stages of W records in flight, dequantize W exactly
//     (the reference's expressions, see pc_dequant), round to bf16 (RNE) and write the stage
//     two ahead of the consumers to LDS.
// A stage is one 32-weight slot of K; one barrier per stage. LDS carries only W (the measured
// LDS bandwidth, about 100 B/clk per CU, could not also carry x at the MFMA rate).

constexpr int kPcLd = 40;     // LDS row pitch in bf16 (32 k + 8 pad: 80 B, conflict-free reads)
constexpr int kPcW = 128;     // W rows per tile
constexpr int kPcDepth = 4;   // stages of producer W loads in flight (a ring of registers)
constexpr int kPcADepth = 4;  // stages of consumer x-fragment loads in flight
constexpr uint32_t kPcOob = 0x80000000u;  // buffer offset past every resource: the load returns 0
constexpr int kPcBufs = 4;    // LDS stages (the producers write two stages ahead)
constexpr int kPcUnroll = 8;  // k_gemm_lm's loop unroll: ring slot, LDS buffer and Q4_K sub-block static
constexpr int kPcPUnroll = kPcDepth > 8 ? kPcDepth : 8;  // the same for k_gemm_pc's producers

struct GemmPcArgs {
    const uint8_t* w0;     // gate (PAIR) or the matrix
    const uint8_t* w1;     // up (PAIR) or null
    const __bf16* xf;      // x in fragment order (k_x_to_frag), m_tiles * BM rows, rows >= n_vec zero
    float* y;
    uint64_t y_stride;
    uint32_t rows, cols, n_vec;
    uint32_t units;        // W tiles [0, units) run whole (PAIR: slabs; else pairs of slabs), all M tiles
    uint32_t m_tiles;
    uint32_t xcd_map;      // whole tiles grouped by XCD so an XCD reuses one slice of x
    // W tiles [split_unit0, split_unit0 + split_units) (all M tiles) run as kchunks K chunks each,
    // one workgroup per chunk after the whole tiles; their fp32 partials go to
    // partials[(split tile * kchunks + chunk)][BM][128] and k_gemm_pc_reduce adds them.
    uint32_t split_units;
    uint32_t kchunks;
    float* partials;
    uint32_t split_unit0 = 0;  // W tile of the first split tile (units when both kinds share a launch)
    // the small-M kernel at up to 8 rows reads x itself (fp32, normalized as k_x_to_frag does
    // when nw is set) instead of the staged fragments
    const float* x = nullptr;
    uint64_t x_stride = 0;
    const float* inv = nullptr;
    const float* nw = nullptr;
};

// Producer barrier: its LDS writes are complete, then s_barrier. Global loads stay in flight.
// The memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void pc_sync() { __asm__ __volatile__("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Consumer barrier: its outstanding LDS reads target a stage no producer writes before the
// next barrier, so it does not wait for them.
__device__ __forceinline__ void pc_barrier() { __asm__ __volatile__("s_barrier" ::: "memory"); }

// Load of a T at a wave-uniform base plus a 32-bit per-lane byte offset (scalar base address,
// vector offset).
template <typename V>
__device__ __forceinline__ V ldg(const uint8_t* ubase, uint32_t voff) {
    return *reinterpret_cast<const V*>(ubase + voff);
}

// x fp32 -> bf16 (RNE) in MFMA A-fragment order. For 32-row block b of x, slot s of K and half
// k16 of the slot, 1 KB holds, for lane l, the 8 values x[32 b + l % 32][32 s + 16 k16 + 8 (l / 32) + e]
// (the A operand of v_mfma_f32_32x32x16_bf16). Rows in [n_vec, m_pad) are zero. One thread
// writes one lane's 16 bytes: the writes of a wave are one contiguous 1 KB.
// With the fused norm (nw set), x is first normalized as cpu::rms_norm does, (x * inv[m]) * nw[k],
// inv from k_rms_inv_rows: the staged values are the CPU's normalized x rounded to bf16.
__global__ void k_x_to_frag(const float* __restrict__ x, uint64_t x_stride, uint32_t n_vec, uint32_t m_pad,
                            uint32_t cols, __bf16* __restrict__ out, const float* __restrict__ inv,
                            const float* __restrict__ nw) {
#pragma clang fp contract(off)
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)m_pad * (cols / 8)) return;
    const uint32_t S = cols / kSlot;
    const uint32_t l = (uint32_t)(idx & 63u);
    const uint64_t f = idx >> 6;  // fragment index: (b * S + s) * 2 + k16
    const uint32_t k16 = (uint32_t)(f & 1u), sl = (uint32_t)((f >> 1) % S);
    const uint32_t b = (uint32_t)((f >> 1) / S);
    const uint32_t m = 32 * b + (l & 31u), k = 32 * sl + 16 * k16 + 8 * (l >> 5);
    bf16x8 v;
    if (m < n_vec) {
        const float4 a = *reinterpret_cast<const float4*>(x + (uint64_t)m * x_stride + k);
        const float4 c = *reinterpret_cast<const float4*>(x + (uint64_t)m * x_stride + k + 4);
        float e[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        if (nw) {
            const float s = inv[m];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float t = e[i] * s;
                e[i] = t * nw[k + i];
            }
        }
        v = bf16x8{(__bf16)e[0], (__bf16)e[1], (__bf16)e[2], (__bf16)e[3], (__bf16)e[4], (__bf16)e[5], (__bf16)e[6], (__bf16)e[7]};
    } else {
        v = bf16x8{};
    }
    *reinterpret_cast<bf16x8*>(out + idx * 8) = v;
}

// One producer thread's share of one slot: 16 weights of one row (half h of the slot record:
// elements 8h..8h+7 and 16+8h..16+8h+7) and what scales them.
template <uint32_t T>
struct PcW;
template <>
struct PcW<kQ4_K> {
    uint2 q;
    uint4 hdr;
};
template <>
struct PcW<kQ4_0> {
    uint2 q;
    uint32_t d;
};
template <>
struct PcW<kQ8_0> {
    uint2 qa, qb;
    uint32_t d;
};
template <>
struct PcW<kQ6_K> {
    uint2 ql;
    uint32_t qh, sc, d;
};
template <>
struct PcW<kQ5_K> {
    uint2 q;
    uint32_t qh;
    uint4 hdr;
};
template <>
struct PcW<kIQ4_XS> {
    uint2 q, hdr;
};

// Buffer resource over [base, base + bytes) for raw buffer loads (gfx9 dword 3: 32-bit data
// format, untyped access). Offsets past `bytes` read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ uint2 bld64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    return uint2{v[0], v[1]};
}
__device__ __forceinline__ uint32_t bld32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
// The same with a cache policy (2: nontemporal) for weight records read once per launch
template <int CP>
__device__ __forceinline__ uint4 bld128p(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CP);
    return uint4{v[0], v[1], v[2], v[3]};
}
template <int CP>
__device__ __forceinline__ uint2 bld64p(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, CP);
    return uint2{v[0], v[1]};
}
template <int CP>
__device__ __forceinline__ uint32_t bld32p(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, CP);
}
template <int CP>
__device__ __forceinline__ uint32_t bld16p(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, CP);
}

// Per-lane byte offsets of a producer thread's records inside one stage of a slab.
struct PcOff {
    uint32_t q, aux, sc, d;
};

template <uint32_t T>
__device__ __forceinline__ PcOff pc_offsets(uint32_t r, uint32_t h) {
    if constexpr (T == kQ4_K) return {r * 16 + 8 * h, r * 16, 0, 0};
    else if constexpr (T == kQ4_0 || T == kQ8_0) return {r * 16 + 8 * h, r * 2, 0, 0};
    else if constexpr (T == kQ5_K) return {r * 16 + 8 * h, r * 4, r * 16, 0};
    else if constexpr (T == kIQ4_XS) return {r * 16 + 8 * h, r * 8, 0, 0};
    else return {r * 16 + 8 * h, r * 8 + 4 * h, r * 16, r * 2};
}

// The per-super-block fields of a weight record (none for the 32-weight block formats).
template <uint32_t T>
struct SmH {};
template <>
struct SmH<kQ4_K> {
    uint4 hdr;
};
template <>
struct SmH<kQ5_K> {
    uint4 hdr;
};
template <>
struct SmH<kIQ4_XS> {
    uint2 hdr;
};
template <>
struct SmH<kQ6_K> {
    uint4 sc;  // the 16 int8 scales of the row's super-block
    uint32_t d;
};

// The per-slot fields of a weight record (codes; Q4_0 / Q8_0's d, Q5_K / Q6_K's high bits). NT:
// nontemporal loads (k_gemm_pc, measured on MI355X at gate/up M = 64: 49.9 -> 49.3 us; the
// M = 512 and small-M kernels measured the same or slower with them)
template <uint32_t T, bool NT = false>
__device__ __forceinline__ void sm_load_q(PcW<T>& R, __amdgpu_buffer_rsrc_t slab, const SlabGeom& g, const PcOff& o,
                                          uint32_t s, bool live) {
    auto so = [&](uint64_t x) { return live ? (uint32_t)x : kPcOob; };
    if constexpr (T == kQ4_K || T == kIQ4_XS) {
        R.q = bld64p<NT ? 2 : 0>(slab, o.q, so(g.q_off + s * 1024));
    } else if constexpr (T == kQ4_0) {
        R.q = bld64p<NT ? 2 : 0>(slab, o.q, so(g.q_off + s * 1024));
        R.d = bld16p<NT ? 2 : 0>(slab, o.aux, so(g.aux_off + s * 128));
    } else if constexpr (T == kQ5_K) {
        R.q = bld64p<NT ? 2 : 0>(slab, o.q, so(g.q_off + s * 1024));
        R.qh = bld32p<NT ? 2 : 0>(slab, o.aux, so(g.aux_off + s * 256));
    } else if constexpr (T == kQ8_0) {
        R.qa = bld64p<NT ? 2 : 0>(slab, o.q, so(g.q_off + s * 2048));
        R.qb = bld64p<NT ? 2 : 0>(slab, o.q, so(g.q_off + s * 2048 + 1024));
        R.d = bld16p<NT ? 2 : 0>(slab, o.aux, so(g.aux_off + s * 128));
    } else {
        R.ql = bld64p<NT ? 2 : 0>(slab, o.q, so(g.q_off + s * 1024));
        R.qh = bld32p<NT ? 2 : 0>(slab, o.aux, so(g.aux_off + s * 512));
    }
}

// The per-super-block fields of super-block sb (NT as sm_load_q's).
template <uint32_t T, bool NT = false>
__device__ __forceinline__ void sm_load_h(SmH<T>& H, __amdgpu_buffer_rsrc_t slab, const SlabGeom& g, const PcOff& o,
                                          uint32_t sb, bool live) {
    auto so = [&](uint64_t x) { return live ? (uint32_t)x : kPcOob; };
    if constexpr (T == kQ4_K) {
        H.hdr = bld128p<NT ? 2 : 0>(slab, o.aux, so(g.aux_off + sb * 1024));
    } else if constexpr (T == kQ5_K) {
        H.hdr = bld128p<NT ? 2 : 0>(slab, o.sc, so(g.sc_off + sb * 1024));
    } else if constexpr (T == kIQ4_XS) {
        H.hdr = bld64p<NT ? 2 : 0>(slab, o.aux, so(g.aux_off + sb * 512));
    } else if constexpr (T == kQ6_K) {
        H.sc = bld128p<NT ? 2 : 0>(slab, o.sc, so(g.sc_off + sb * 1024));
        H.d = bld16p<NT ? 2 : 0>(slab, o.d, so(g.d_off + sb * 128));
    }
}

// Completes R with sub-block j's fields of the super-block header H.
template <uint32_t T>
__device__ __forceinline__ void sm_merge(PcW<T>& R, const SmH<T>& H, int j) {
    if constexpr (T == kQ4_K || T == kQ5_K || T == kIQ4_XS) {
        R.hdr = H.hdr;
    } else if constexpr (T == kQ6_K) {
        const uint32_t w = (j >> 1) == 0 ? H.sc.x : (j >> 1) == 1 ? H.sc.y : (j >> 1) == 2 ? H.sc.z : H.sc.w;
        R.sc = (w >> (16 * (j & 1))) & 0xFFFFu;
        R.d = H.d;
    }
}

// q4k_sc_m for a sub-block index known only at run time, without branches.
__device__ __forceinline__ void q4k_sc_m_sel(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j, uint32_t& sc,
                                             uint32_t& m) {
    const uint32_t sh = 8 * (j & 3u);
    const uint32_t b8 = (s2 >> sh) & 0xFFu;
    const uint32_t lsc = (s0 >> sh) & 63u, lm = (s1 >> sh) & 63u;
    const uint32_t hsc = (b8 & 15u) | (((s0 >> (sh + 6)) & 3u) << 4);
    const uint32_t hm = (b8 >> 4) | (((s1 >> (sh + 6)) & 3u) << 4);
    sc = j < 4 ? lsc : hsc;
    m = j < 4 ? lm : hm;
}

// The 16 weights of a PcW, exact (each is one correctly rounded fp32 operation on exact
// products, equal to the reference's expression), then rounded to bf16.
//   Q4_K d1 q - m1 = fma(d1 / u, q u, -m1)      (q u from the fp8 convert, u = fp8_unit())
//   Q4_0 (q - 8) d = fma(d / u, q u, -8 d)      (exact: d (q - 8) is representable)
//   Q8_0 q d       = fma(d, q + 128, -128 d)    (q + 128 as an unsigned byte; exact)
//   Q6_K (d sc)(q - 32) = fma(d sc, q, -32 d sc) (exact)
//   Q5_K d1 q - m1 = fma(d1, q, -m1)             (d1 q exact: 17 x 5 bits)
//   IQ4_XS dl v    = fma(dl, v + 128, -128 dl)   (v + 128 from the biased table; exact)
template <uint32_t T>
__device__ __forceinline__ void pc_dequant(const PcW<T>& R, uint32_t h, uint32_t j, float inv_unit, bf16x8& lo,
                                           bf16x8& hi) {
    float a[8], b[8];
    if constexpr (T == kQ4_K || T == kQ4_0) {
        float sA, oA;
        if constexpr (T == kQ4_K) {
            uint32_t sc, m;
            q4k_sc_m_sel(R.hdr.y, R.hdr.z, R.hdr.w, j, sc, m);
            const float d1 = h2f(R.hdr.x & 0xFFFFu) * (float)sc, m1 = h2f(R.hdr.x >> 16) * (float)m;
            sA = d1 * inv_unit;
            oA = -m1;
        } else {
            const float d = h2f(R.d);
            sA = d * inv_unit;
            oA = -8.0f * d;
        }
        const uint32_t Q[2] = {R.q.x, R.q.y};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t lc = and_opaque<0x0F0F0F0Fu>(Q[w]), hc = and_opaque<0x0F0F0F0Fu>(Q[w] >> 4);
            const float2v l01 = __builtin_amdgcn_cvt_pk_f32_fp8(lc, false), l23 = __builtin_amdgcn_cvt_pk_f32_fp8(lc, true);
            const float2v h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hc, false), h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hc, true);
            a[4 * w + 0] = fmaf(sA, l01[0], oA);
            a[4 * w + 1] = fmaf(sA, l01[1], oA);
            a[4 * w + 2] = fmaf(sA, l23[0], oA);
            a[4 * w + 3] = fmaf(sA, l23[1], oA);
            b[4 * w + 0] = fmaf(sA, h01[0], oA);
            b[4 * w + 1] = fmaf(sA, h01[1], oA);
            b[4 * w + 2] = fmaf(sA, h23[0], oA);
            b[4 * w + 3] = fmaf(sA, h23[1], oA);
        }
    } else if constexpr (T == kQ5_K) {
        uint32_t sc, m;
        q4k_sc_m_sel(R.hdr.y, R.hdr.z, R.hdr.w, j, sc, m);
        const float d1 = h2f(R.hdr.x & 0xFFFFu) * (float)sc, o = -(h2f(R.hdr.x >> 16) * (float)m);
        // record dword i = 2 h + w: fifth bits at (qh << (4 - i)) and (qh >> i), masked to bit 4
        // of each byte; the shift by 2 h first (bits 0..1 of qh belong to h = 0 only)
        const uint32_t hq = R.qh >> (2 * h);
        const uint32_t Q[2] = {R.q.x, R.q.y};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t lc = and_or_opaque(Q[w], 0x0F0F0F0Fu, (hq << (4 - w)) & 0x10101010u);
            const uint32_t hc = and_or_opaque(Q[w] >> 4, 0x0F0F0F0Fu, (hq >> w) & 0x10101010u);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[4 * w + k] = fmaf(d1, ubyte(lc, k), o);
                b[4 * w + k] = fmaf(d1, ubyte(hc, k), o);
            }
        }
    } else if constexpr (T == kIQ4_XS) {
        const float dl = h2f(R.hdr.x & 0xFFFFu) * (float)iq4xs_ls(R.hdr.x >> 16, R.hdr.y, j), o = -128.0f * dl;
        const uint32_t Q[2] = {R.q.x, R.q.y};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t lc = iq4_lookup4(Q[w]), hc = iq4_lookup4(Q[w] >> 4);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[4 * w + k] = fmaf(dl, ubyte(lc, k), o);
                b[4 * w + k] = fmaf(dl, ubyte(hc, k), o);
            }
        }
    } else if constexpr (T == kQ8_0) {
        const float d = h2f(R.d), o = -128.0f * d;
        const uint32_t A[2] = {xor_opaque<0x80808080u>(R.qa.x), xor_opaque<0x80808080u>(R.qa.y)};
        const uint32_t B[2] = {xor_opaque<0x80808080u>(R.qb.x), xor_opaque<0x80808080u>(R.qb.y)};
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[4 * w + k] = fmaf(d, ubyte(A[w], k), o);
                b[4 * w + k] = fmaf(d, ubyte(B[w], k), o);
            }
    } else {
        const float d = h2f(R.d);
        const float dA = d * sbyte(R.sc, 0), dB = d * sbyte(R.sc, 1);
        const float oA = -32.0f * dA, oB = -32.0f * dB;
        const uint32_t x0 = R.ql.x, x1 = R.ql.y, hq = R.qh;
        const uint32_t L[2] = {and_or_opaque(x0, 0x0F0F0F0Fu, hq & 0x30303030u), and_or_opaque(x1, 0x0F0F0F0Fu, (hq << 4) & 0x30303030u)};
        const uint32_t H[2] = {and_or_opaque(x0 >> 4, 0x0F0F0F0Fu, (hq >> 2) & 0x30303030u),
                               and_or_opaque(x1 >> 4, 0x0F0F0F0Fu, (hq << 2) & 0x30303030u)};
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a[4 * w + k] = fmaf(dA, ubyte(L[w], k), oA);
                b[4 * w + k] = fmaf(dB, ubyte(H[w], k), oB);
            }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo[i] = (__bf16)a[i];
        hi[i] = (__bf16)b[i];
    }
}

// Row (M index) of accumulator element r (0..15) held by `lane` in a 32x32 MFMA result; the
// column (N index) is lane % 32.
__device__ __forceinline__ uint32_t mfma32_row(uint32_t r, uint32_t lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// grid = units * m_tiles * kchunks, block = 512; BM = 64 MB x rows per tile.
//
// A workgroup runs the stages (slots of K) [s_begin, s_end) of its tile; s_begin is a multiple
// of 8 (one Q4_K / Q6_K super-block). Barrier B_i (i = 0..n_pad) orders them: the producers
// write local stages 0 and 1 before B_0 and stage i + 2 between B_i and B_{i+1} (LDS buffer
// (i + 2) % 4); the consumers compute stage i between B_i and B_{i+1}, and read the first W
// fragments of stage i + 1 at its end (complete since B_i). A buffer is rewritten two barriers
// after its last read.
//
// Consumer waves: WM along M x WN along N; a wave owns MBW 32-row x blocks and NBW 32-row W
// blocks. With PAIR its first NBW / 2 W blocks are gate rows and the others the up rows of the
// same range, so every lane holds matching gate and up sums.
constexpr uint32_t kPcStage = kPcW * kPcLd;  // bf16 per LDS stage of k_gemm_pc (W only)

// The body of workgroup `bid` of a k_gemm_pc launch over the matrix of `a` (also one segment of a
// grouped launch, k_gemm_pc_group); lds: kPcBufs stages.
template <uint32_t T, bool PAIR, int MB>
__device__ __forceinline__ void gemm_pc_body(const GemmPcArgs& a, uint32_t bid, __bf16* lds) {
    constexpr int BM = 64 * MB;
    // KH (64-row tiles): wave w multiplies x block w % 2 by all four W blocks over K half w / 2
    // of every stage, so each x fragment is loaded by one wave; the pairs' sums meet at the end
    constexpr bool KH = MB == 1;
    constexpr int WM = MB == 1 ? 2 : 4, WN = KH ? 1 : 4 / WM;
    constexpr int MBW = BM / WM / 32, NBW = 4 / WN;
    constexpr uint32_t STAGE = kPcStage;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t S = a.cols / kSlot;
    const SlabGeom g = slab_geom(T, a.cols);
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;

    // workgroup -> (W tile u, M tile mt) for a whole tile, or (split tile st, K chunk)
    const uint32_t whole = a.units * a.m_tiles;
    const bool split = bid >= whole;
    uint32_t u, mt, st = 0, chunk = 0;
    if (!split) {
        const uint32_t wg = bid;
        if (a.xcd_map) {
            const uint32_t grp = 8 / a.m_tiles, xcd = wg % 8;
            mt = xcd / grp;
            u = (wg / 8) * grp + xcd % grp;
        } else {
            u = wg / a.m_tiles;
            mt = wg % a.m_tiles;
        }
    } else {
        st = (bid - whole) / a.kchunks;
        chunk = (bid - whole) % a.kchunks;
        u = a.split_unit0 + st / a.m_tiles;
        mt = st % a.m_tiles;
    }
    const uint32_t m0 = mt * BM;
    // this chunk's stages: whole groups of 8 slots when K is split
    uint32_t s_begin = 0, s_end = S;
    if (split) {
        const uint32_t ng = S / 8, base = ng / a.kchunks, extra = ng % a.kchunks;
        const uint32_t g0 = chunk * base + min(chunk, extra);
        s_begin = 8 * g0;
        s_end = 8 * (g0 + base + (chunk < extra ? 1u : 0u));
    }
    const uint32_t n = s_end - s_begin;
    const uint32_t n_pad = (n + kPcPUnroll - 1) / kPcPUnroll * kPcPUnroll;

    if (wave < 4) {
        // ---------------- consumers ----------------
        const uint32_t wm = wave % WM, wn = KH ? 0u : wave / WM, kh = KH ? wave / WM : 0u;
        floatx16 acc[MBW][NBW];
#pragma unroll
        for (int i = 0; i < MBW; ++i)
#pragma unroll
            for (int j = 0; j < NBW; ++j) acc[i][j] = floatx16{};
        const uint32_t lr = lane & 31u, koff = 8 * (lane >> 5);
        uint32_t wrow[NBW];  // first W-tile row of each of this wave's W blocks
#pragma unroll
        for (int j = 0; j < NBW; ++j)
            wrow[j] = PAIR ? (j < NBW / 2 ? 32 * (wn * NBW / 2 + j) : 64 + 32 * (wn * NBW / 2 + j - NBW / 2))
                           : 32 * (wn * NBW + j);
        uint32_t boff[NBW];
#pragma unroll
        for (int j = 0; j < NBW; ++j) boff[j] = (wrow[j] + lr) * kPcLd + koff;
        // x fragments: this M tile's fragment-ordered rows; block (wm * MBW + i), slot s, half k
        // is at ((blk * S + s) * 2 + k) KB, lane l at 16 l bytes
        const __amdgpu_buffer_rsrc_t xres = make_rsrc(a.xf + (uint64_t)m0 * a.cols, (uint32_t)(BM * a.cols * 2));
        const uint32_t xlane = lane * 16;
        constexpr int NK = KH ? 1 : 2;  // K halves per wave and stage
        uint4 AR[kPcADepth][MBW][NK];
        // stages past s_end read zeros (out of range), so padded stages add exactly 0
        auto load_a = [&](int slot, uint32_t s) {
#pragma unroll
            for (int i = 0; i < MBW; ++i)
#pragma unroll
                for (int k = 0; k < NK; ++k)
                    AR[slot][i][k] = bld128(xres, xlane,
                                            s < s_end ? (((wm * MBW + i) * S + s) * 2 + kh + k) * 1024 : kPcOob);
        };
        bf16x8 B0[NBW], B1[NBW];
        auto read_b = [&](uint32_t buf, int k, bf16x8 (&B)[NBW]) {
            const __bf16* st = lds + buf * STAGE + 16 * k;
#pragma unroll
            for (int j = 0; j < NBW; ++j) B[j] = *reinterpret_cast<const bf16x8*>(st + boff[j]);
        };
        auto mma = [&](int slot, int k, const bf16x8 (&B)[NBW]) {
#pragma unroll
            for (int i = 0; i < MBW; ++i)
#pragma unroll
                for (int j = 0; j < NBW; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, AR[slot][i][k]), B[j],
                                                                        acc[i][j], 0, 0, 0);
        };
#pragma unroll
        for (int p = 0; p < kPcADepth; ++p) load_a(p, s_begin + p);
        pc_barrier();  // B_0: stages 0 and 1 are in LDS
        read_b(0, KH ? kh : 0u, B0);
        // stage i: x fragments from ring slot i % 4, W from LDS buffer i % 4; unrolled so both
        // are static, and branch-free so the loads' waits are exact (padded stages are zeros)
        static_assert(kPcADepth == kPcBufs, "one static index for the x ring and the LDS buffers");
        if constexpr (KH) {
            for (uint32_t i0 = 0; i0 < n_pad; i0 += kPcBufs) {
#pragma unroll
                for (int q = 0; q < kPcBufs; ++q) {
                    read_b((q + 1) % kPcBufs, kh, B1);  // stage i + 1 (complete since B_i)
                    mma(q, 0, B0);
                    load_a(q, s_begin + i0 + q + kPcADepth);
                    __builtin_amdgcn_sched_group_barrier(0x100, NBW, 0);  // DS read: next stage
                    __builtin_amdgcn_sched_group_barrier(0x008, NBW, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // VMEM read: x ring
                    pc_barrier();  // B_{i+1}
#pragma unroll
                    for (int j = 0; j < NBW; ++j) B0[j] = B1[j];
                }
            }
            // the K halves meet: after every LDS access of the loop has completed (a barrier
            // the producers join too), the second wave of each pair leaves its sums in LDS
            // and the first adds them
            pc_sync();
            float* red = reinterpret_cast<float*>(lds) + wm * (NBW * 16 * 64) + lane;
            static_assert(2 * NBW * 16 * 64 * 4 <= kPcBufs * kPcStage * sizeof(__bf16), "the pair sums fit the stage buffers");
            if (kh == 1) {
#pragma unroll
                for (int j = 0; j < NBW; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) red[(j * 16 + r) * 64] = acc[0][j][r];
            }
            pc_sync();
            if (kh == 1) return;
#pragma unroll
            for (int j = 0; j < NBW; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[0][j][r] += red[(j * 16 + r) * 64];
        } else {
            for (uint32_t i0 = 0; i0 < n_pad; i0 += kPcBufs) {
#pragma unroll
                for (int q = 0; q < kPcBufs; ++q) {
                    read_b(q, 1, B1);
                    mma(q, 0, B0);
                    read_b((q + 1) % kPcBufs, 0, B0);  // stage i + 1 (zeros or junk past the end)
                    mma(q, 1, B1);
                    load_a(q, s_begin + i0 + q + kPcADepth);
                    // issue order: W reads for the second half first, so neither batch of MFMAs waits
                    // for LDS; then the next stage's first W reads behind the first batch
                    __builtin_amdgcn_sched_group_barrier(0x100, NBW, 0);        // DS read: B1
                    __builtin_amdgcn_sched_group_barrier(0x008, MBW * NBW, 0);  // MFMA: k16 = 0
                    __builtin_amdgcn_sched_group_barrier(0x100, NBW, 0);        // DS read: next B0
                    __builtin_amdgcn_sched_group_barrier(0x008, MBW * NBW, 0);  // MFMA: k16 = 1
                    __builtin_amdgcn_sched_group_barrier(0x020, 2 * MBW, 0);    // VMEM read: x ring
                    pc_barrier();  // B_{i+1}
                }
            }
        }
        if (split) {
            // fp32 partial tile [BM][128] of this chunk
            float* P = a.partials + ((uint64_t)st * a.kchunks + chunk) * BM * kPcW;
#pragma unroll
            for (int i = 0; i < MBW; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t ml = (wm * MBW + i) * 32 + mfma32_row(r, lane);
#pragma unroll
                    for (int j = 0; j < NBW; ++j) P[ml * kPcW + wrow[j] + lr] = acc[i][j][r];
                }
            return;
        }
        // epilogue: columns of this lane, rows m per accumulator element
#pragma unroll
        for (int i = 0; i < MBW; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + (wm * MBW + i) * 32 + mfma32_row(r, lane);
                if (m >= a.n_vec) continue;
                float* yrow = a.y + (uint64_t)m * a.y_stride;
                if constexpr (PAIR) {
#pragma unroll
                    for (int j = 0; j < NBW / 2; ++j) {
                        const uint32_t col = u * kSlabRows + wrow[j] + lr;
                        if (col < a.rows) yrow[col] = silu_fast(acc[i][j][r]) * acc[i][j + NBW / 2][r];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < NBW; ++j) {
                        const uint32_t col = 2 * u * kSlabRows + wrow[j] + lr;
                        if (col < a.rows) yrow[col] = acc[i][j][r];
                    }
                }
            }
        return;
    }

    // ---------------- producers ----------------
    const uint32_t pw = wave - 4;
    const uint32_t mat = pw >> 1;  // two waves per matrix
    // lane -> (row, half): 32 consecutive rows per half-wave, so the 8 lanes of a ds_write_b128
    // group hit 8 distinct bank quads (80-byte row pitch); the record loads stay one 512-byte run
    const uint32_t r = 32 * (pw & 1u) + (lane & 31u), h = lane >> 5;
    const uint8_t* slab_ptr;
    if constexpr (PAIR) {
        slab_ptr = (mat ? a.w1 : a.w0) + (uint64_t)u * g.slab_bytes;
    } else {
        // a missing second slab reads the last one again: its outputs are never stored
        slab_ptr = a.w0 + (uint64_t)min(2 * u + mat, slabs - 1) * g.slab_bytes;
    }
    const __amdgpu_buffer_rsrc_t slab = make_rsrc(slab_ptr, (uint32_t)g.slab_bytes);
    const PcOff off = pc_offsets<T>(r, h);
    const float inv_unit = __uint_as_float(0x7F000000u - __float_as_uint(fp8_unit()));
    const uint32_t wdst = (mat * 64 + r) * kPcLd + 8 * h;
    // per-slot codes in a ring of kPcDepth stages; the super-block fields (scales, mins, d) once
    // per super-block, loaded with the codes of its first slot: H[0] serves the stages being
    // written, H[1 ..] the super-blocks whose first slot is already loaded
    constexpr int NH = (kPcDepth + 7) / 8 + 1;
    PcW<T> R[kPcDepth];
    SmH<T> H[NH];
    // first: s starts a super-block (known statically: s_begin is a multiple of 8)
    auto load = [&](int slot, uint32_t s, bool first, int hslot) {
        if (first) sm_load_h<T, true>(H[hslot], slab, g, off, s / 8, s < s_end);
        sm_load_q<T, true>(R[slot], slab, g, off, s, s < s_end);
    };
    // j: the stage's slot within its super-block (static in the unrolled loop)
    auto store = [&](int slot, uint32_t j, int buf) {
        PcW<T> W = R[slot];
        sm_merge<T>(W, H[0], j);
        bf16x8 lo, hi;
        pc_dequant<T>(W, h, j, inv_unit, lo, hi);
        __bf16* st = lds + buf * STAGE;
        *reinterpret_cast<bf16x8*>(st + wdst) = lo;
        *reinterpret_cast<bf16x8*>(st + wdst + 16) = hi;
    };
#pragma unroll
    for (int p = 0; p < kPcDepth; ++p) load(p, s_begin + p, p % 8 == 0, p / 8);
    store(0, 0, 0);
    load(0, s_begin + kPcDepth, kPcDepth % 8 == 0, kPcDepth / 8);
    store(1, 1, 1);
    load(1, s_begin + kPcDepth + 1, (kPcDepth + 1) % 8 == 0, (kPcDepth + 1) / 8);
    pc_sync();  // B_0
    // iteration i writes local stage i + 2 from ring slot (i + 2) % kPcDepth into buffer
    // (i + 2) % 4 and loads stage i + 2 + kPcDepth into that slot; unrolled so slot, buffer and
    // sub-block are static, and branch-free so the loads' waits are exact (stages past the end
    // are junk that no consumer reads). Writing the first stage of a super-block moves the
    // header ring on by one.
    static_assert(kPcPUnroll % 8 == 0 && kPcPUnroll % kPcDepth == 0 && kPcPUnroll % kPcBufs == 0,
                  "static ring slots, LDS buffers and sub-blocks");
    for (uint32_t i0 = 0; i0 < n_pad; i0 += kPcPUnroll) {
#pragma unroll
        for (int q = 0; q < kPcPUnroll; ++q) {
            const int k = (q + 2) % kPcDepth;
            if ((q + 2) % 8 == 0) {
#pragma unroll
                for (int e = 0; e + 1 < NH; ++e) H[e] = H[e + 1];
            }
            store(k, (q + 2) % 8, (q + 2) % kPcBufs);
            load(k, s_begin + i0 + q + 2 + kPcDepth, (q + 2 + kPcDepth) % 8 == 0, NH - 1);
            pc_sync();  // B_{i+1}
            // keep each stage's work between its barriers: hoisting a later stage's decode would
            // make it wait for that stage's loads
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if constexpr (KH) {  // the consumers' two barriers around the meeting of the K halves
        pc_sync();
        pc_sync();
    }
}

// Sum of the K-chunk partials of a split launch (in chunk order) and the epilogue.
// grid = (tiles * BM * 128 / 256), block 256; one output element (pair) per thread.
// With one M tile the grid covers only its n_vec rows (reduce_rows).
__host__ __device__ inline uint32_t reduce_rows(uint32_t bm, uint32_t m_tiles, uint32_t n_vec) {
    return m_tiles == 1 && n_vec < bm ? n_vec : bm;
}

template <uint32_t T, bool PAIR, int MB>
__global__ __launch_bounds__(512) void k_gemm_pc(GemmPcArgs a) {
    __shared__ __bf16 lds[kPcBufs * kPcStage];
    gemm_pc_body<T, PAIR, MB>(a, blockIdx.x, lds);
}

// One thread: four consecutive output columns of one row (16-byte partial loads; the loads of
// four chunks are issued before their additions, which stay in chunk order per output).
template <bool PAIR, int BM>
__device__ __forceinline__ void pc_reduce_elem(const GemmPcArgs& a, uint64_t idx) {
    constexpr uint32_t NC = PAIR ? 64 : kPcW;  // output columns per tile
    constexpr uint32_t NQ = NC / 4;            // four-column groups per tile row
    const uint64_t tiles = (uint64_t)a.split_units * a.m_tiles;
    const uint32_t R = reduce_rows(BM, a.m_tiles, a.n_vec);
    if (idx >= tiles * R * NQ) return;
    const uint32_t tile = (uint32_t)(idx / (R * NQ)), e = (uint32_t)(idx % (R * NQ));
    const uint32_t ml = e / NQ, nl = 4 * (e % NQ);
    const uint32_t u = a.split_unit0 + tile / a.m_tiles, mt = tile % a.m_tiles;
    const uint32_t m = mt * BM + ml;
    if (m >= a.n_vec) return;
    const float* P = a.partials + (uint64_t)tile * a.kchunks * BM * kPcW + ml * kPcW + nl;
    constexpr uint64_t CS = (uint64_t)BM * kPcW;  // floats per chunk
    float4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
    auto add = [](float4& s, const float4 v) {
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
    };
    uint32_t c = 0;
    for (; c + 4 <= a.kchunks; c += 4) {
        float4 q0[4], q1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q0[i] = *reinterpret_cast<const float4*>(P + (c + i) * CS);
            if constexpr (PAIR) q1[i] = *reinterpret_cast<const float4*>(P + (c + i) * CS + 64);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            add(s0, q0[i]);
            if constexpr (PAIR) add(s1, q1[i]);
        }
    }
    for (; c < a.kchunks; ++c) {
        add(s0, *reinterpret_cast<const float4*>(P + c * CS));
        if constexpr (PAIR) add(s1, *reinterpret_cast<const float4*>(P + c * CS + 64));
    }
    float* yrow = a.y + (uint64_t)m * a.y_stride;
    const float g[4] = {s0.x, s0.y, s0.z, s0.w}, up[4] = {s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (PAIR) {
            const uint32_t col = u * kSlabRows + nl + i;
            if (col < a.rows) yrow[col] = silu_fast(g[i]) * up[i];
        } else {
            const uint32_t col = 2 * u * kSlabRows + nl + i;
            if (col < a.rows) yrow[col] = g[i];
        }
    }
}

template <bool PAIR, int BM>
__global__ void k_gemm_pc_reduce(GemmPcArgs a) {
    pc_reduce_elem<PAIR, BM>(a, (uint64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// ---- grouped bf16 GEMM (halo_mi_gemm_group): SLAB matrices sharing x ----------------------
// The x rows are staged once; the segments' tiles (all whole, or all split over the same K
// chunks) form one launch per pair of weight types, each workgroup running the k_gemm_pc body of
// its segment's type; split tiles are reduced by one launch over all segments.
struct GemmGroupArgs {
    GemmPcArgs seg[HALO_MI_GEMV_GROUP_MAX];
    uint32_t type[HALO_MI_GEMV_GROUP_MAX];
    uint32_t wg_end[HALO_MI_GEMV_GROUP_MAX];   // workgroups of segments [0, i]
    uint64_t out_end[HALO_MI_GEMV_GROUP_MAX];  // reduce threads (four columns each) of segments [0, i]
    uint32_t n;
};

template <uint32_t TA, uint32_t TB, int MB>
__global__ __launch_bounds__(512) void k_gemm_pc_group(GemmGroupArgs g) {
    __shared__ __bf16 lds[kPcBufs * kPcStage];
    uint32_t s = 0;
    while (s + 1 < g.n && blockIdx.x >= g.wg_end[s]) ++s;
    const uint32_t bid = blockIdx.x - (s ? g.wg_end[s - 1] : 0u);
    if (g.type[s] == TA) {
        gemm_pc_body<TA, false, MB>(g.seg[s], bid, lds);
    } else {
        if constexpr (TB != TA) gemm_pc_body<TB, false, MB>(g.seg[s], bid, lds);
    }
}

template <int BM>
__global__ void k_gemm_pc_reduce_group(GemmGroupArgs g) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t s = 0;
    while (s + 1 < g.n && idx >= g.out_end[s]) ++s;
    pc_reduce_elem<false, BM>(g.seg[s], idx - (s ? g.out_end[s - 1] : 0ull));
}

// ------------------------------------------------------------------------------------------
// Large-M GEMM: k_gemm_lm<T, PAIR> (M > 256)
//
// A workgroup owns a 512 x 128 tile: the 512 x rows of one M tile times 128 W rows (PAIR: the
// 64 gate rows of slab u, then the 64 up rows of the same slab; else slabs 2u and 2u + 1).
// Four waves, each of which both dequantizes and multiplies. With no producer waves a wave can
// hold 256 fp32 accumulators, twice k_gemm_pc's, which halves the LDS bytes and the barriers
// per MFMA:
//   - wave w dequantizes W-tile rows [32 w, 32 w + 32) of every stage (lane: row 32 w + lane % 32,
//     half lane / 32 of the slot record) with pc_dequant, rounds to bf16 and writes them to LDS
//     (three buffers of one stage each);
//   - wave w multiplies x rows [128 w, 128 w + 128) (4 blocks of 32; fragments straight from the
//     fragment-ordered staging buffer) by all 128 W rows (4 blocks of 32, from LDS): 16 32x32
//     accumulators, 32 v_mfma_f32_32x32x16_bf16 per stage.
// Per stage the LDS carries 8 KB of writes and 32 KB of reads for 128 MFMAs, one barrier.
//
// Iteration i (stage i of this workgroup's range; LDS buffer i % 3 holds stage i, x ring slot
// i % 2 its x fragments; stage i's W fragments are already in registers):
//   region A: the first K half's MFMAs, with stage i + 1's W fragments read from LDS (written
//     in iteration i - 1, complete since the barrier that ended it), stage i + 2 dequantized
//     (its records were loaded four iterations ago) and that half's x fragments reloaded with
//     stage i + 2 in between;
//   region B: the second K half's MFMAs, with stage i + 2 written to buffer (i + 2) % 3, the
//     second half's x fragments reloaded and stage i + 6's records loaded into the freed ring
//     slot in between; then the barrier (after this wave's LDS accesses complete).
// Buffer (i + 2) % 3 was last read in iteration i - 2, which every wave finished before the
// barrier that ended it. The next stage's first MFMAs need nothing from LDS, so the barrier's
// latency and the LDS round trip overlap the MFMA pipe. Both regions interleave the other
// instructions between the MFMAs (sched_group_barrier), so the dequantization's VALU work
// co-issues with the matrix core. Stages past the end read zeros (out-of-range buffer loads),
// so the loop is branch-free and padded stages add exactly 0.
// ------------------------------------------------------------------------------------------
constexpr int kLmBM = 512;    // x rows per tile (MBW = 4)
constexpr int kLmWDepth = 4;  // stages of W records in flight per wave
constexpr uint32_t kLmMinRows = 256;  // x rows above which the GEMM takes k_gemm_lm

// MBW: 32-row x blocks per wave, so the tile has 128 MBW x rows. 4 for the main tiles; 1 for
// the K-split tiles that spread a launch's last partial round over the GPU (a quarter of the
// rows per tile, so four times the tiles, and a quarter of the partial sums per chunk).
template <uint32_t T, bool PAIR, int MBW>
__global__ __launch_bounds__(256) void k_gemm_lm(GemmPcArgs a) {
    constexpr uint32_t BM = 128 * MBW;
    constexpr uint32_t STAGE = kPcW * kPcLd;  // bf16 per LDS stage
    __shared__ __bf16 lds[3 * STAGE];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t S = a.cols / kSlot;
    const SlabGeom g = slab_geom(T, a.cols);
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;

    // workgroup -> (W tile u, M tile mt) for a whole tile, or (split tile st, K chunk)
    const uint32_t whole = a.units * a.m_tiles;
    const bool split = blockIdx.x >= whole;
    uint32_t u, mt, st = 0, chunk = 0;
    if (!split) {
        u = blockIdx.x / a.m_tiles;
        mt = blockIdx.x % a.m_tiles;
    } else {
        st = (blockIdx.x - whole) / a.kchunks;
        chunk = (blockIdx.x - whole) % a.kchunks;
        u = a.split_unit0 + st / a.m_tiles;
        mt = st % a.m_tiles;
    }
    uint32_t s_begin = 0, s_end = S;
    if (split) {
        const uint32_t ng = S / 8, base = ng / a.kchunks, extra = ng % a.kchunks;
        const uint32_t g0 = chunk * base + min(chunk, extra);
        s_begin = 8 * g0;
        s_end = 8 * (g0 + base + (chunk < extra ? 1u : 0u));
    }
    const uint32_t n_pad = (s_end - s_begin + kPcUnroll - 1) / kPcUnroll * kPcUnroll;

    // ---- dequantization role: W-tile rows [32 wave, 32 wave + 32) ----
    const uint32_t r = lane & 31u, h = lane >> 5;
    const uint32_t mat = wave >> 1, srow = 32 * (wave & 1u) + r;
    const uint8_t* slab_ptr;
    if constexpr (PAIR) {
        slab_ptr = (mat ? a.w1 : a.w0) + (uint64_t)u * g.slab_bytes;
    } else {
        // a missing second slab reads the last one again: its outputs are never stored
        slab_ptr = a.w0 + (uint64_t)min(2 * u + mat, slabs - 1) * g.slab_bytes;
    }
    const __amdgpu_buffer_rsrc_t wres = make_rsrc(slab_ptr, (uint32_t)g.slab_bytes);
    const PcOff off = pc_offsets<T>(srow, h);
    const float inv_unit = __uint_as_float(0x7F000000u - __float_as_uint(fp8_unit()));
    const uint32_t wdst = (32 * wave + r) * kPcLd + 8 * h;
    // per-slot codes kLmWDepth stages ahead; the super-block fields once per super-block (Hc
    // serves the stages being dequantized, Hn is the next super-block's)
    PcW<T> R[kLmWDepth];
    SmH<T> Hc, Hn;
    auto load_w = [&](int slot, uint32_t s) { sm_load_q<T>(R[slot], wres, g, off, s, s < s_end); };
    auto dequant = [&](int slot, uint32_t j, bf16x8& lo, bf16x8& hi) {
        PcW<T> W = R[slot];
        sm_merge<T>(W, Hc, j);
        pc_dequant<T>(W, h, j, inv_unit, lo, hi);
    };
    auto store_w = [&](int slot, uint32_t j, int buf) {
        bf16x8 lo, hi;
        dequant(slot, j, lo, hi);
        __bf16* dst = lds + buf * STAGE + wdst;
        *reinterpret_cast<bf16x8*>(dst) = lo;
        *reinterpret_cast<bf16x8*>(dst + 16) = hi;
    };

    // ---- multiply role: x rows [32 MBW wave, 32 MBW (wave + 1)) x all 128 W rows ----
    floatx16 acc[MBW][4];
#pragma unroll
    for (int i = 0; i < MBW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{};
    const uint32_t lr = lane & 31u;
    const uint32_t boff = lr * kPcLd + 8 * (lane >> 5);  // + 32 j rows, + 16 for the second K half
    const uint32_t m0 = mt * BM;
    const __amdgpu_buffer_rsrc_t xres = make_rsrc(a.xf + (uint64_t)m0 * a.cols, (uint32_t)((uint64_t)BM * a.cols * 2));
    const uint32_t xlane = lane * 16;
    uint4 A[2][2][MBW];  // [ring slot][K half][x block]
    auto load_a = [&](int slot, int k, uint32_t s) {
#pragma unroll
        for (int i = 0; i < MBW; ++i)
            A[slot][k][i] = bld128(xres, xlane, s < s_end ? (((MBW * wave + i) * S + s) * 2 + k) * 1024 : kPcOob);
    };
    auto mma = [&](int slot, int k, const bf16x8 (&B)[4]) {
#pragma unroll
        for (int i = 0; i < MBW; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, A[slot][k][i]), B[j],
                                                                    acc[i][j], 0, 0, 0);
    };
    auto read_b = [&](uint32_t buf, bf16x8 (&B)[2][4]) {
        const __bf16* Lb = lds + buf * STAGE + boff;
#pragma unroll
        for (int j = 0; j < 4; ++j) B[0][j] = *reinterpret_cast<const bf16x8*>(Lb + 32 * j * kPcLd);
#pragma unroll
        for (int j = 0; j < 4; ++j) B[1][j] = *reinterpret_cast<const bf16x8*>(Lb + 32 * j * kPcLd + 16);
    };

    // prologue: W records of stages 0..3; stages 0 and 1 dequantized into LDS buffers 0 and 1;
    // x of stages 0 and 1; stage 0's W fragments
    static_assert(kPcUnroll == 8 && kLmWDepth == 4, "one super-block per unrolled iteration");
    sm_load_h<T>(Hc, wres, g, off, s_begin / 8, s_begin < s_end);
#pragma unroll
    for (int p = 0; p < kLmWDepth; ++p) load_w(p, s_begin + p);
    load_a(0, 0, s_begin);
    load_a(0, 1, s_begin);
    load_a(1, 0, s_begin + 1);
    load_a(1, 1, s_begin + 1);
    store_w(0, 0, 0);
    store_w(1, 1, 1);
    load_w(0, s_begin + kLmWDepth);
    load_w(1, s_begin + kLmWDepth + 1);
    pc_sync();
    bf16x8 Bc[2][4];  // W fragments of the current stage: [K half][W block]
    read_b(0, Bc);
    uint32_t bufc = 0;  // LDS buffer of the current stage (stage i in buffer i % 3)
    for (uint32_t i0 = 0; i0 < n_pad; i0 += kPcUnroll) {
#pragma unroll
        for (int q = 0; q < kPcUnroll; ++q) {
            const int xb = q & 1, ws = (q + 2) % kLmWDepth;
            const uint32_t bufn = bufc == 2 ? 0u : bufc + 1, bufw = bufn == 2 ? 0u : bufn + 1;
            bf16x8 Bn[2][4];
            // Region A: the first K half's 16 MFMAs (distinct accumulators, any order) with the
            // next stage's W fragments read in between and stage i + 2 dequantized in between.
            mma(xb, 0, Bc[0]);
            read_b(bufn, Bn);
            bf16x8 lo, hi;
            if (q == 6) Hc = Hn;  // stage i + 2 starts the next super-block
            dequant(ws, (q + 2) % 8, lo, hi);
            load_a(xb, 0, s_begin + i0 + q + 2);
            if constexpr (MBW == 4) {  // with fewer MFMAs the VALU work dominates: no pattern
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // one MFMA
                    if (k < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      // a DS read
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);                 // up to 5 VALU
                    if (k >= 12) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // a VMEM read
                }
            }
            // Both K halves update every accumulator: a region boundary keeps each pair 16 MFMAs
            // apart (the scheduler would otherwise issue a dependent pair back to back).
            __builtin_amdgcn_sched_barrier(0);
            // Region B: the second K half's MFMAs with the LDS writes of stage i + 2 and the loads
            // of stage i + 2's x fragments and stage i + 6's W records in between.
            mma(xb, 1, Bc[1]);
            __bf16* dst = lds + bufw * STAGE + wdst;
            *reinterpret_cast<bf16x8*>(dst) = lo;
            *reinterpret_cast<bf16x8*>(dst + 16) = hi;
            // x before W: vmcnt counts in order, so the wait for these x fragments (two stages
            // on) then covers only W records issued a stage earlier, which have come from HBM
            load_a(xb, 1, s_begin + i0 + q + 2);
            const uint32_t sl = s_begin + i0 + q + 2 + kLmWDepth;
            load_w(ws, sl);
            if (q == 2) sm_load_h<T>(Hn, wres, g, off, sl / 8, sl < s_end);  // the next super-block
            if constexpr (MBW == 4) {
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // one MFMA
                    if (k < 2) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);      // a DS write
                    if (k >= 2 && k < 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a VMEM read
                }
            }
            pc_sync();
            // keep each stage's work between its barriers: hoisting a later stage's decode would
            // make it wait for that stage's loads (and with them every load in flight)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) Bc[k][j] = Bn[k][j];
            bufc = bufn;
        }
    }

    if (split) {
        // fp32 partial tile [BM][128] of this chunk
        float* P = a.partials + ((uint64_t)st * a.kchunks + chunk) * BM * kPcW;
#pragma unroll
        for (int i = 0; i < MBW; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t ml = 32 * (MBW * wave + i) + mfma32_row(e, lane);
#pragma unroll
                for (int j = 0; j < 4; ++j) P[ml * kPcW + 32 * j + lr] = acc[i][j][e];
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MBW; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t m = m0 + 32 * (MBW * wave + i) + mfma32_row(e, lane);
            if (m >= a.n_vec) continue;
            float* yrow = a.y + (uint64_t)m * a.y_stride;
            if constexpr (PAIR) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t col = u * kSlabRows + 32 * j + lr;
                    if (col < a.rows) yrow[col] = silu_fast(acc[i][j][e]) * acc[i][j + 2][e];
                }
                // one row of outputs at a time: interleaving the SiLUs of many rows would need
                // more VGPRs than the accumulators leave
                __builtin_amdgcn_sched_barrier(0);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t col = 2 * u * kSlabRows + 32 * j + lr;
                    if (col < a.rows) yrow[col] = acc[i][j][e];
                }
            }
        }
}

// ------------------------------------------------------------------------------------------
// Small-M GEMM: k_gemm_sm<T, PAIR, XR> (at most 32 x rows; XR = 8, 12, 16, 24 or 32 rows kept)
//
// A workgroup owns W unit u (PAIR: the gate and up rows of slab u; else slabs 2u and 2u + 1)
// over K chunk `chunk` (whole super-blocks) and all x rows. Wave w takes matrix w / 2 and row
// block w % 2 (32 W rows). Lane l dequantizes row l % 32, half l / 32 of each slot record,
// which is exactly its B operand of v_mfma_f32_32x32x16_bf16 for the slot's two K halves: no
// W through LDS, no barrier in the loop. What the vector-memory path carries per slot is only
// the weights themselves:
//   - x: the chunk's x fragments (rows < XR of the staged buffer) are copied into LDS once, at
//     the start; each slot's A operands are then two ds_read_b128 (lanes of rows past XR read
//     row XR - 1's entry: an A row feeds only its own output row, and rows past the x rows are
//     never stored, so no zero entry is kept and a 5-group chunk at XR = 16 takes exactly 40 KB,
//     four workgroups per CU). Loading them from global memory per wave and slot took 2 KB of L1 traffic per
//     64 x 32 weights and kept the texture path busy three quarters of the kernel;
//   - the block headers (Q4_K / Q5_K scales and mins, IQ4_XS scales, Q6_K's scales and d) are
//     loaded once per super-block, two ahead, not once per slot;
//   - the per-slot codes stream kSmAhead slots ahead (a ring of 8: the kernel then fits five
//     workgroups per CU, so the M = 8 gate/up launch of 4 K chunks x 272 units runs in one round).
// Each wave writes its 32 x 32 partial to partials[(u * kchunks + chunk)][32][128] (columns 64 *
// matrix + 32 * block), and k_gemm_pc_reduce adds the chunks in order and applies the epilogue.
// ------------------------------------------------------------------------------------------
constexpr int kSmDepth = 16;  // slots per loop iteration (two super-blocks)
constexpr int kSmAhead = 8;   // slots of weight codes in flight per wave (a ring; divides kSmDepth)
constexpr uint32_t kSmRows = 32;  // x rows of the small-M GEMM (one MFMA block)
constexpr uint32_t kSmLdsMax = 48 * 1024;  // x bytes of one workgroup's K chunk in LDS
constexpr uint32_t kSmLdsMax8 = 24 * 1024;  // the same at 8 rows, read from fp32 x by the kernel
// 24 rows: 40 KB, so 3-group chunks of 36 KB and four workgroups per CU (32 rows: 48 KB, three)
__host__ __device__ constexpr uint32_t sm_lds_max(uint32_t xr) { return xr == 8 ? kSmLdsMax8 : xr == 24 ? 40u * 1024 : kSmLdsMax; }

// x bytes in LDS per slot of K: two K halves x two lane halves x XR rows x 16 B.
__host__ __device__ constexpr uint32_t sm_x_bytes_per_slot(uint32_t xr) { return 64u * xr; }

template <uint32_t T, bool PAIR, uint32_t XR>
__global__ __launch_bounds__(256, 3) void k_gemm_sm(GemmPcArgs a) {
    extern __shared__ uint4 xl[];  // [slot][K half][lane half][XR rows]
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t S = a.cols / kSlot;
    const SlabGeom g = slab_geom(T, a.cols);
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    const uint32_t u = blockIdx.x / a.kchunks, chunk = blockIdx.x % a.kchunks;
    const uint32_t ng = S / 8, base = ng / a.kchunks, extra = ng % a.kchunks;
    const uint32_t g0 = chunk * base + min(chunk, extra);
    const uint32_t s_begin = 8 * g0, s_end = 8 * (g0 + base + (chunk < extra ? 1u : 0u));
    const uint32_t ns = s_end - s_begin;
    const uint32_t mat = wave >> 1, rb = wave & 1u;
    const uint32_t r = lane & 31u, h = lane >> 5;
    const uint8_t* slab_ptr;
    if constexpr (PAIR) {
        slab_ptr = (mat ? a.w1 : a.w0) + (uint64_t)u * g.slab_bytes;
    } else {
        // a missing second slab reads the last one again: its outputs are never stored
        slab_ptr = a.w0 + (uint64_t)min(2 * u + mat, slabs - 1) * g.slab_bytes;
    }
    const __amdgpu_buffer_rsrc_t wres = make_rsrc(slab_ptr, (uint32_t)g.slab_bytes);
    const PcOff off = pc_offsets<T>(32 * rb + r, h);
    const float inv_unit = __uint_as_float(0x7F000000u - __float_as_uint(fp8_unit()));

    // x of the chunk into LDS: the loads first, then the weight stream's first loads, then the
    // LDS stores (which wait only for the x loads: loads return in order). At 8 rows the kernel
    // reads fp32 x itself and rounds it to bf16 (RNE) as k_x_to_frag does, so no staging launch
    // runs; above, the staged fragments are copied.
    constexpr bool kFuseX = XR == 8;
    constexpr uint32_t kXPer = sm_lds_max(XR) / 16 / 256;  // 16-byte entries per thread: the largest chunk's
    const uint32_t n16 = ns * 4 * XR;
    PcW<T> R[kSmAhead];
    SmH<T> H[2];
    auto load_q = [&](int q, uint32_t s) { sm_load_q<T>(R[q], wres, g, off, s, s < s_end); };
    auto load_h = [&](int i, uint32_t sb) { sm_load_h<T>(H[i], wres, g, off, sb, 8 * sb < s_end); };
    if constexpr (kFuseX) {
        float4 xa[kXPer], xb[kXPer];
#pragma unroll
        for (int i = 0; i < (int)kXPer; ++i) {
            const uint32_t e = threadIdx.x + 256u * i;
            const uint32_t row = e % 8, k8 = (e / 8) & 1u, hk = e / 16;  // hk = 2 (slot - s_begin) + K half
            const uint32_t k = 32 * (s_begin + hk / 2) + 16 * (hk & 1u) + 8 * k8;
            xa[i] = xb[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
            if (e < n16 && row < a.n_vec) {
                const float* xp = a.x + (uint64_t)row * a.x_stride + k;
                xa[i] = *reinterpret_cast<const float4*>(xp);
                xb[i] = *reinterpret_cast<const float4*>(xp + 4);
            }
        }
        load_h(0, s_begin / 8);
        load_h(1, s_begin / 8 + 1);
#pragma unroll
        for (int q = 0; q < kSmAhead; ++q) load_q(q, s_begin + q);
#pragma unroll
        for (int i = 0; i < (int)kXPer; ++i) {
            const uint32_t e = threadIdx.x + 256u * i;
            if (e >= n16) break;
            float v[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
            const uint32_t row = e % 8;
            if (a.nw && row < a.n_vec) {
#pragma clang fp contract(off)
                const uint32_t k8 = (e / 8) & 1u, hk = e / 16;
                const uint32_t k = 32 * (s_begin + hk / 2) + 16 * (hk & 1u) + 8 * k8;
                const float sc = a.inv[row];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float t = v[j] * sc;
                    v[j] = t * a.nw[k + j];
                }
            }
            const bf16x8 b{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3],
                           (__bf16)v[4], (__bf16)v[5], (__bf16)v[6], (__bf16)v[7]};
            xl[e] = __builtin_bit_cast(uint4, b);
        }
    } else {
        const __amdgpu_buffer_rsrc_t xres = make_rsrc(a.xf, (uint32_t)((uint64_t)kSmRows * a.cols * 2));
        uint4 xv[kXPer];
#pragma unroll
        for (int i = 0; i < (int)kXPer; ++i) {
            const uint32_t e = threadIdx.x + 256u * i;
            const uint32_t row = e % XR, k8 = (e / XR) & 1u, hk = e / (2 * XR);  // hk = 2 (slot - s_begin) + K half
            // a per-lane condition goes in the lane offset: the scalar offset must stay uniform
            xv[i] = bld128(xres, e < n16 ? (s_begin * 2 + hk) * 1024 + (k8 * 32 + row) * 16 : kPcOob, 0);
        }
        load_h(0, s_begin / 8);
        load_h(1, s_begin / 8 + 1);
#pragma unroll
        for (int q = 0; q < kSmAhead; ++q) load_q(q, s_begin + q);
#pragma unroll
        for (int i = 0; i < (int)kXPer; ++i) {
            const uint32_t e = threadIdx.x + 256u * i;
            if (e < n16) xl[e] = xv[i];
        }
    }
    __syncthreads();

    // this lane's A entries: row r, lane half h; rows past XR read row XR - 1 (their output rows
    // are never stored)
    const uint32_t xrow = h * XR + min(r, XR - 1);
    floatx16 acc = floatx16{};
    auto step = [&](int q, uint32_t s) {
        PcW<T> W = R[q % kSmAhead];
        sm_merge<T>(W, H[q >> 3], q & 7);
        bf16x8 lo, hi;
        pc_dequant<T>(W, h, q & 7, inv_unit, lo, hi);  // s_begin: a multiple of 8
        const uint32_t ls = s - s_begin;
        const uint4 x0 = xl[(2 * ls) * 2 * XR + xrow];
        const uint4 x1 = xl[(2 * ls + 1) * 2 * XR + xrow];
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x0), lo, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x1), hi, acc, 0, 0, 0);
        load_q(q % kSmAhead, s + kSmAhead);
    };
    // two super-blocks per iteration: H[0] serves the first, H[1] the second; each is reloaded
    // with the super-block two ahead once its own is done
    for (uint32_t i0 = s_begin; i0 < s_end; i0 += kSmDepth) {
#pragma unroll
        for (int q = 0; q < 8; ++q) step(q, i0 + q);
        load_h(0, i0 / 8 + 2);
        if (i0 + 8 >= s_end) break;
#pragma unroll
        for (int q = 8; q < kSmDepth; ++q) step(q, i0 + q);
        load_h(1, i0 / 8 + 3);
    }
    float* P = a.partials + ((uint64_t)u * a.kchunks + chunk) * kSmRows * kPcW + 64 * mat + 32 * rb + r;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t m = mfma32_row(e, lane);
        if (m < a.n_vec) P[m * kPcW] = acc[e];  // the reduce reads only the rows of x
    }
}

template <bool PAIR, uint32_t XR>
void launch_gemm_sm_xr(uint32_t type, const GemmPcArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL((k_gemm_sm<kQ4_0, PAIR, XR>), grid, dim3(256), lds, st, a); break;
        case kQ8_0: hipLaunchKernelGGL((k_gemm_sm<kQ8_0, PAIR, XR>), grid, dim3(256), lds, st, a); break;
        case kQ4_K: hipLaunchKernelGGL((k_gemm_sm<kQ4_K, PAIR, XR>), grid, dim3(256), lds, st, a); break;
        case kQ5_K: hipLaunchKernelGGL((k_gemm_sm<kQ5_K, PAIR, XR>), grid, dim3(256), lds, st, a); break;
        case kIQ4_XS: hipLaunchKernelGGL((k_gemm_sm<kIQ4_XS, PAIR, XR>), grid, dim3(256), lds, st, a); break;
        default: hipLaunchKernelGGL((k_gemm_sm<kQ6_K, PAIR, XR>), grid, dim3(256), lds, st, a); break;
    }
}

template <bool PAIR, int MBW>
void launch_gemm_lm_type(uint32_t type, const GemmPcArgs& a, dim3 grid, hipStream_t st) {
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL((k_gemm_lm<kQ4_0, PAIR, MBW>), grid, dim3(256), 0, st, a); break;
        case kQ8_0: hipLaunchKernelGGL((k_gemm_lm<kQ8_0, PAIR, MBW>), grid, dim3(256), 0, st, a); break;
        case kQ4_K: hipLaunchKernelGGL((k_gemm_lm<kQ4_K, PAIR, MBW>), grid, dim3(256), 0, st, a); break;
        case kQ5_K: hipLaunchKernelGGL((k_gemm_lm<kQ5_K, PAIR, MBW>), grid, dim3(256), 0, st, a); break;
        case kIQ4_XS: hipLaunchKernelGGL((k_gemm_lm<kIQ4_XS, PAIR, MBW>), grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((k_gemm_lm<kQ6_K, PAIR, MBW>), grid, dim3(256), 0, st, a); break;
    }
}

template <bool PAIR, int MB>
void launch_gemm_pc_type(uint32_t type, const GemmPcArgs& a, dim3 grid, hipStream_t st) {
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL((k_gemm_pc<kQ4_0, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        case kQ8_0: hipLaunchKernelGGL((k_gemm_pc<kQ8_0, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        case kQ4_K: hipLaunchKernelGGL((k_gemm_pc<kQ4_K, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        case kQ5_K: hipLaunchKernelGGL((k_gemm_pc<kQ5_K, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        case kIQ4_XS: hipLaunchKernelGGL((k_gemm_pc<kIQ4_XS, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        default: hipLaunchKernelGGL((k_gemm_pc<kQ6_K, PAIR, MB>), grid, dim3(512), 0, st, a); break;
    }
}

// k_gemm_pc_reduce over the split tiles of p (BM-row tiles)
template <bool PAIR, int BM>
void launch_reduce(const GemmPcArgs& p, hipStream_t st) {
    // threads: four output columns each
    const uint64_t outs = (uint64_t)p.split_units * p.m_tiles * reduce_rows(BM, p.m_tiles, p.n_vec) * (PAIR ? 64 : kPcW) / 4;
    hipLaunchKernelGGL((k_gemm_pc_reduce<PAIR, BM>), dim3((uint32_t)((outs + 255) / 256)), dim3(256), 0, st, p);
}

// Rows [m_start, m_start + mc) of x to bf16 fragments, zero-padded to m_pad rows; with the
// fused norm, each row's 1 / rms first (k_rms_inv_rows into ws->inv).
int stage_x(const GemmArgs& a, uint64_t m_start, uint32_t mc, uint32_t m_pad, Workspace* ws, hipStream_t st) {
    const float* x = a.x + m_start * a.x_stride;
    if (a.norm_w)
        if (int rc = launch_rms_inv(x, a.x_stride, mc, a.cols, a.norm_eps, ws->inv, st)) return rc;
    const uint64_t n8 = (uint64_t)m_pad * (a.cols / 8);
    hipLaunchKernelGGL(k_x_to_frag, dim3((uint32_t)((n8 + 255) / 256)), dim3(256), 0, st, x, a.x_stride, mc, m_pad,
                       a.cols, ws->xb, ws->inv, a.norm_w);
    return hip_status(hipGetLastError(), "x staging launch");
}

uint32_t cu_count() {
    static const uint32_t cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return (uint32_t)std::max(n, 1);
    }();
    return cus;
}

// The k_gemm_lm path. Whole rounds of 512-row tiles; the W tiles past the last whole round run
// as 128-row tiles split over K (four times the tiles of a 512-row tile and a quarter of the
// partial sums per chunk), so the partial round is spread over the GPU; k_gemm_pc_reduce adds
// their partials in chunk order. With fewer 512-row tiles than CUs, those are split over K.
template <bool PAIR>
int launch_gemm_lm(uint32_t type, const GemmArgs& a, Workspace* ws, uint32_t units, hipStream_t st) {
    const uint32_t S = a.cols / kSlot, cus = cu_count();
    const uint64_t cap_rows = std::min(kXbElems / a.cols, kInvFloats) / kLmBM * kLmBM;
    if (cap_rows == 0) return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for the x staging buffer", a.cols);
    if ((uint64_t)kLmBM * a.cols * 2 > 0xFFFFFFFFull)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for one M tile", a.cols);
    for (uint64_t m_start = 0; m_start < a.n_vec; m_start += cap_rows) {
        const uint32_t mc = (uint32_t)std::min<uint64_t>(cap_rows, a.n_vec - m_start);
        const uint32_t m_tiles = (mc + kLmBM - 1) / kLmBM;
        if (int rc = stage_x(a, m_start, mc, m_tiles * kLmBM, ws, st)) return rc;
        const uint64_t tiles = (uint64_t)units * m_tiles;
        GemmPcArgs p{a.w0, a.w1, ws->xb, a.y + m_start * a.y_stride, a.y_stride, a.rows, a.cols, mc, units, m_tiles, 0u,
                     0u, 1u, ws->partials};
        if (tiles >= cus) {
            uint32_t main_units = (uint32_t)(tiles / cus * cus / m_tiles), rest = units - main_units, kc = 0;
            const uint32_t mt_t = (mc + 127) / 128;
            if (rest > 0 && S % 8 == 0) {
                const uint64_t tt = (uint64_t)rest * mt_t;
                kc = (uint32_t)std::min<uint64_t>({std::max<uint64_t>(cus / tt, 1), S / 8, 16});
                while (kc > 1 && tt * kc * 128 * kPcW > kPartialFloats) --kc;
                if (tt * kc * 128 * kPcW > kPartialFloats) kc = 0;  // partials do not fit: run them whole
            }
            if (rest > 0 && kc == 0) main_units = units, rest = 0;
            p.units = main_units;
            launch_gemm_lm_type<PAIR, 4>(type, p, dim3(main_units * m_tiles), st);
            if (rest > 0) {
                GemmPcArgs t = p;
                t.units = 0;
                t.m_tiles = mt_t;
                t.split_units = rest;
                t.kchunks = kc;
                t.split_unit0 = main_units;
                launch_gemm_lm_type<PAIR, 1>(type, t, dim3(rest * mt_t * kc), st);
                launch_reduce<PAIR, 128>(t, st);
            }
        } else {
            uint32_t kc = S % 8 == 0 ? (uint32_t)std::min<uint64_t>({cus / tiles, S / 8, 16}) : 1u;
            while (kc > 1 && tiles * kc * kLmBM * kPcW > kPartialFloats) --kc;
            if (kc >= 2) {
                p.units = 0;
                p.split_units = units;
                p.kchunks = kc;
                launch_gemm_lm_type<PAIR, 4>(type, p, dim3((uint32_t)(tiles * kc)), st);
                launch_reduce<PAIR, kLmBM>(p, st);
            } else {
                launch_gemm_lm_type<PAIR, 4>(type, p, dim3((uint32_t)tiles), st);
            }
        }
        if (int rc = hip_status(hipGetLastError(), "gemm_lm launch")) return rc;
    }
    return HALO_MI_OK;
}

// The k_gemm_sm launch plan: the x rows kept (XR) and the K chunks per unit. About four
// workgroups per CU (four or five are resident at the kernel's registers), at least enough chunks that
// one chunk's x fits kSmLdsMax, and the partials within the workspace. False if none fits.
struct SmPlan {
    uint32_t xr, kc;
    size_t lds;
};
bool sm_plan(uint32_t units, uint32_t S, uint32_t n_vec, SmPlan& pl) {
    if (n_vec > kSmRows || S % 8 != 0 || S == 0) return false;
    const uint32_t ng = S / 8, cus = cu_count();
    // 12 rows: a 5-group chunk in 30 KB, so five workgroups per CU (16 rows: 40 KB, four)
    pl.xr = n_vec <= 8 ? 8u : n_vec <= 12 ? 12u : n_vec <= 16 ? 16u : n_vec <= 24 ? 24u : 32u;
    const uint32_t max_groups = sm_lds_max(pl.xr) / (8 * sm_x_bytes_per_slot(pl.xr));
    const uint32_t kc_min = (ng + max_groups - 1) / max_groups;
    pl.kc = std::clamp<uint32_t>((4 * cus + units - 1) / units, kc_min, ng);
    while (pl.kc > kc_min && (uint64_t)units * pl.kc * kSmRows * kPcW > kPartialFloats) --pl.kc;
    if ((uint64_t)units * pl.kc * kSmRows * kPcW > kPartialFloats) return false;
    const uint32_t groups = (ng + pl.kc - 1) / pl.kc;  // the largest chunk
    pl.lds = (size_t)groups * 8 * sm_x_bytes_per_slot(pl.xr);
    return true;
}

// The k_gemm_sm path (at most 32 x rows, K in whole super-blocks): x staged as one 32-row
// block, every unit split over K (sm_plan), then the chunk-order reduce.
template <bool PAIR>
int launch_gemm_sm(uint32_t type, const GemmArgs& a, Workspace* ws, uint32_t units, hipStream_t st) {
    const uint32_t S = a.cols / kSlot;
    if ((uint64_t)kSmRows * a.cols > kXbElems || (uint64_t)kSmRows * a.cols * 2 > 0xFFFFFFFFull)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for the x staging buffer", a.cols);
    SmPlan pl;
    if (!sm_plan(units, S, a.n_vec, pl))
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: %u rows exceed the small-M partials workspace", a.rows);
    GemmPcArgs p{a.w0, a.w1, ws->xb, a.y, a.y_stride, a.rows, a.cols, a.n_vec, 0u, 1u, 0u, units, pl.kc, ws->partials};
    p.split_unit0 = 0;
    if (pl.xr == 8) {  // the kernel reads x itself; with the norm, 1 / rms per row first
        p.x = a.x;
        p.x_stride = a.x_stride;
        p.nw = a.norm_w;
        p.inv = ws->inv;
        if (a.norm_w)
            if (int rc = launch_rms_inv(a.x, a.x_stride, a.n_vec, a.cols, a.norm_eps, ws->inv, st)) return rc;
    } else if (int rc = stage_x(a, 0, a.n_vec, kSmRows, ws, st)) {
        return rc;
    }
    const dim3 grid(units * pl.kc);
    switch (pl.xr) {
        case 8: launch_gemm_sm_xr<PAIR, 8>(type, p, grid, pl.lds, st); break;
        case 12: launch_gemm_sm_xr<PAIR, 12>(type, p, grid, pl.lds, st); break;
        case 16: launch_gemm_sm_xr<PAIR, 16>(type, p, grid, pl.lds, st); break;
        case 24: launch_gemm_sm_xr<PAIR, 24>(type, p, grid, pl.lds, st); break;
        default: launch_gemm_sm_xr<PAIR, 32>(type, p, grid, pl.lds, st); break;
    }
    launch_reduce<PAIR, kSmRows>(p, st);
    return hip_status(hipGetLastError(), "gemm_sm launch");
}

}  // namespace

// x -> bf16 staging (in chunks of rows that fit the workspace), then the GEMM: k_gemm_sm for at
// most 32 x rows and k_gemm_lm for large M when the variant leaves the choice to the shape
// (launch_gemm_sm, launch_gemm_lm), else the producer/consumer k_gemm_pc. When k_gemm_pc's tiles do not
// fill whole rounds of the chip (e.g. 272 slabs on 256 CUs), the tiles past the last whole round
// are split over K so that the last round is spread over all CUs: their fp32 partials go to the
// workspace and k_gemm_pc_reduce adds them in a fixed order.
template <bool PAIR>
int launch_gemm_pc(uint32_t type, const GemmArgs& a, hipStream_t st) {
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    if (!ws)
        return set_error(HALO_MI_E_MEMORY, "gemm: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    const int MB = a.n_vec <= 64 ? 1 : a.n_vec <= 128 ? 2 : 4;
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    const uint32_t units = PAIR ? slabs : (slabs + 1) / 2;
    if (a.tiles == kGemmTilesSx || a.tiles == kGemmTilesSxFixed) return launch_gemm_sx(type, PAIR, a, ws, units, st);
    const uint32_t S = a.cols / kSlot, cus = cu_count();
    // k_gemm_lm (512-row M tiles) when its tiles alone fill the GPU; with fewer, the smaller
    // tiles of k_gemm_pc spread the work over more CUs
    if (a.tiles == kGemmTilesLm || (a.tiles == kGemmTilesAuto && a.n_vec > kLmMinRows &&
                                    (uint64_t)units * ((a.n_vec + kLmBM - 1) / kLmBM) >= cus))
        return launch_gemm_lm<PAIR>(type, a, ws, units, st);
    // the small-M kernel: about 1.5x k_gemm_pc's rate at M = 8 (no per-stage barrier chain)
    SmPlan sm_pl;
    const bool sm_fits = sm_plan(units, S, a.n_vec, sm_pl);
    if (a.tiles == kGemmTilesSm && !sm_fits)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: the small-M kernel takes at most %u x rows, cols a multiple of "
                                                "256 and at most %llu rows", kSmRows,
                         (unsigned long long)(kPartialFloats / (kSmRows * kPcW) * (PAIR ? 64 : 128)));
    if ((a.tiles == kGemmTilesAuto || a.tiles == kGemmTilesSm) && sm_fits)
        return launch_gemm_sm<PAIR>(type, a, ws, units, st);
    const uint32_t BM = 64u * MB;
    const uint64_t cap_rows = std::min(kXbElems / a.cols, kInvFloats) / BM * BM;
    if (cap_rows == 0) return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for the x staging buffer", a.cols);
    if ((uint64_t)BM * a.cols * 2 > 0xFFFFFFFFull)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for one M tile", a.cols);
    auto launch = [&](const GemmPcArgs& p) {
        const dim3 grid(p.units * p.m_tiles + p.split_units * p.m_tiles * p.kchunks);
        switch (MB) {
            case 1: launch_gemm_pc_type<PAIR, 1>(type, p, grid, st); break;
            case 2: launch_gemm_pc_type<PAIR, 2>(type, p, grid, st); break;
            default: launch_gemm_pc_type<PAIR, 4>(type, p, grid, st); break;
        }
    };
    auto xcd_ok = [](uint32_t n_units, uint32_t m_tiles) {
        return (m_tiles <= 8 && 8 % m_tiles == 0 && ((uint64_t)n_units * m_tiles) % 8 == 0) ? 1u : 0u;
    };
    for (uint64_t m_start = 0; m_start < a.n_vec; m_start += cap_rows) {
        const uint32_t mc = (uint32_t)std::min<uint64_t>(cap_rows, a.n_vec - m_start);
        const uint32_t m_tiles = (mc + BM - 1) / BM;
        if (int rc = stage_x(a, m_start, mc, m_tiles * BM, ws, st)) return rc;
        float* y = a.y + m_start * a.y_stride;
        // whole rounds of tiles, then the rest split over K; a matrix whose tiles cannot fill
        // half the chip is split over K altogether
        const uint64_t tiles = (uint64_t)units * m_tiles;
        uint32_t main_units = units, kc = 1;
        if (S % 8 == 0 && ((tiles > cus && tiles % cus != 0) || 2 * tiles < cus)) {
            main_units = tiles > cus ? (uint32_t)(tiles / cus * cus / m_tiles) : 0u;
            const uint64_t rest = (uint64_t)(units - main_units) * m_tiles;
            // Tiles left over beside a whole round: 64-row tiles run two workgroups per CU, so
            // their chunks run beside the whole tiles and 2 chunks suffice (the fewer partials,
            // the shorter the reduce); larger tiles hold a CU alone, so their chunks run after
            // the round and 8 keep that tail short (measured on MI355X, gate/up 17408 x 5120:
            // M = 64 57.3 -> 49.0 us, M = 128 70.4 -> 68.4, M = 256 105.2 -> 102.5, against 16)
            const uint32_t cap = main_units == 0 ? 16u : (MB == 1 ? 2u : 8u);
            kc = (uint32_t)std::min<uint64_t>({cus / std::max<uint64_t>(rest, 1), S / 8, cap});
            while (kc > 1 && rest * kc * BM * kPcW > kPartialFloats) --kc;
            if (kc < 2) main_units = units;  // nothing to gain: one launch
        }
        // one launch: the whole tiles, then the split tiles' chunks (dispatched as CUs free up)
        GemmPcArgs p{a.w0, a.w1, ws->xb, y, a.y_stride, a.rows, a.cols, mc, main_units, m_tiles, 0u,
                     units - main_units, kc, ws->partials};
        p.split_unit0 = main_units;
        p.xcd_map = xcd_ok(main_units, m_tiles);
        launch(p);
        if (p.split_units > 0) {
            switch (MB) {
                case 1: launch_reduce<PAIR, 64>(p, st); break;
                case 2: launch_reduce<PAIR, 128>(p, st); break;
                default: launch_reduce<PAIR, 256>(p, st); break;
            }
        }
        if (int rc = hip_status(hipGetLastError(), "gemm_pc launch")) return rc;
    }
    return HALO_MI_OK;
}

template int launch_gemm_pc<false>(uint32_t, const GemmArgs&, hipStream_t);
template int launch_gemm_pc<true>(uint32_t, const GemmArgs&, hipStream_t);

namespace {

constexpr uint32_t kGroupGemmTypes[6] = {kQ4_0, kQ8_0, kQ4_K, kQ5_K, kQ6_K, kIQ4_XS};

int group_type_index(uint32_t t) {
    for (int i = 0; i < 6; ++i)
        if (kGroupGemmTypes[i] == t) return i;
    return -1;
}

template <int MB, int IA, int IB>
bool gemm_group_pair(uint32_t ta, uint32_t tb, const GemmGroupArgs& g, dim3 grid, hipStream_t st) {
    constexpr uint32_t TA = kGroupGemmTypes[IA], TB = kGroupGemmTypes[IB];
    if (ta != TA || tb != TB) return false;
    hipLaunchKernelGGL((k_gemm_pc_group<TA, TB, MB>), grid, dim3(512), 0, st, g);
    return true;
}

// (ta, tb) with ta's index <= tb's in kGroupGemmTypes
template <int MB>
bool gemm_group_types(uint32_t ta, uint32_t tb, const GemmGroupArgs& g, dim3 grid, hipStream_t st) {
#define HALO_MI_GPAIR(A, B) gemm_group_pair<MB, A, B>(ta, tb, g, grid, st)
    return HALO_MI_GPAIR(0, 0) || HALO_MI_GPAIR(0, 1) || HALO_MI_GPAIR(0, 2) || HALO_MI_GPAIR(0, 3) || HALO_MI_GPAIR(0, 4) ||
           HALO_MI_GPAIR(0, 5) || HALO_MI_GPAIR(1, 1) || HALO_MI_GPAIR(1, 2) || HALO_MI_GPAIR(1, 3) || HALO_MI_GPAIR(1, 4) ||
           HALO_MI_GPAIR(1, 5) || HALO_MI_GPAIR(2, 2) || HALO_MI_GPAIR(2, 3) || HALO_MI_GPAIR(2, 4) || HALO_MI_GPAIR(2, 5) ||
           HALO_MI_GPAIR(3, 3) || HALO_MI_GPAIR(3, 4) || HALO_MI_GPAIR(3, 5) || HALO_MI_GPAIR(4, 4) || HALO_MI_GPAIR(4, 5) ||
           HALO_MI_GPAIR(5, 5);
#undef HALO_MI_GPAIR
}

// One launch over the segments of weight types ta and tb on the staged rows (mc of them, m_tiles
// M tiles of 64 MB rows): whole tiles when they fill half the GPU or more (as k_gemm_pc's
// choice), else every tile split over the same K chunks into the workspace's partials, then one
// reduce over all of them. (Config 5's q|k|v at M = 512 is 128 whole tiles; two K chunks each
// plus the reduce measured 533.0 against 531.3 us for the whole layer, same box.)
template <int MB>
int gemm_group_launch(const GroupSeg* segs, uint32_t n, uint32_t ta, uint32_t tb, uint32_t cols, uint32_t mc, uint32_t m_tiles,
                      uint64_t m_start, Workspace* ws, hipStream_t st) {
    constexpr uint32_t BM = 64u * MB;
    const uint32_t S = cols / kSlot, cus = cu_count();
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < n; ++i) tiles += (uint64_t)(((segs[i].rows + kSlabRows - 1) / kSlabRows + 1) / 2) * m_tiles;
    if (tiles == 0) return HALO_MI_OK;
    uint32_t kc = 1;
    if (S % 8 == 0 && 2 * tiles < cus) {
        kc = (uint32_t)std::min<uint64_t>({cus / tiles, S / 8, 16});
        while (kc > 1 && tiles * kc * BM * kPcW > kPartialFloats) --kc;
    }
    GemmGroupArgs g{};
    g.n = n;
    uint32_t wg = 0;
    uint64_t outs = 0, poff = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t units = ((segs[i].rows + kSlabRows - 1) / kSlabRows + 1) / 2;
        GemmPcArgs p{static_cast<const uint8_t*>(segs[i].w), nullptr, ws->xb, segs[i].y + m_start * segs[i].y_stride,
                     segs[i].y_stride, segs[i].rows, cols, mc, units, m_tiles, 0u, 0u, 1u, ws->partials + poff};
        if (kc > 1) {  // every tile split over K
            p.units = 0;
            p.split_units = units;
            p.split_unit0 = 0;
            p.kchunks = kc;
            poff += (uint64_t)units * m_tiles * kc * BM * kPcW;
            outs += (uint64_t)units * m_tiles * reduce_rows(BM, m_tiles, mc) * kPcW / 4;  // four columns a thread
        } else if (wg % 8 == 0 && m_tiles <= 8 && 8 % m_tiles == 0 && ((uint64_t)units * m_tiles) % 8 == 0) {
            p.xcd_map = 1;  // the segment starts on XCD 0 of the round robin
        }
        wg += units * m_tiles * kc;
        g.seg[i] = p;
        g.type[i] = segs[i].type;
        g.wg_end[i] = wg;
        g.out_end[i] = outs;
    }
    if (!gemm_group_types<MB>(ta, tb, g, dim3(wg), st))
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm_group: no kernel for types %u and %u", ta, tb);
    if (kc > 1) hipLaunchKernelGGL((k_gemm_pc_reduce_group<BM>), dim3((uint32_t)((outs + 255) / 256)), dim3(256), 0, st, g);
    return hip_status(hipGetLastError(), "gemm_group launch");
}

}  // namespace

// The grouped bf16 GEMM (halo_mi_gemm_group): x staged once per block of rows (with the fused
// norm as the single-matrix GEMM stages it), then one launch per pair of weight types, in the
// order the types first appear. M tiles as k_gemm_pc: 64 rows up to 64 vectors, 128 up to 128,
// 256 beyond.
int launch_gemm_group(const GroupSeg* segs, uint32_t n, const float* x, uint64_t x_stride, uint32_t cols, uint32_t n_vec,
                      const float* norm_w, float eps, hipStream_t st) {
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    if (!ws)
        return set_error(HALO_MI_E_MEMORY, "gemm_group: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    const int MB = n_vec <= 64 ? 1 : n_vec <= 128 ? 2 : 4;
    const uint32_t BM = 64u * MB;
    const uint64_t cap_rows = std::min(kXbElems / cols, kInvFloats) / BM * BM;
    if (cap_rows == 0) return set_error(HALO_MI_E_UNSUPPORTED, "gemm_group: cols %u too large for the x staging buffer", cols);
    if ((uint64_t)BM * cols * 2 > 0xFFFFFFFFull)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm_group: cols %u too large for one M tile", cols);
    uint32_t types[HALO_MI_GEMV_GROUP_MAX], nt = 0;
    for (uint32_t i = 0; i < n; ++i) {
        bool seen = false;
        for (uint32_t k = 0; k < nt; ++k) seen |= types[k] == segs[i].type;
        if (!seen) types[nt++] = segs[i].type;
    }
    GemmArgs a{nullptr, nullptr, x, x_stride, nullptr, 0, 0, cols, n_vec};
    a.norm_w = norm_w;
    a.norm_eps = eps;
    for (uint64_t m_start = 0; m_start < n_vec; m_start += cap_rows) {
        const uint32_t mc = (uint32_t)std::min<uint64_t>(cap_rows, n_vec - m_start);
        const uint32_t m_tiles = (mc + BM - 1) / BM;
        if (int rc = stage_x(a, m_start, mc, m_tiles * BM, ws, st)) return rc;
        for (uint32_t k0 = 0; k0 < nt; k0 += 2) {
            uint32_t ta = types[k0], tb = k0 + 1 < nt ? types[k0 + 1] : types[k0];
            if (group_type_index(ta) > group_type_index(tb)) std::swap(ta, tb);
            GroupSeg part[HALO_MI_GEMV_GROUP_MAX];
            uint32_t np = 0;
            for (uint32_t i = 0; i < n; ++i)
                if (segs[i].type == ta || segs[i].type == tb) part[np++] = segs[i];
            int rc;
            switch (MB) {
                case 1: rc = gemm_group_launch<1>(part, np, ta, tb, cols, mc, m_tiles, m_start, ws, st); break;
                case 2: rc = gemm_group_launch<2>(part, np, ta, tb, cols, mc, m_tiles, m_start, ws, st); break;
                default: rc = gemm_group_launch<4>(part, np, ta, tb, cols, mc, m_tiles, m_start, ws, st); break;
            }
            if (rc) return rc;
        }
    }
    return HALO_MI_OK;
}

int launch_swiglu(const float* g, uint64_t gs, const float* u, uint64_t us, float* out, uint64_t os, uint32_t rows,
                  uint32_t cols, hipStream_t st) {
    const uint64_t n = (uint64_t)rows * cols;
    hipLaunchKernelGGL(k_swiglu, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, g, gs, u, us, out, os, rows, cols);
    return hip_status(hipGetLastError(), "swiglu launch");
}

}  // namespace halo_mi
