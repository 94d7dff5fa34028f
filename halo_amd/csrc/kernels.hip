// gfx950 (CDNA4) kernels of the halo_mi355x quantized matrix-multiply backend and their
// extern "C" launchers. Wave64 throughout.
//
//   k_gemv_gguf_ref   GGUF layout, 8 lanes per output in cpu::detail::dot's order
//                     (backends/cpu/kernel_common.h:16-27): bit-identical to the CPU backend.
//   k_gemv_slab       SLAB layout, one row per lane, a wave streams 64 rows slot by slot
//                     (1 KB contiguous per load), x is wave-uniform (scalar loads), the
//                     workgroup splits K over its waves and reduces in LDS in a fixed order.
//   k_gemm_slab_bf16  SLAB layout, M >= 8: W slots dequantized exactly, rounded to bf16 and
//                     staged in LDS with x; v_mfma_f32_16x16x32_bf16; optional gate/up pair
//                     with the SwiGLU epilogue.
//   k_dequant_*       exact fp32 dequantization (shares the unpacking code).
//   k_repack / k_unpack  GGUF <-> SLAB.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "common.h"
#include "decode.h"
#include "slab_layout.h"

namespace halo_mi {
namespace {

using namespace dev;

constexpr uint32_t kMaxGemvVec = 4;  // vectors per slab-gemv launch
// Auto choice for the fused gate/up pair: the GEMV kernel streams each weight matrix once per
// 4 vectors, so beyond one launch the MFMA GEMM (which streams it once) is faster.
constexpr uint32_t kGateUpGemvMax = 4;


__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ float ubyte(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sbyte(uint32_t v, int k) { return (float)(int)(int8_t)((v >> (8 * k)) & 0xFFu); }

// ==========================================================================================
// Repack / unpack / dequantize
// ==========================================================================================

// One thread per (slab, block, row), row fastest: the 64 threads of a (slab, block) write each
// of the block's slot records as one contiguous 1 KB, and each reads its row's block.
__global__ void k_repack_slab(uint32_t type, const uint8_t* __restrict__ src, uint64_t src_stride, uint32_t rows,
                              uint32_t cols, uint8_t* __restrict__ dst) {
    const SlabGeom g = slab_geom(type, cols);
    const uint32_t nblk = cols / block_elems(type), S = cols / kSlot;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t slabs = (rows + kSlabRows - 1) / kSlabRows;
    if (idx >= slabs * nblk * kSlabRows) return;
    const uint32_t r = (uint32_t)(idx % kSlabRows);
    const uint64_t sb = idx / kSlabRows;
    const uint32_t b = (uint32_t)(sb % nblk);
    const uint64_t slab = sb / nblk, row = slab * kSlabRows + r;
    uint8_t* out = dst + slab * g.slab_bytes;
    const uint8_t* s = src + row * src_stride + (uint64_t)b * block_bytes(type);
    if (type == kQ4_K && ((reinterpret_cast<uintptr_t>(s) | src_stride) % 16) == 0) {
        // vector path: 9 x 16 B in; 8 slot records and the header out as 16-byte stores
        uint4 blk[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) blk[i] = row < rows ? reinterpret_cast<const uint4*>(s)[i] : uint4{0, 0, 0, 0};
        *reinterpret_cast<uint4*>(out + g.aux_off + ((uint64_t)b * 64 + r) * 16) = blk[0];
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {  // 32 quant bytes: sub-blocks 2 grp (low nibbles), 2 grp + 1 (high)
            const uint4 A = blk[1 + 2 * grp], B = blk[2 + 2 * grp];
            const uint32_t a[4] = {A.x, A.y, A.z, A.w}, c[4] = {B.x, B.y, B.z, B.w};
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                lo[k] = (a[k] & 0x0F0F0F0Fu) | ((c[k] & 0x0F0F0F0Fu) << 4);
                hi[k] = ((a[k] >> 4) & 0x0F0F0F0Fu) | (c[k] & 0xF0F0F0F0u);
            }
            *reinterpret_cast<uint4*>(out + g.q_off + (((uint64_t)b * 8 + 2 * grp) * 64 + r) * 16) = uint4{lo[0], lo[1], lo[2], lo[3]};
            *reinterpret_cast<uint4*>(out + g.q_off + (((uint64_t)b * 8 + 2 * grp + 1) * 64 + r) * 16) = uint4{hi[0], hi[1], hi[2], hi[3]};
        }
        return;
    }
    uint8_t blk[210];
    const uint32_t bb = block_bytes(type);
    if (row < rows) {
        for (uint32_t i = 0; i < bb; ++i) blk[i] = s[i];
    } else {
        for (uint32_t i = 0; i < bb; ++i) blk[i] = 0;
    }
    slab_pack_block(type, blk, out, g, S, r, b);
}

__global__ void k_unpack_slab(uint32_t type, const uint8_t* __restrict__ src, uint32_t rows, uint32_t cols,
                              uint8_t* __restrict__ dst, uint64_t dst_stride) {
    const SlabGeom g = slab_geom(type, cols);
    const uint32_t nblk = cols / block_elems(type), S = cols / kSlot;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)rows * nblk) return;
    const uint64_t row = idx / nblk;
    const uint32_t b = (uint32_t)(idx % nblk);
    uint8_t blk[210];
    slab_unpack_block(type, src + (row / kSlabRows) * g.slab_bytes, blk, g, S, (uint32_t)(row % kSlabRows), b);
    uint8_t* d = dst + row * dst_stride + (uint64_t)b * block_bytes(type);
    for (uint32_t i = 0; i < block_bytes(type); ++i) d[i] = blk[i];
}

__global__ void k_dequant_gguf(uint32_t type, const uint8_t* __restrict__ w, uint64_t w_stride, uint32_t cols,
                               uint32_t first_row, uint32_t n_rows, float* __restrict__ out, uint64_t out_stride) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)n_rows * cols) return;
    const uint64_t r = idx / cols;
    const uint32_t i = (uint32_t)(idx % cols);
    out[r * out_stride + i] = gguf_elem(type, w + (first_row + r) * w_stride, i);
}

// Exact fp32 weights of slot s of the row at lane r of `slab` (the reference's expressions).
template <uint32_t T>
__device__ __forceinline__ void slab_slot_weights(const uint8_t* __restrict__ slab, const SlabGeom& g, uint32_t r,
                                                  uint32_t s, float w[32]) {
#pragma clang fp contract(off)
    if constexpr (T == kQ4_0) {
        const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + r) * 16);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(slab + g.aux_off + ((uint64_t)s * 64 + r) * 2));
        const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t b = (Q[i] >> (8 * k)) & 0xFFu;
                w[4 * i + k] = (float)((int)(b & 15u) - 8) * d;
                w[16 + 4 * i + k] = (float)((int)(b >> 4) - 8) * d;
            }
    } else if constexpr (T == kQ8_0) {
        const float d = h2f(*reinterpret_cast<const uint16_t*>(slab + g.aux_off + ((uint64_t)s * 64 + r) * 2));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + (((uint64_t)s * 2 + h) * 64 + r) * 16);
            const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) w[16 * h + 4 * i + k] = sbyte(Q[i], k) * d;
        }
    } else if constexpr (T == kQ4_K) {
        const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + r) * 16);
        const uint4 hdr = *reinterpret_cast<const uint4*>(slab + g.aux_off + ((uint64_t)(s / 8) * 64 + r) * 16);
        float d1, m1;
        q4k_scales(hdr, s % 8, d1, m1);
        const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t b = (Q[i] >> (8 * k)) & 0xFFu;
                w[4 * i + k] = d1 * (float)(b & 15u) - m1;
                w[16 + 4 * i + k] = d1 * (float)(b >> 4) - m1;
            }
    } else {  // Q6_K
        const uint4 ql = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + r) * 16);
        const uint2 qh = *reinterpret_cast<const uint2*>(slab + g.aux_off + ((uint64_t)s * 64 + r) * 8);
        const uint32_t sb = s / 8, j = s % 8;
        const uint8_t* scp = slab + g.sc_off + ((uint64_t)sb * 64 + r) * 16;
        const float d = h2f(*reinterpret_cast<const uint16_t*>(slab + g.d_off + ((uint64_t)sb * 64 + r) * 2));
        const float dA = d * (float)(int8_t)scp[2 * j], dB = d * (float)(int8_t)scp[2 * j + 1];
        uint32_t lo[4], hi[4];
        q6_slot_bytes(ql, qh, lo, hi);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w[4 * i + k] = dA * (float)((int)((lo[i] >> (8 * k)) & 0xFFu) - 32);
                w[16 + 4 * i + k] = dB * (float)((int)((hi[i] >> (8 * k)) & 0xFFu) - 32);
            }
    }
}

template <uint32_t T>
__global__ void k_dequant_slab(const uint8_t* __restrict__ w, uint32_t cols, uint32_t first_row, uint32_t n_rows,
                               float* __restrict__ out, uint64_t out_stride) {
    const SlabGeom g = slab_geom(T, cols);
    const uint32_t S = cols / kSlot;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)n_rows * S) return;
    const uint32_t s = (uint32_t)(idx % S);
    const uint64_t row = first_row + idx / S;
    float wv[32];
    slab_slot_weights<T>(w + (row / kSlabRows) * g.slab_bytes, g, (uint32_t)(row % kSlabRows), s, wv);
    float* o = out + (idx / S) * out_stride + (uint64_t)s * 32;
    for (int i = 0; i < 32; ++i) o[i] = wv[i];
}

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

struct GemvSlabArgs {
    const uint8_t* w0;  // slab image (gate, or the only matrix)
    const uint8_t* w1;  // up matrix (PAIR) or null
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
    uint32_t rows, cols, n_vec;
    uint32_t ks;          // K chunks per slab
    uint64_t* slots;      // [slabs][chunks][NV][64] partials as (value, ready) words, 0 between launches
    uint32_t* counters;   // [slabs], zero between launches
};

// ---- inner products of one 32-weight slot against x[0..31] (x in LDS, 16-byte aligned) ----

typedef float float2v __attribute__((ext_vector_type(2)));

// AND with a mask the compiler cannot see through: it would otherwise fold the mask into
// per-byte bit-field extracts and lose the v_cvt_f32_ubyteN patterns.
template <uint32_t M>
__device__ __forceinline__ uint32_t and_opaque(uint32_t v) {
    uint32_t r;
    __asm__("v_and_b32 %0, %1, %2" : "=v"(r) : "i"(M), "v"(v));
    return r;
}
template <uint32_t M>
__device__ __forceinline__ uint32_t xor_opaque(uint32_t v) {
    uint32_t r;
    __asm__("v_xor_b32 %0, %1, %2" : "=v"(r) : "i"(M), "v"(v));
    return r;
}

// (a & m) | b, opaque to the compiler (keeps the byte-convert patterns, see and_opaque)
__device__ __forceinline__ uint32_t and_or_opaque(uint32_t a, uint32_t m, uint32_t b) {
    uint32_t r;
    __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(b));
    return r;
}

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

// Value of the fp8 (e4m3) code 1 on this device: every code c < 16 converts to exactly
// c * fp8_unit(), so v_cvt_pk_f32_fp8 turns two 4-bit quants into two exact floats.
__device__ __forceinline__ float fp8_unit() { return __builtin_amdgcn_cvt_pk_f32_fp8(1u, false)[0]; }

// 4-bit slot record: lo = sum x[t] q[t] (t < 16), hi = sum x[16 + t] q[16 + t], both in units
// of fp8_unit().
__device__ __forceinline__ void dot_nibbles(const uint4& q, const float* xs, float& lo, float& hi) {
    const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
    const float4* x4 = reinterpret_cast<const float4*>(xs);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = Q[i] & 0x0F0F0F0Fu, b = (Q[i] >> 4) & 0x0F0F0F0Fu;
        const float2v a01 = __builtin_amdgcn_cvt_pk_f32_fp8(a, false), a23 = __builtin_amdgcn_cvt_pk_f32_fp8(a, true);
        const float2v b01 = __builtin_amdgcn_cvt_pk_f32_fp8(b, false), b23 = __builtin_amdgcn_cvt_pk_f32_fp8(b, true);
        const float4 xl = x4[i], xh = x4[4 + i];
        lo = fmaf(xl.x, a01[0], lo);
        lo = fmaf(xl.y, a01[1], lo);
        lo = fmaf(xl.z, a23[0], lo);
        lo = fmaf(xl.w, a23[1], lo);
        hi = fmaf(xh.x, b01[0], hi);
        hi = fmaf(xh.y, b01[1], hi);
        hi = fmaf(xh.z, b23[0], hi);
        hi = fmaf(xh.w, b23[1], hi);
    }
}

// Byte quants (one per weight) A (t < 16) and B (16 + t), unsigned.
__device__ __forceinline__ void dot_bytes(const uint32_t A[4], const uint32_t B[4], const float* xs, float& lo,
                                          float& hi) {
    const float4* x4 = reinterpret_cast<const float4*>(xs);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 xl = x4[i], xh = x4[4 + i];
        lo = fmaf(xl.x, ubyte(A[i], 0), lo);
        lo = fmaf(xl.y, ubyte(A[i], 1), lo);
        lo = fmaf(xl.z, ubyte(A[i], 2), lo);
        lo = fmaf(xl.w, ubyte(A[i], 3), lo);
        hi = fmaf(xh.x, ubyte(B[i], 0), hi);
        hi = fmaf(xh.y, ubyte(B[i], 1), hi);
        hi = fmaf(xh.z, ubyte(B[i], 2), hi);
        hi = fmaf(xh.w, ubyte(B[i], 3), hi);
    }
}

// The loaded records of one slot group (up to 8 slots) of one row.
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

template <uint32_t T>
__device__ __forceinline__ void load_group(SlotGroup<T>& G, const uint8_t* __restrict__ slab, const SlabGeom& g,
                                           uint32_t lane, uint32_t grp, uint32_t S) {
    const uint32_t sb = grp * 8;
    // scales first, then the quants in slot order: loads complete in order, so slot j can be
    // used as soon as its own record has arrived
    if constexpr (T == kQ4_K) {
        G.hdr = ld_nt16(slab + g.aux_off + ((uint64_t)grp * 64 + lane) * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) G.q[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
    } else if constexpr (T == kQ6_K) {
        G.d = ld_nt2(slab + g.d_off + ((uint64_t)grp * 64 + lane) * 2);
        G.sc = ld_nt16(slab + g.sc_off + ((uint64_t)grp * 64 + lane) * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            G.ql[j] = ld_nt16(slab + g.q_off + ((uint64_t)(sb + j) * 64 + lane) * 16);
            G.qh[j] = ld_nt8(slab + g.aux_off + ((uint64_t)(sb + j) * 64 + lane) * 8);
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

// End of a slab-GEMV workgroup: the waves' partial sums meet in LDS in wave order, then (split
// K) the workgroups of a slab meet in the workspace, and the result (SiLU(gate) * up for the
// pair) is written. acc0 holds this wave's sums in fp32, rows = lanes.
// Split-K: the workgroup's start ticket for its slab (0 .. nch - 1), taken when it starts and
// used only at its end, so the device-scope round trip overlaps the weight stream.
__device__ __forceinline__ uint32_t gemv_ticket(const GemvSlabArgs& a, uint32_t slab, uint32_t nch) {
    uint32_t t = 0;
    if (nch > 1 && threadIdx.x == 0)
        t = __hip_atomic_fetch_add(&a.counters[slab], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return t;
}

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
    const uint32_t row = slab * kSlabRows + lane;
    float acc1[NV];  // the up sums (PAIR)
#pragma unroll
    for (int v = 0; v < NV; ++v) acc1[v] = 0.0f;
    if (nch > 1) {
        // Split-K meeting point, without cache maintenance and without a round trip at the end
        // of most workgroups. The workgroup with the slab's last start ticket is the reducer:
        // every other chunk of the slab started before it, so they are all running. The others
        // store their partials as 64-bit words (fp32 bits, 1 = ready: one atomic access
        // carries the value and its mark) and finish. The reducer loads those words, re-reads
        // (bounded, with a pause) any not yet ready, adds the chunks in chunk order
        // (deterministic), and clears the words and the ticket counter for the next launch.
        uint64_t* P = a.slots + (uint64_t)slab * nch * NV * 64;
        if (__builtin_amdgcn_readfirstlane(ticket) != nch - 1) {
#pragma unroll
            for (int v = 0; v < NV; ++v)
                __hip_atomic_store(P + ((uint64_t)c * NV + v) * 64 + lane,
                                   (uint64_t)__float_as_uint(acc0[v]) | (1ull << 32), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        float own[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            own[v] = acc0[v];
            acc0[v] = 0.0f;
        }
        // The loads of 8 chunks are issued before any is used (one memory round trip per 8
        // chunks); past the last chunk the address is clamped and the value dropped.
        constexpr uint32_t KB = 8;
        constexpr uint32_t kSpinLimit = 1u << 20;  // the other chunks are running: a few microseconds
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
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    float val = own[v];
                    if (k != c) {
                        uint64_t w = q[kk][v];
                        for (uint32_t spin = 0; (w >> 32) == 0 && spin < kSpinLimit; ++spin) {
                            __builtin_amdgcn_s_sleep(2);
                            w = __hip_atomic_load(P + ((uint64_t)k * NV + v) * 64 + lane, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                        }
                        val = (w >> 32) ? __uint_as_float((uint32_t)w) : __builtin_nanf("");
                    }
                    if (k < a.ks) acc0[v] += val;
                    else acc1[v] += val;
                }
            }
        }
        for (uint32_t k = 0; k < nch; ++k)
            if (k != c)
#pragma unroll
                for (int v = 0; v < NV; ++v)
                    __hip_atomic_store(P + ((uint64_t)k * NV + v) * 64 + lane, 0ull, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) __hip_atomic_store(&a.counters[slab], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (row >= a.rows) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        if ((uint32_t)v >= a.n_vec) break;
        a.y[(uint64_t)v * a.y_stride + row] = PAIR ? silu_f(acc0[v]) * acc1[v] : acc0[v];
    }
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
__device__ __forceinline__ void mx_load_x(float (&xr)[NV][4], const float* __restrict__ x, uint64_t x_stride,
                                          uint32_t grp, uint32_t S, uint32_t lane) {
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
        } else {  // Q6_K: the two halves have their own scales
            uint32_t lo6[4], hi6[4];
            q6_slot_bytes_gemv(G.ql[j], G.qh[j], lo6, hi6);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mx_kstep<NV>(A, as_b(lo6[i] & 0x00FF00FFu, __builtin_amdgcn_perm(0u, lo6[i], 0x0C030C01u)), j, i, D);
                mx_kstep<NV>(A, as_b(hi6[i] & 0x00FF00FFu, __builtin_amdgcn_perm(0u, hi6[i], 0x0C030C01u)), j, 4 + i, Dh);
            }
        }
        if constexpr (T == kQ4_K) {
            uint32_t sc, m;
            q4k_sc_m(G.hdr.y, G.hdr.z, G.hdr.w, (uint32_t)j, sc, m);
            const float fsc = (float)sc, fm = (float)m;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                sa[v] = fmaf(fsc, mx_dot<NV>(D, v), sa[v]);
                sb[v] = fmaf(fm, xsum_at(xs[v], 8 * j), sb[v]);
            }
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
    if constexpr (T == kQ4_K) {
        const float d = h2f(G.hdr.x & 0xFFFFu), dmin = h2f(G.hdr.x >> 16);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = fmaf(d, sa[v], -(dmin * sb[v]));
    } else if constexpr (T == kQ6_K) {
        const float d = h2f(G.d);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = d * sa[v];
    }
}

// Workgroup size bound: single-vector kernels fit 128 VGPRs (16 waves per workgroup), except
// the Q8_0 and Q6_K loops (two register groups); the others run at most 8 waves.
template <uint32_t T, int NV, bool ONE>
constexpr uint32_t mx_max_threads() { return (NV == 1 && (ONE || (T != kQ8_0 && T != kQ6_K))) ? 1024u : 512u; }

// grid, split and LDS as k_gemv_slab, plus one A table per wave after the partials. ONE: every
// wave has at most one slot group (no second register buffer, so more waves fit per SIMD).
template <uint32_t T, int NV, bool PAIR, bool ONE>
__global__ __launch_bounds__((mx_max_threads<T, NV, ONE>())) void k_gemv_mx(GemvSlabArgs a) {
    extern __shared__ float smem[];
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    constexpr int M = mx_blocks<NV>();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint32_t S = a.cols / kSlot, ngrp = (S + 7) / 8;
    const uint32_t nch = a.ks * MATS;
    const uint32_t slab = blockIdx.x / nch, c = blockIdx.x % nch;
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
    if constexpr (ONE) {
        if (w0 < w1) {
            SlotGroup<T> G;
            mx_load_x<NV>(xr, a.x, a.x_stride, w0, S, lane);
            load_group<T>(G, slab0, geo, lane, w0, S);
            ticket = gemv_ticket(a, slab, nch);
            s16x4 A[4 * M];
            int es[NV];
            float xs[NV];
            mx_build<T, NV>(xr, tab, lane, A, es, xs);
            mx_group<T, NV>(G, A, xs, min(8u, S - w0 * 8), acc0);
#pragma unroll
            for (int v = 0; v < NV; ++v) acc0[v] = ldexpf(acc0[v], es[v]);
        } else {
            ticket = gemv_ticket(a, slab, nch);
        }
        gemv_finish<NV, PAIR>(a, acc0, red, wave, nw, lane, slab, c, nch, ticket);
        return;
    }
    SlotGroup<T> cur, nxt;
    if (w0 < w1) {  // x first: the A table is built while the weights are on their way
        mx_load_x<NV>(xr, a.x, a.x_stride, w0, S, lane);
        load_group<T>(cur, slab0, geo, lane, w0, S);
    }
    ticket = gemv_ticket(a, slab, nch);
    // One group: build its A table from xr, prefetch x and the weights of the next group (past
    // the last group: the last one again, an L2 hit, so the loop stays branch-free), multiply.
    auto step = [&](const SlotGroup<T>& G, SlotGroup<T>& next, uint32_t grp) {
        s16x4 A[4 * M];
        int es[NV];
        float xs[NV];
        mx_build<T, NV>(xr, tab, lane, A, es, xs);
        const uint32_t gn = min(grp + 1, w1 - 1);
        mx_load_x<NV>(xr, a.x, a.x_stride, gn, S, lane);
        load_group<T>(next, slab0, geo, lane, gn, S);
        float accg[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) accg[v] = 0.0f;
        mx_group<T, NV>(G, A, xs, min(8u, S - grp * 8), accg);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc0[v] += ldexpf(accg[v], es[v]);
    };
    for (uint32_t grp = w0; grp < w1; ++grp) {
        step(cur, nxt, grp);
        if (grp + 1 >= w1) break;
        ++grp;
        step(nxt, cur, grp);
    }
    gemv_finish<NV, PAIR>(a, acc0, red, wave, nw, lane, slab, c, nch, ticket);
}

__global__ void k_fill_u32(uint32_t* p, uint64_t n, uint32_t v) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
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
// SLAB GEMM on bf16 MFMA (M >= 8)
// ==========================================================================================

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 128;        // x rows per workgroup
constexpr int kGemmBN = 64;         // W rows per workgroup and matrix (one slab)
constexpr int kGemmLd = 32 + 8;     // LDS row pitch in bf16 (32 k + 8 pad)

struct GemmArgs {
    const uint8_t* w0;
    const uint8_t* w1;
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
    uint32_t rows, cols, n_vec;
};

// Workgroup of 256 threads (4 waves); tile 128 x 64 of y per matrix; K step = one slot (32).
// Wave w owns x rows [32w, 32w + 32) of the tile: 2 m-tiles x 4 n-tiles x MATS of 16x16.
// v_mfma_f32_16x16x32_bf16 operands: lane l holds A[l % 16][8 (l / 16) .. +8],
// B[8 (l / 16) .. +8][l % 16]; result D[4 (l / 16) + i][l % 16], i < 4.
template <uint32_t T, bool PAIR>
__global__ __launch_bounds__(256) void k_gemm_slab_bf16(GemmArgs a) {
    constexpr int MATS = PAIR ? 2 : 1;
    __shared__ __bf16 xs[kGemmBM * kGemmLd];
    __shared__ __bf16 ws[MATS * kGemmBN * kGemmLd];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t S = a.cols / kSlot;
    const uint32_t slab = blockIdx.x;          // W rows [64 slab, +64)
    const uint32_t m0 = blockIdx.y * kGemmBM;  // x rows
    const SlabGeom g = slab_geom(T, a.cols);
    const uint8_t* wb[2] = {a.w0 + (uint64_t)slab * g.slab_bytes, PAIR ? a.w1 + (uint64_t)slab * g.slab_bytes : nullptr};

    floatx4 acc[MATS][2][4];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[m][i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // x tile loader: thread -> (row tid / 2, 16 k at 16 (tid % 2))
    const uint32_t xr = tid >> 1, xh = tid & 1u;
    const bool xlive = m0 + xr < a.n_vec;
    const float* xrow = a.x + (uint64_t)(xlive ? m0 + xr : 0) * a.x_stride + 16 * xh;
    // W loader: thread -> (matrix, row, 16-weight half)
    const uint32_t wm = PAIR ? (tid >> 7) : 0u, wr = (tid & 127u) >> 1, wh = tid & 1u;
    const bool wlive = PAIR || tid < 128;

    for (uint32_t s = 0; s < S; ++s) {
        {
            float v[16];
            if (xlive) {
                const float4* p = reinterpret_cast<const float4*>(xrow + (uint64_t)s * 32);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 f = p[i];
                    v[4 * i] = f.x;
                    v[4 * i + 1] = f.y;
                    v[4 * i + 2] = f.z;
                    v[4 * i + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = 0.0f;
            }
            bf16x8 lo, hi;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = (__bf16)v[i];
                hi[i] = (__bf16)v[8 + i];
            }
            *reinterpret_cast<bf16x8*>(&xs[xr * kGemmLd + 16 * xh]) = lo;
            *reinterpret_cast<bf16x8*>(&xs[xr * kGemmLd + 16 * xh + 8]) = hi;
        }
        if (wlive) {
            float wv[32];
            slab_slot_weights<T>(wb[wm], g, wr, s, wv);
            bf16x8 lo, hi;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = (__bf16)wv[16 * wh + i];
                hi[i] = (__bf16)wv[16 * wh + 8 + i];
            }
            __bf16* dst = &ws[(wm * kGemmBN + wr) * kGemmLd + 16 * wh];
            *reinterpret_cast<bf16x8*>(dst) = lo;
            *reinterpret_cast<bf16x8*>(dst + 8) = hi;
        }
        __syncthreads();
        bf16x8 A[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            A[i] = *reinterpret_cast<const bf16x8*>(&xs[(32 * wave + 16 * i + (lane & 15)) * kGemmLd + 8 * (lane >> 4)]);
#pragma unroll
        for (int m = 0; m < MATS; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bf16x8 B =
                    *reinterpret_cast<const bf16x8*>(&ws[(m * kGemmBN + 16 * j + (lane & 15)) * kGemmLd + 8 * (lane >> 4)]);
#pragma unroll
                for (int i = 0; i < 2; ++i) acc[m][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], B, acc[m][i][j], 0, 0, 0);
            }
        __syncthreads();
    }
    // epilogue
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t n = slab * kGemmBN + 16 * j + (lane & 15);
            if (n >= a.rows) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + 32 * wave + 16 * i + 4 * (lane >> 4) + e;
                if (m >= a.n_vec) continue;
                float out;
                if constexpr (PAIR) out = silu_f(acc[0][i][j][e]) * acc[1][i][j][e];
                else out = acc[0][i][j][e];
                a.y[(uint64_t)m * a.y_stride + n] = out;
            }
        }
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

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kPcLd = 40;     // LDS row pitch in bf16 (32 k + 8 pad: 80 B, conflict-free reads)
constexpr int kPcW = 128;     // W rows per tile
constexpr int kPcDepth = 4;   // stages of producer W loads in flight (a ring of registers)
constexpr int kPcADepth = 4;  // stages of consumer x-fragment loads in flight
constexpr uint32_t kPcOob = 0x80000000u;  // buffer offset past every resource: the load returns 0
constexpr int kPcBufs = 4;    // LDS stages (the producers write two stages ahead)
constexpr int kPcUnroll = 8;  // producer loop unroll: ring slot, LDS buffer and Q4_K sub-block static

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
    // W tiles [units, units + split_units) (all M tiles) run as kchunks K chunks each, one
    // workgroup per chunk after the whole tiles; their fp32 partials go to
    // partials[(split tile * kchunks + chunk)][BM][128] and k_gemm_pc_reduce adds them.
    uint32_t split_units;
    uint32_t kchunks;
    float* partials;
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
__global__ void k_x_to_frag(const float* __restrict__ x, uint64_t x_stride, uint32_t n_vec, uint32_t m_pad,
                            uint32_t cols, __bf16* __restrict__ out) {
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
        v = bf16x8{(__bf16)a.x, (__bf16)a.y, (__bf16)a.z, (__bf16)a.w, (__bf16)c.x, (__bf16)c.y, (__bf16)c.z, (__bf16)c.w};
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

// Per-lane byte offsets of a producer thread's records inside one stage of a slab.
struct PcOff {
    uint32_t q, aux, sc, d;
};

template <uint32_t T>
__device__ __forceinline__ PcOff pc_offsets(uint32_t r, uint32_t h) {
    if constexpr (T == kQ4_K) return {r * 16 + 8 * h, r * 16, 0, 0};
    else if constexpr (T == kQ4_0 || T == kQ8_0) return {r * 16 + 8 * h, r * 2, 0, 0};
    else return {r * 16 + 8 * h, r * 8 + 4 * h, r * 16, r * 2};
}

// Stage s (slot s of K) of one producer thread's records; `slab` is the wave's slab resource.
// Stage s of one producer thread's records; `slab` is the wave's slab resource. A stage that is
// not live reads past the resource (no branch): zero records, i.e. zero weights.
template <uint32_t T>
__device__ __forceinline__ void pc_load_w(PcW<T>& R, __amdgpu_buffer_rsrc_t slab, const SlabGeom& g, const PcOff& o,
                                          uint32_t s, bool live) {
    const uint32_t sb = s / 8;
    auto so = [&](uint64_t x) { return live ? (uint32_t)x : kPcOob; };
    if constexpr (T == kQ4_K) {
        R.q = bld64(slab, o.q, so(g.q_off + s * 1024));
        R.hdr = bld128(slab, o.aux, so(g.aux_off + sb * 1024));
    } else if constexpr (T == kQ4_0) {
        R.q = bld64(slab, o.q, so(g.q_off + s * 1024));
        R.d = bld16(slab, o.aux, so(g.aux_off + s * 128));
    } else if constexpr (T == kQ8_0) {
        R.qa = bld64(slab, o.q, so(g.q_off + s * 2048));
        R.qb = bld64(slab, o.q, so(g.q_off + s * 2048 + 1024));
        R.d = bld16(slab, o.aux, so(g.aux_off + s * 128));
    } else {
        R.ql = bld64(slab, o.q, so(g.q_off + s * 1024));
        R.qh = bld32(slab, o.aux, so(g.aux_off + s * 512));
        R.sc = bld16(slab, o.sc, so(g.sc_off + sb * 1024 + 2 * (s % 8)));
        R.d = bld16(slab, o.d, so(g.d_off + sb * 128));
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
template <uint32_t T, bool PAIR, int MB>
__global__ __launch_bounds__(512) void k_gemm_pc(GemmPcArgs a) {
    constexpr int BM = 64 * MB;
    constexpr int WM = MB == 1 ? 2 : 4, WN = 4 / WM;
    constexpr int MBW = BM / WM / 32, NBW = 4 / WN;
    constexpr uint32_t STAGE = kPcW * kPcLd;  // bf16 per LDS stage (W only)
    __shared__ __bf16 lds[kPcBufs * STAGE];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t S = a.cols / kSlot;
    const SlabGeom g = slab_geom(T, a.cols);
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;

    // workgroup -> (W tile u, M tile mt) for a whole tile, or (split tile st, K chunk)
    const uint32_t whole = a.units * a.m_tiles;
    const bool split = blockIdx.x >= whole;
    uint32_t u, mt, st = 0, chunk = 0;
    if (!split) {
        const uint32_t wg = blockIdx.x;
        if (a.xcd_map) {
            const uint32_t grp = 8 / a.m_tiles, xcd = wg % 8;
            mt = xcd / grp;
            u = (wg / 8) * grp + xcd % grp;
        } else {
            u = wg / a.m_tiles;
            mt = wg % a.m_tiles;
        }
    } else {
        st = (blockIdx.x - whole) / a.kchunks;
        chunk = (blockIdx.x - whole) % a.kchunks;
        u = a.units + st / a.m_tiles;
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
    const uint32_t n_pad = (n + kPcUnroll - 1) / kPcUnroll * kPcUnroll;

    if (wave < 4) {
        // ---------------- consumers ----------------
        const uint32_t wm = wave % WM, wn = wave / WM;
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
        uint4 AR[kPcADepth][MBW][2];
        // stages past s_end read zeros (out of range), so padded stages add exactly 0
        auto load_a = [&](int slot, uint32_t s) {
#pragma unroll
            for (int i = 0; i < MBW; ++i)
#pragma unroll
                for (int k = 0; k < 2; ++k)
                    AR[slot][i][k] = bld128(xres, xlane, s < s_end ? (((wm * MBW + i) * S + s) * 2 + k) * 1024 : kPcOob);
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
        read_b(0, 0, B0);
        // stage i: x fragments from ring slot i % 4, W from LDS buffer i % 4; unrolled so both
        // are static, and branch-free so the loads' waits are exact (padded stages are zeros)
        static_assert(kPcADepth == kPcBufs, "one static index for the x ring and the LDS buffers");
        for (uint32_t i0 = 0; i0 < n_pad; i0 += kPcBufs) {
#pragma unroll
            for (int q = 0; q < kPcBufs; ++q) {
                read_b(q, 1, B1);
                mma(q, 0, B0);
                read_b((q + 1) % kPcBufs, 0, B0);  // stage i + 1 (zeros or junk past the end, unused)
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
                        if (col < a.rows) yrow[col] = silu_f(acc[i][j][r]) * acc[i][j + NBW / 2][r];
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
    const uint32_t pt = tid - 256;
    const uint32_t mat = __builtin_amdgcn_readfirstlane(pt >> 7);  // one matrix per wave
    const uint32_t r = (pt >> 1) & 63u, h = pt & 1u;
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
    PcW<T> R[kPcDepth];
    auto load = [&](int slot, uint32_t s) { pc_load_w<T>(R[slot], slab, g, off, s, s < s_end); };
    // j: the stage's slot within its super-block (static in the unrolled loop)
    auto store = [&](int slot, uint32_t j, int buf) {
        bf16x8 lo, hi;
        pc_dequant<T>(R[slot], h, j, inv_unit, lo, hi);
        __bf16* st = lds + buf * STAGE;
        *reinterpret_cast<bf16x8*>(st + wdst) = lo;
        *reinterpret_cast<bf16x8*>(st + wdst + 16) = hi;
    };
#pragma unroll
    for (int p = 0; p < kPcDepth; ++p) load(p, s_begin + p);
    store(0, 0, 0);
    load(0, s_begin + kPcDepth);
    store(1, 1, 1);
    load(1, s_begin + kPcDepth + 1);
    pc_sync();  // B_0
    // iteration i writes local stage i + 2 from ring slot (i + 2) % 4 into buffer (i + 2) % 4;
    // unrolled by 8 so slot, buffer and sub-block are static, and branch-free so the loads'
    // waits are exact (stages past the end are junk that no consumer reads)
    for (uint32_t i0 = 0; i0 < n_pad; i0 += kPcUnroll) {
#pragma unroll
        for (int q = 0; q < kPcUnroll; ++q) {
            const int k = (q + 2) % kPcDepth;
            store(k, (q + 2) % 8, (q + 2) % kPcBufs);
            load(k, s_begin + i0 + q + 2 + kPcDepth);
            pc_sync();  // B_{i+1}
            // keep each stage's work between its barriers: hoisting a later stage's decode would
            // make it wait for that stage's loads
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Sum of the K-chunk partials of a split launch (in chunk order) and the epilogue.
// grid = (tiles * BM * 128 / 256), block 256; one output element (pair) per thread.
template <bool PAIR, int BM>
__global__ void k_gemm_pc_reduce(GemmPcArgs a) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    constexpr uint32_t NC = PAIR ? 64 : kPcW;  // output columns per tile
    const uint64_t tiles = (uint64_t)a.split_units * a.m_tiles;
    if (idx >= tiles * BM * NC) return;
    const uint32_t tile = (uint32_t)(idx / (BM * NC)), e = (uint32_t)(idx % (BM * NC));
    const uint32_t ml = e / NC, nl = e % NC;
    const uint32_t u = a.units + tile / a.m_tiles, mt = tile % a.m_tiles;
    const uint32_t m = mt * BM + ml;
    if (m >= a.n_vec) return;
    const float* P = a.partials + (uint64_t)tile * a.kchunks * BM * kPcW + ml * kPcW;
    float s0 = 0.0f, s1 = 0.0f;
    for (uint32_t c = 0; c < a.kchunks; ++c) {
        s0 += P[(uint64_t)c * BM * kPcW + nl];
        if constexpr (PAIR) s1 += P[(uint64_t)c * BM * kPcW + 64 + nl];
    }
    float* yrow = a.y + (uint64_t)m * a.y_stride;
    if constexpr (PAIR) {
        const uint32_t col = u * kSlabRows + nl;
        if (col < a.rows) yrow[col] = silu_f(s0) * s1;
    } else {
        const uint32_t col = 2 * u * kSlabRows + nl;
        if (col < a.rows) yrow[col] = s0;
    }
}

// ==========================================================================================
// host-side validation and launchers
// ==========================================================================================

int hip_status(hipError_t e, const char* op) {
    if (e == hipSuccess) return HALO_MI_OK;
    return set_error(HALO_MI_E_DEVICE, "%s: %s", op, hipGetErrorString(e));
}

bool ranges_overlap(const void* a, uint64_t na, const void* b, uint64_t nb) {
    if (na == 0 || nb == 0 || a == nullptr || b == nullptr) return false;
    const auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + nb && pb < pa + na;
}

// Extent in bytes of `rows` rows of `row_bytes` spaced `stride` bytes apart.
uint64_t extent(uint64_t rows, uint64_t stride, uint64_t row_bytes) { return rows ? (rows - 1) * stride + row_bytes : 0; }

// ---- split-K workspace, one per (device, stream) ------------------------------------------
// Calls on one stream run in order, so they can share it. It is allocated on the first call
// on a stream (hipMalloc; counters cleared by a fill kernel on that stream, never a memset);
// a call on a stream that is being captured into a graph and has no workspace yet runs
// without split-K.
constexpr uint64_t kPartialFloats = 8ull << 20;  // GEMM split-tile partials: 32 MiB
constexpr uint64_t kSlots = 4ull << 20;          // GEMV split-K words: 32 MiB
constexpr uint64_t kCounters = 1ull << 20;        // slabs (64M rows)
constexpr uint64_t kXbElems = 16ull << 20;        // bf16 copy of x for the GEMM: 32 MiB

struct Workspace {
    float* partials = nullptr;
    uint64_t* slots = nullptr;
    uint32_t* counters = nullptr;
    __bf16* xb = nullptr;
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

int workspace_for(hipStream_t st, Workspace** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(HALO_MI_E_DEVICE, "gemv: hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find({dev, st});
    if (it != g_ws.end()) {
        *out = &it->second;
        return HALO_MI_OK;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (st != nullptr && hipStreamIsCapturing(st, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
        *out = nullptr;  // cannot allocate under capture: caller runs without split-K
        return HALO_MI_OK;
    }
    Workspace w;
    if (hipMalloc(&w.partials, kPartialFloats * sizeof(float)) != hipSuccess)
        return set_error(HALO_MI_E_MEMORY, "gemv: cannot allocate the split-K workspace");
    if (hipMalloc(&w.counters, kCounters * sizeof(uint32_t)) != hipSuccess) {
        (void)hipFree(w.partials);
        return set_error(HALO_MI_E_MEMORY, "gemv: cannot allocate the split-K counters");
    }
    if (hipMalloc(&w.xb, kXbElems * sizeof(__bf16)) != hipSuccess) {
        (void)hipFree(w.partials);
        (void)hipFree(w.counters);
        return set_error(HALO_MI_E_MEMORY, "gemm: cannot allocate the bf16 staging buffer for x");
    }
    if (hipMalloc(&w.slots, kSlots * sizeof(uint64_t)) != hipSuccess) {
        (void)hipFree(w.partials);
        (void)hipFree(w.counters);
        (void)hipFree(w.xb);
        return set_error(HALO_MI_E_MEMORY, "gemv: cannot allocate the split-K slots");
    }
    hipLaunchKernelGGL(k_fill_u32, dim3((uint32_t)(kCounters / 256)), dim3(256), 0, st, w.counters, kCounters, 0u);
    hipLaunchKernelGGL(k_fill_u32, dim3((uint32_t)(2 * kSlots / 256)), dim3(256), 0, st,
                       reinterpret_cast<uint32_t*>(w.slots), 2 * kSlots, 0u);
    if (hipGetLastError() != hipSuccess) return set_error(HALO_MI_E_DEVICE, "gemv: workspace init failed");
    *out = &(g_ws[{dev, st}] = w);
    return HALO_MI_OK;
}

// Work split of a slab-GEMV launch: ks K chunks per slab (more than one only when the slabs
// alone cannot fill the chip; the chunks then meet in the workspace), nw waves per workgroup
// (about two slot groups per wave, so each wave streams with one group in flight).
struct GemvSplit {
    uint32_t ks, nw;
};

GemvSplit pick_split(uint32_t slabs, uint32_t S, uint32_t nv, uint32_t mats, bool have_ws) {
    // One slot group per wave for mid-size matrices, two for large ones (measured on MI355X,
    // 17408 x 5120 and 151936 x 5120 Q4_K).
    static const uint32_t target_env = [] {
        const char* e = std::getenv("HALO_MI_GEMV_WGS");  // tuning knob: min workgroups per launch
        return e ? (uint32_t)std::max(1, std::atoi(e)) : 0u;
    }();
    static const int gpw_env = [] {
        const char* e = std::getenv("HALO_MI_GEMV_GPW");  // tuning knob: slot groups per wave
        return e ? std::max(1, std::atoi(e)) : 0;
    }();
    const uint32_t groups_per_wave = gpw_env ? (uint32_t)gpw_env : (slabs >= 1024 ? 2u : 1u);
    const uint32_t ngrp = (S + 7) / 8;
    uint32_t ks = 1;
    const uint32_t units = std::max(slabs, 1u) * mats;
    // Measured on MI355X: about 4 workgroups per slab up to 1088 per launch; small matrices
    // gain more from a short split-K fix-up than from more workgroups (floor of 128).
    const uint32_t target_wg = target_env ? target_env : std::clamp(4 * units, 128u, 1088u);
    if (have_ws && units < target_wg) ks = std::min((target_wg + units - 1) / units, ngrp);
    while (ks > 1 && (uint64_t)slabs * ks * mats * nv * 64 > kSlots) --ks;
    const uint32_t gwg = (ngrp + ks - 1) / ks;
    uint32_t nw = std::clamp((gwg + groups_per_wave - 1) / groups_per_wave, 1u, 16u);
    // a wave holds the x sums of at most 4 groups (one per lane)
    while (ks < ngrp && (gwg + nw - 1) / nw > 4) {
        if (nw < 16) ++nw;
        else ++ks;
        const uint32_t g2 = (ngrp + ks - 1) / ks;
        if ((g2 + nw - 1) / nw <= 4) break;
    }
    return {ks, nw};
}

template <uint32_t T, int NV, bool PAIR>
int launch_gemv_slab_t(GemvSlabArgs a, uint32_t slabs, Workspace* ws, hipStream_t st) {
    const uint32_t S = a.cols / kSlot;
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    const GemvSplit sp = pick_split(slabs, S, NV, MATS, ws != nullptr && slabs <= kCounters);
    a.ks = sp.ks;
    a.slots = ws ? ws->slots : nullptr;
    a.counters = ws ? ws->counters : nullptr;
    static const bool valu = [] {
        const char* e = std::getenv("HALO_MI_GEMV_VALU");
        return e && *e == '1';
    }();
    if (valu) {
        const size_t lds = (size_t)sp.nw * NV * 64 * sizeof(float);
        hipLaunchKernelGGL((k_gemv_slab<T, NV, PAIR>), dim3(slabs * a.ks * MATS), dim3(64 * sp.nw), lds, st, a);
        return hip_status(hipGetLastError(), "gemv_slab launch");
    }
    // MFMA kernel. Below 1024 slabs it runs one slot group per wave: enough K chunks that a
    // chunk's groups fit one workgroup (at most 16 waves, 64 KB of LDS with the waves' A tables).
    const size_t per_wave = NV * 64 * sizeof(float) + mx_table_bytes<NV>();
    const uint32_t ngrp = (S + 7) / 8;
    uint32_t nw1 = mx_max_threads<T, NV, true>() / 64;
    while (nw1 > 1 && nw1 * per_wave > 65536) --nw1;
    if (ws && slabs < 1024 && slabs <= kCounters) {
        uint32_t ks = std::max(a.ks, (ngrp + nw1 - 1) / nw1);
        ks = std::min(ks, ngrp);
        if ((uint64_t)slabs * ks * MATS * NV * 64 <= kSlots) a.ks = ks;
    }
    const uint32_t gwg = (ngrp + a.ks - 1) / a.ks;  // groups of the largest chunk
    if (gwg <= nw1 && (a.ks == 1 || ws)) {
        hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, true>), dim3(slabs * a.ks * MATS), dim3(64 * gwg), gwg * per_wave, st, a);
        return hip_status(hipGetLastError(), "gemv_slab launch");
    }
    uint32_t nw = std::min(sp.nw, mx_max_threads<T, NV, false>() / 64);
    while (nw > 1 && nw * per_wave > 65536) --nw;
    hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, false>), dim3(slabs * a.ks * MATS), dim3(64 * nw), nw * per_wave, st, a);
    return hip_status(hipGetLastError(), "gemv_slab launch");
}

template <uint32_t T, bool PAIR>
int launch_gemv_slab_nv(const GemvSlabArgs& a, uint32_t slabs, Workspace* ws, hipStream_t st) {
    switch (a.n_vec) {
        case 1: return launch_gemv_slab_t<T, 1, PAIR>(a, slabs, ws, st);
        case 2: return launch_gemv_slab_t<T, 2, PAIR>(a, slabs, ws, st);
        case 3: return launch_gemv_slab_t<T, 3, PAIR>(a, slabs, ws, st);
        default: return launch_gemv_slab_t<T, 4, PAIR>(a, slabs, ws, st);
    }
}

template <bool PAIR>
int launch_gemv_slab(uint32_t type, GemvSlabArgs a, hipStream_t st) {
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    // the pair's gate and up sums always meet in the workspace
    if (PAIR && !ws)
        return set_error(HALO_MI_E_MEMORY, "gate_up: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    if (PAIR && slabs > kCounters) return set_error(HALO_MI_E_UNSUPPORTED, "gate_up: %u rows exceed the workspace", a.rows);
    const uint32_t total = a.n_vec;
    for (uint32_t t0 = 0; t0 < total; t0 += kMaxGemvVec) {
        GemvSlabArgs c = a;
        c.n_vec = std::min(kMaxGemvVec, total - t0);
        c.x = a.x + (uint64_t)t0 * a.x_stride;
        c.y = a.y + (uint64_t)t0 * a.y_stride;
        int rc;
        switch (type) {
            case kQ4_0: rc = launch_gemv_slab_nv<kQ4_0, PAIR>(c, slabs, ws, st); break;
            case kQ8_0: rc = launch_gemv_slab_nv<kQ8_0, PAIR>(c, slabs, ws, st); break;
            case kQ4_K: rc = launch_gemv_slab_nv<kQ4_K, PAIR>(c, slabs, ws, st); break;
            default: rc = launch_gemv_slab_nv<kQ6_K, PAIR>(c, slabs, ws, st); break;
        }
        if (rc) return rc;
    }
    return HALO_MI_OK;
}

template <bool PAIR, int MB>
void launch_gemm_pc_type(uint32_t type, const GemmPcArgs& a, dim3 grid, hipStream_t st) {
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL((k_gemm_pc<kQ4_0, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        case kQ8_0: hipLaunchKernelGGL((k_gemm_pc<kQ8_0, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        case kQ4_K: hipLaunchKernelGGL((k_gemm_pc<kQ4_K, PAIR, MB>), grid, dim3(512), 0, st, a); break;
        default: hipLaunchKernelGGL((k_gemm_pc<kQ6_K, PAIR, MB>), grid, dim3(512), 0, st, a); break;
    }
}

// x -> bf16 staging (in chunks of rows that fit the workspace), then the producer/consumer GEMM.
// When the tiles do not fill whole rounds of the chip (e.g. 272 slabs on 256 CUs), the tiles
// past the last whole round are split over K so that the last round is spread over all CUs:
// their fp32 partials go to the workspace and k_gemm_pc_reduce adds them in a fixed order.
template <bool PAIR>
int launch_gemm_pc(uint32_t type, const GemmArgs& a, hipStream_t st) {
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    if (!ws)
        return set_error(HALO_MI_E_MEMORY, "gemm: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    const int MB = a.n_vec <= 64 ? 1 : a.n_vec <= 128 ? 2 : 4;
    const uint32_t BM = 64u * MB;
    const uint64_t cap_rows = kXbElems / a.cols / BM * BM;
    if (cap_rows == 0) return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for the x staging buffer", a.cols);
    if ((uint64_t)BM * a.cols * 2 > 0xFFFFFFFFull)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemm: cols %u too large for one M tile", a.cols);
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    const uint32_t units = PAIR ? slabs : (slabs + 1) / 2;
    const uint32_t S = a.cols / kSlot;
    static const uint32_t cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return (uint32_t)std::max(n, 1);
    }();
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
        const uint64_t n8 = (uint64_t)m_tiles * BM * (a.cols / 8);
        hipLaunchKernelGGL(k_x_to_frag, dim3((uint32_t)((n8 + 255) / 256)), dim3(256), 0, st, a.x + m_start * a.x_stride,
                           a.x_stride, mc, m_tiles * BM, a.cols, ws->xb);
        float* y = a.y + m_start * a.y_stride;
        // whole rounds of tiles, then the rest split over K; a matrix whose tiles cannot fill
        // half the chip is split over K altogether
        const uint64_t tiles = (uint64_t)units * m_tiles;
        uint32_t main_units = units, kc = 1;
        if (S % 8 == 0 && ((tiles > cus && tiles % cus != 0) || 2 * tiles < cus)) {
            main_units = tiles > cus ? (uint32_t)(tiles / cus * cus / m_tiles) : 0u;
            const uint64_t rest = (uint64_t)(units - main_units) * m_tiles;
            kc = (uint32_t)std::min<uint64_t>({cus / std::max<uint64_t>(rest, 1), S / 8, 16});
            while (kc > 1 && rest * kc * BM * kPcW > kPartialFloats) --kc;
            if (kc < 2) main_units = units;  // nothing to gain: one launch
        }
        // one launch: the whole tiles, then the split tiles' chunks (dispatched as CUs free up)
        GemmPcArgs p{a.w0, a.w1, ws->xb, y, a.y_stride, a.rows, a.cols, mc, main_units, m_tiles, 0u,
                     units - main_units, kc, ws->partials};
        p.xcd_map = xcd_ok(main_units, m_tiles);
        launch(p);
        if (p.split_units > 0) {
            const uint64_t outs = (uint64_t)p.split_units * p.m_tiles * BM * (PAIR ? 64 : kPcW);
            const dim3 rg((uint32_t)((outs + 255) / 256));
            switch (MB) {
                case 1: hipLaunchKernelGGL((k_gemm_pc_reduce<PAIR, 64>), rg, dim3(256), 0, st, p); break;
                case 2: hipLaunchKernelGGL((k_gemm_pc_reduce<PAIR, 128>), rg, dim3(256), 0, st, p); break;
                default: hipLaunchKernelGGL((k_gemm_pc_reduce<PAIR, 256>), rg, dim3(256), 0, st, p); break;
            }
        }
        if (int rc = hip_status(hipGetLastError(), "gemm_pc launch")) return rc;
    }
    return HALO_MI_OK;
}

template <bool PAIR>
int launch_gemm_slab(uint32_t type, const GemmArgs& a, hipStream_t st) {
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    const dim3 grid(slabs, (a.n_vec + kGemmBM - 1) / kGemmBM);
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL((k_gemm_slab_bf16<kQ4_0, PAIR>), grid, dim3(256), 0, st, a); break;
        case kQ8_0: hipLaunchKernelGGL((k_gemm_slab_bf16<kQ8_0, PAIR>), grid, dim3(256), 0, st, a); break;
        case kQ4_K: hipLaunchKernelGGL((k_gemm_slab_bf16<kQ4_K, PAIR>), grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((k_gemm_slab_bf16<kQ6_K, PAIR>), grid, dim3(256), 0, st, a); break;
    }
    return hip_status(hipGetLastError(), "gemm_slab launch");
}

// Common checks for the x / y operands of a gemv-shaped call.
int check_xy(const char* op, const float* x, uint64_t x_stride, const float* y, uint64_t y_stride, uint32_t rows,
             uint32_t cols, uint32_t n_vec) {
    if (n_vec == 0 || rows == 0 || cols == 0) return HALO_MI_OK;
    if (!x || !y) return set_error(HALO_MI_E_KERNEL, "%s: operand x or y is empty", op);
    if (n_vec > 1 && x_stride < cols)
        return set_error(HALO_MI_E_KERNEL, "%s: x row stride %llu < %u floats", op, (unsigned long long)x_stride, cols);
    if (n_vec > 1 && y_stride < rows)
        return set_error(HALO_MI_E_KERNEL, "%s: y row stride %llu < %u floats", op, (unsigned long long)y_stride, rows);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: x and y must be 4-byte aligned", op);
    if (ranges_overlap(y, extent(n_vec, y_stride * 4, (uint64_t)rows * 4), x, extent(n_vec, x_stride * 4, (uint64_t)cols * 4)))
        return set_error(HALO_MI_E_KERNEL, "%s: y overlaps x", op);
    return HALO_MI_OK;
}

}  // namespace
}  // namespace halo_mi

using namespace halo_mi;

extern "C" {

int halo_mi_gemv(const halo_mi_gemv_params* p, void* stream) {
    clear_error();
    if (!p) return set_error(HALO_MI_E_KERNEL, "gemv: null params");
    const char* op = "MATMUL";
    int code;
    const uint64_t rb = row_bytes_checked(p->type, p->cols, &code, op);
    if (code) return code;
    uint32_t variant = p->variant;
    if (variant > HALO_MI_GEMV_SLAB_AUTO) return set_error(HALO_MI_E_CONFIG, "%s: unknown kernel variant id %u", op, variant);
    if (variant == HALO_MI_GEMV_DEFAULT)
        variant = p->layout == HALO_MI_LAYOUT_SLAB ? HALO_MI_GEMV_SLAB_AUTO : HALO_MI_GEMV_GGUF_REF;
    const uint64_t xs = p->x_stride ? p->x_stride : p->cols;
    const uint64_t ys = p->y_stride ? p->y_stride : p->rows;
    if ((code = check_xy(op, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec))) return code;
    if (p->n_vec == 0 || p->rows == 0) return HALO_MI_OK;
    if (!p->w) return set_error(HALO_MI_E_KERNEL, "%s: operand w is empty", op);
    auto st = static_cast<hipStream_t>(stream);
    const uint64_t yext = extent(p->n_vec, ys * 4, (uint64_t)p->rows * 4);
    if (variant == HALO_MI_GEMV_GGUF_REF) {
        if (p->layout != HALO_MI_LAYOUT_GGUF)
            return set_error(HALO_MI_E_CONFIG, "%s: variant %u needs the GGUF layout", op, variant);
        const uint64_t ws = p->w_stride ? p->w_stride : rb;
        if (p->rows > 1 && ws < rb)
            return set_error(HALO_MI_E_KERNEL, "%s: operand w row stride %llu < row bytes %llu", op, (unsigned long long)ws,
                             (unsigned long long)rb);
        if (p->type == kF32 && ((reinterpret_cast<uintptr_t>(p->w) | ws) % 4))
            return set_error(HALO_MI_E_KERNEL, "%s: operand w is not 4-byte aligned", op);
        if (ranges_overlap(p->y, yext, p->w, extent(p->rows, ws, rb))) return set_error(HALO_MI_E_KERNEL, "%s: y overlaps w", op);
        hipLaunchKernelGGL(k_gemv_gguf_ref, dim3((p->rows + 31) / 32), dim3(256), 0, st, p->type,
                           static_cast<const uint8_t*>(p->w), ws, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec);
        return hip_status(hipGetLastError(), "gemv_gguf_ref launch");
    }
    if (p->layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: variant %u needs the SLAB layout", op, variant);
    if (!is_quant(p->type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, p->type);
    if (p->w_stride != 0) return set_error(HALO_MI_E_KERNEL, "%s: a SLAB operand has no row stride", op);
    if (reinterpret_cast<uintptr_t>(p->w) % 16) return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
    if (ranges_overlap(p->y, yext, p->w, halo_mi_slab_bytes(p->type, p->rows, p->cols)))
        return set_error(HALO_MI_E_KERNEL, "%s: y overlaps w", op);
    if (variant == HALO_MI_GEMV_SLAB_AUTO) variant = p->n_vec <= 8 ? HALO_MI_GEMV_SLAB : HALO_MI_GEMM_SLAB_BF16;
    if (variant == HALO_MI_GEMV_SLAB) {
        GemvSlabArgs a{static_cast<const uint8_t*>(p->w), nullptr, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec};
        return launch_gemv_slab<false>(p->type, a, st);
    }
    if (p->x_stride % 4 || reinterpret_cast<uintptr_t>(p->x) % 16)
        return set_error(HALO_MI_E_KERNEL, "%s: the MFMA GEMM needs 16-byte aligned x rows", op);
    GemmArgs a{static_cast<const uint8_t*>(p->w), nullptr, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec};
    return launch_gemm_pc<false>(p->type, a, st);
}

int halo_mi_gate_up_swiglu(const halo_mi_gate_up_params* p, void* stream) {
    clear_error();
    if (!p) return set_error(HALO_MI_E_KERNEL, "gate_up: null params");
    const char* op = "GATE_UP_SWIGLU";
    int code;
    (void)row_bytes_checked(p->type, p->cols, &code, op);
    if (code) return code;
    if (p->layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: needs the SLAB layout", op);
    if (!is_quant(p->type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, p->type);
    uint32_t variant = p->variant;
    if (variant == HALO_MI_GEMV_GGUF_REF || variant > HALO_MI_GEMV_SLAB_AUTO)
        return set_error(HALO_MI_E_CONFIG, "%s: unknown kernel variant id %u", op, variant);
    const uint64_t xs = p->x_stride ? p->x_stride : p->cols;
    const uint64_t os = p->out_stride ? p->out_stride : p->rows;
    if ((code = check_xy(op, p->x, xs, p->out, os, p->rows, p->cols, p->n_vec))) return code;
    if (p->n_vec == 0 || p->rows == 0) return HALO_MI_OK;
    if (!p->w_gate || !p->w_up) return set_error(HALO_MI_E_KERNEL, "%s: operand w_gate or w_up is empty", op);
    if ((reinterpret_cast<uintptr_t>(p->w_gate) | reinterpret_cast<uintptr_t>(p->w_up)) % 16)
        return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
    const uint64_t wbytes = halo_mi_slab_bytes(p->type, p->rows, p->cols);
    const uint64_t oext = extent(p->n_vec, os * 4, (uint64_t)p->rows * 4);
    if (ranges_overlap(p->out, oext, p->w_gate, wbytes) || ranges_overlap(p->out, oext, p->w_up, wbytes))
        return set_error(HALO_MI_E_KERNEL, "%s: out overlaps a weight operand", op);
    if (variant == HALO_MI_GEMV_DEFAULT || variant == HALO_MI_GEMV_SLAB_AUTO)
        variant = p->n_vec <= kGateUpGemvMax ? HALO_MI_GEMV_SLAB : HALO_MI_GEMM_SLAB_BF16;
    auto st = static_cast<hipStream_t>(stream);
    if (variant == HALO_MI_GEMV_SLAB) {
        GemvSlabArgs a{static_cast<const uint8_t*>(p->w_gate), static_cast<const uint8_t*>(p->w_up), p->x, xs, p->out, os,
                       p->rows, p->cols, p->n_vec};
        return launch_gemv_slab<true>(p->type, a, st);
    }
    if (xs % 4 || reinterpret_cast<uintptr_t>(p->x) % 16)
        return set_error(HALO_MI_E_KERNEL, "%s: the MFMA GEMM needs 16-byte aligned x rows", op);
    GemmArgs a{static_cast<const uint8_t*>(p->w_gate), static_cast<const uint8_t*>(p->w_up), p->x, xs, p->out, os,
               p->rows, p->cols, p->n_vec};
    return launch_gemm_pc<true>(p->type, a, st);
}

int halo_mi_swiglu(const float* gate, uint64_t gate_stride, const float* up, uint64_t up_stride, float* out,
                   uint64_t out_stride, uint32_t rows, uint32_t cols, void* stream) {
    clear_error();
    const char* op = "SWIGLU";
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    if (!gate || !up || !out) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (gate_stride == 0) gate_stride = cols;
    if (up_stride == 0) up_stride = cols;
    if (out_stride == 0) out_stride = cols;
    if (rows > 1 && (gate_stride < cols || up_stride < cols || out_stride < cols))
        return set_error(HALO_MI_E_KERNEL, "%s: row stride < cols", op);
    if ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(out)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: operands must be 4-byte aligned", op);
    const uint64_t oext = extent(rows, out_stride * 4, (uint64_t)cols * 4);
    if (ranges_overlap(out, oext, gate, extent(rows, gate_stride * 4, (uint64_t)cols * 4)) ||
        ranges_overlap(out, oext, up, extent(rows, up_stride * 4, (uint64_t)cols * 4)))
        return set_error(HALO_MI_E_KERNEL, "%s: out overlaps an input", op);
    const uint64_t n = (uint64_t)rows * cols;
    hipLaunchKernelGGL(k_swiglu, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream), gate,
                       gate_stride, up, up_stride, out, out_stride, rows, cols);
    return hip_status(hipGetLastError(), "swiglu launch");
}

int halo_mi_dequant_rows(uint32_t type, uint32_t layout, const void* w, uint64_t w_stride, uint32_t rows, uint32_t cols,
                         uint32_t first_row, uint32_t n_rows, float* out, uint64_t out_stride, void* stream) {
    clear_error();
    const char* op = "DEQUANT";
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, op);
    if (code) return code;
    if (first_row > rows || n_rows > rows - first_row)
        return set_error(HALO_MI_E_KERNEL, "%s: rows [%u, %u) out of %u", op, first_row, first_row + n_rows, rows);
    if (n_rows == 0 || cols == 0) return HALO_MI_OK;
    if (!w || !out) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (out_stride == 0) out_stride = cols;
    if (n_rows > 1 && out_stride < cols) return set_error(HALO_MI_E_KERNEL, "%s: out stride < cols", op);
    auto st = static_cast<hipStream_t>(stream);
    if (layout == HALO_MI_LAYOUT_GGUF) {
        if (w_stride == 0) w_stride = rb;
        if (rows > 1 && w_stride < rb) return set_error(HALO_MI_E_KERNEL, "%s: w stride < row bytes", op);
        const uint64_t n = (uint64_t)n_rows * cols;
        hipLaunchKernelGGL(k_dequant_gguf, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, type,
                           static_cast<const uint8_t*>(w), w_stride, cols, first_row, n_rows, out, out_stride);
        return hip_status(hipGetLastError(), "dequant_gguf launch");
    }
    if (layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: unknown layout %u", op, layout);
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, type);
    const uint64_t n = (uint64_t)n_rows * (cols / kSlot);
    const dim3 grid((uint32_t)((n + 255) / 256)), block(256);
    const auto* wb = static_cast<const uint8_t*>(w);
    switch (type) {
        case kQ4_0: hipLaunchKernelGGL(k_dequant_slab<kQ4_0>, grid, block, 0, st, wb, cols, first_row, n_rows, out, out_stride); break;
        case kQ8_0: hipLaunchKernelGGL(k_dequant_slab<kQ8_0>, grid, block, 0, st, wb, cols, first_row, n_rows, out, out_stride); break;
        case kQ4_K: hipLaunchKernelGGL(k_dequant_slab<kQ4_K>, grid, block, 0, st, wb, cols, first_row, n_rows, out, out_stride); break;
        default: hipLaunchKernelGGL(k_dequant_slab<kQ6_K>, grid, block, 0, st, wb, cols, first_row, n_rows, out, out_stride); break;
    }
    return hip_status(hipGetLastError(), "dequant_slab launch");
}

int halo_mi_repack_slab(uint32_t type, const void* src, uint64_t src_stride, uint32_t rows, uint32_t cols, void* dst,
                        void* stream) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "repack_slab");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "repack_slab: type %u has no SLAB layout", type);
    if (src_stride == 0) src_stride = rb;
    if (rows > 1 && src_stride < rb) return set_error(HALO_MI_E_KERNEL, "repack_slab: row stride < row bytes");
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    if (ranges_overlap(dst, halo_mi_slab_bytes(type, rows, cols), src, extent(rows, src_stride, rb)))
        return set_error(HALO_MI_E_KERNEL, "repack_slab: dst overlaps src");
    const uint64_t n = (uint64_t)(rows + kSlabRows - 1) / kSlabRows * kSlabRows * (cols / block_elems(type));
    hipLaunchKernelGGL(k_repack_slab, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream), type,
                       static_cast<const uint8_t*>(src), src_stride, rows, cols, static_cast<uint8_t*>(dst));
    return hip_status(hipGetLastError(), "repack_slab launch");
}

int halo_mi_unpack_slab(uint32_t type, const void* src, uint32_t rows, uint32_t cols, void* dst, uint64_t dst_stride,
                        void* stream) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "unpack_slab");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "unpack_slab: type %u has no SLAB layout", type);
    if (dst_stride == 0) dst_stride = rb;
    if (rows > 1 && dst_stride < rb) return set_error(HALO_MI_E_KERNEL, "unpack_slab: row stride < row bytes");
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    const uint64_t n = (uint64_t)rows * (cols / block_elems(type));
    hipLaunchKernelGGL(k_unpack_slab, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream), type,
                       static_cast<const uint8_t*>(src), rows, cols, static_cast<uint8_t*>(dst), dst_stride);
    return hip_status(hipGetLastError(), "unpack_slab launch");
}

int halo_mi_upload_slab(uint32_t type, const void* host_src, uint64_t src_stride, uint32_t rows, uint32_t cols, void* dst,
                        uint64_t chunk_bytes, void* stream) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "upload_slab");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "upload_slab: type %u has no SLAB layout", type);
    if (src_stride == 0) src_stride = rb;
    if (rows > 1 && src_stride < rb) return set_error(HALO_MI_E_KERNEL, "upload_slab: row stride < row bytes");
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    if (chunk_bytes == 0) chunk_bytes = 64ull << 20;
    // Chunks are whole slabs so every repack writes complete slabs.
    uint64_t chunk_rows = std::max<uint64_t>(chunk_bytes / rb / kSlabRows, 1) * kSlabRows;
    chunk_rows = std::min<uint64_t>(chunk_rows, (uint64_t)(rows + kSlabRows - 1) / kSlabRows * kSlabRows);
    auto st = static_cast<hipStream_t>(stream);
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, chunk_rows * rb);
    if (e != hipSuccess) return set_error(HALO_MI_E_MEMORY, "upload_slab: cannot allocate %llu staging bytes",
                                          (unsigned long long)(chunk_rows * rb));
    const SlabGeom g = slab_geom(type, cols);
    const auto* src = static_cast<const uint8_t*>(host_src);
    int rc = HALO_MI_OK;
    for (uint64_t r0 = 0; r0 < rows && rc == HALO_MI_OK; r0 += chunk_rows) {
        const uint32_t n = (uint32_t)std::min<uint64_t>(chunk_rows, rows - r0);
        if (src_stride == rb) e = hipMemcpyAsync(staging, src + r0 * rb, (uint64_t)n * rb, hipMemcpyHostToDevice, st);
        else e = hipMemcpy2DAsync(staging, rb, src + r0 * src_stride, src_stride, rb, n, hipMemcpyHostToDevice, st);
        if (e != hipSuccess) { rc = hip_status(e, "upload_slab copy"); break; }
        rc = halo_mi_repack_slab(type, staging, rb, n, cols, static_cast<uint8_t*>(dst) + (r0 / kSlabRows) * g.slab_bytes, st);
        if (rc == HALO_MI_OK) {
            e = hipStreamSynchronize(st);  // the staging buffer is reused by the next chunk
            if (e != hipSuccess) rc = hip_status(e, "upload_slab sync");
        }
    }
    (void)hipFree(staging);
    return rc;
}

}  // extern "C"
