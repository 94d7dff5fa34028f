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
#include <cstring>

#include "common.h"
#include "decode.h"
#include "slab_layout.h"

namespace halo_mi {
namespace {

using namespace dev;

constexpr uint32_t kMaxGemvVec = 4;  // vectors per slab-gemv launch

typedef __attribute__((address_space(4))) const float cfloat;  // constant address space
constexpr uint32_t kMaxWaves = 16;   // waves per workgroup

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ float ubyte(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sbyte(uint32_t v, int k) { return (float)(int)(int8_t)((v >> (8 * k)) & 0xFFu); }

// ==========================================================================================
// Repack / unpack / dequantize
// ==========================================================================================

__global__ void k_repack_slab(uint32_t type, const uint8_t* __restrict__ src, uint64_t src_stride, uint32_t rows,
                              uint32_t cols, uint8_t* __restrict__ dst) {
    const SlabGeom g = slab_geom(type, cols);
    const uint32_t nblk = cols / block_elems(type), S = cols / kSlot;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t padded = (uint64_t)(rows + kSlabRows - 1) / kSlabRows * kSlabRows;
    if (idx >= padded * nblk) return;
    const uint64_t row = idx / nblk;
    const uint32_t b = (uint32_t)(idx % nblk);
    uint8_t blk[210];
    const uint32_t bb = block_bytes(type);
    if (row < rows) {
        const uint8_t* s = src + row * src_stride + (uint64_t)b * bb;
        for (uint32_t i = 0; i < bb; ++i) blk[i] = s[i];
    } else {
        for (uint32_t i = 0; i < bb; ++i) blk[i] = 0;
    }
    slab_pack_block(type, blk, dst + (row / kSlabRows) * g.slab_bytes, g, S, (uint32_t)(row % kSlabRows), b);
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
// SLAB GEMV: one row per lane, K split over the waves of the workgroup
// ==========================================================================================

struct GemvSlabArgs {
    const uint8_t* w0;  // slab image (gate, or the only matrix)
    const uint8_t* w1;  // up matrix (PAIR) or null
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
    uint32_t rows, cols, n_vec;
};

// 16 low-nibble and 16 high-nibble weights of a 4-bit slot record against x[0..31]:
// lo = sum x[t] q_lo[t], hi = sum x[16+t] (16 q_hi[t]) (the high nibbles are left in place,
// i.e. scaled by 16, and rescaled by the caller).
__device__ __forceinline__ void dot_nibbles(const uint4& q, cfloat* xs, float& lo, float& hi) {
    const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = Q[i] & 0x0F0F0F0Fu, b = Q[i] & 0xF0F0F0F0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            lo = fmaf(xs[4 * i + k], ubyte(a, k), lo);
            hi = fmaf(xs[16 + 4 * i + k], ubyte(b, k), hi);
        }
    }
}

// One slot (32 weights) of one row for NV x vectors, added to acc[]. xsum = LDS sums of the
// two 16-element halves of every slot of every vector: xsum[(v * S + s) * 2 + h].
template <uint32_t T, int NV>
__device__ __forceinline__ void slab_slot_gemv(const uint8_t* __restrict__ slab, const SlabGeom& g, uint32_t lane,
                                               uint32_t s, cfloat* x, uint64_t x_stride,
                                               const float* xsum, uint32_t S, float acc[NV]) {
    if constexpr (T == kQ4_K) {
        const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + lane) * 16);
        const uint4 hdr = *reinterpret_cast<const uint4*>(slab + g.aux_off + ((uint64_t)(s >> 3) * 64 + lane) * 16);
        float d1, m1;
        q4k_scales(hdr, s & 7u, d1, m1);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            cfloat* xs = x + v * x_stride + (uint64_t)s * 32;
            float lo = 0.0f, hi = 0.0f;
            dot_nibbles(q, xs, lo, hi);
            const float sq = fmaf(hi, 0.0625f, lo);
            const float X = xsum[(v * S + s) * 2] + xsum[(v * S + s) * 2 + 1];
            acc[v] = fmaf(d1, sq, acc[v]);
            acc[v] = fmaf(-m1, X, acc[v]);
        }
    } else if constexpr (T == kQ4_0) {
        const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + lane) * 16);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(slab + g.aux_off + ((uint64_t)s * 64 + lane) * 2));
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            cfloat* xs = x + v * x_stride + (uint64_t)s * 32;
            float lo = 0.0f, hi = 0.0f;
            dot_nibbles(q, xs, lo, hi);
            const float X = xsum[(v * S + s) * 2] + xsum[(v * S + s) * 2 + 1];
            float t = fmaf(hi, 0.0625f, lo);
            t = fmaf(-8.0f, X, t);
            acc[v] = fmaf(d, t, acc[v]);
        }
    } else if constexpr (T == kQ8_0) {
        const uint4 qa = *reinterpret_cast<const uint4*>(slab + g.q_off + (((uint64_t)s * 2) * 64 + lane) * 16);
        const uint4 qb = *reinterpret_cast<const uint4*>(slab + g.q_off + (((uint64_t)s * 2 + 1) * 64 + lane) * 16);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(slab + g.aux_off + ((uint64_t)s * 64 + lane) * 2));
        const uint32_t A[4] = {qa.x, qa.y, qa.z, qa.w}, B[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            cfloat* xs = x + v * x_stride + (uint64_t)s * 32;
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    lo = fmaf(xs[4 * i + k], sbyte(A[i], k), lo);
                    hi = fmaf(xs[16 + 4 * i + k], sbyte(B[i], k), hi);
                }
            acc[v] = fmaf(d, lo + hi, acc[v]);
        }
    } else {  // Q6_K
        const uint4 ql = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + lane) * 16);
        const uint2 qh = *reinterpret_cast<const uint2*>(slab + g.aux_off + ((uint64_t)s * 64 + lane) * 8);
        const uint32_t sb = s >> 3, j = s & 7u;
        const uint4 sc4 = *reinterpret_cast<const uint4*>(slab + g.sc_off + ((uint64_t)sb * 64 + lane) * 16);
        const float d = h2f(*reinterpret_cast<const uint16_t*>(slab + g.d_off + ((uint64_t)sb * 64 + lane) * 2));
        const uint32_t SC[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
        const uint32_t scw = SC[j >> 1];
        const float dA = d * sbyte(scw, 2 * (j & 1)), dB = d * sbyte(scw, 2 * (j & 1) + 1);
        uint32_t lo6[4], hi6[4];
        q6_slot_bytes(ql, qh, lo6, hi6);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            cfloat* xs = x + v * x_stride + (uint64_t)s * 32;
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    lo = fmaf(xs[4 * i + k], ubyte(lo6[i], k), lo);
                    hi = fmaf(xs[16 + 4 * i + k], ubyte(hi6[i], k), hi);
                }
            const float ta = fmaf(-32.0f, xsum[(v * S + s) * 2], lo);
            const float tb = fmaf(-32.0f, xsum[(v * S + s) * 2 + 1], hi);
            acc[v] = fmaf(dA, ta, acc[v]);
            acc[v] = fmaf(dB, tb, acc[v]);
        }
    }
}

// grid.x = slabs; block = 64 * waves. LDS: xsum [NV][S][2], red [waves][NV * (PAIR ? 2 : 1)][64].
template <uint32_t T, int NV, bool PAIR>
__global__ __launch_bounds__(1024) void k_gemv_slab(GemvSlabArgs a) {
    extern __shared__ float smem[];
    const uint32_t S = a.cols / kSlot;
    // wave index via readfirstlane so the compiler knows it (and the slot loop) is uniform
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = blockDim.x >> 6;
    float* xsum = smem;
    float* red = smem + NV * S * 2;
    // x is read-only and wave-uniform in the main loop: reading it through the constant
    // address space lets the compiler use scalar loads (x lands in SGPRs, no VGPR cost).
    cfloat* x = reinterpret_cast<cfloat*>(reinterpret_cast<uintptr_t>(a.x));
    for (uint32_t i = threadIdx.x; i < NV * S * 2; i += blockDim.x) {
        const uint32_t v = i / (S * 2), r = i % (S * 2);
        const float* xp = a.x + v * a.x_stride + (uint64_t)r * 16;
        float sum = 0.0f;
        for (int k = 0; k < 16; ++k) sum += xp[k];
        xsum[i] = sum;
    }
    __syncthreads();
    const uint32_t base = S / nw, extra = S % nw;
    const uint32_t s0 = wave * base + min(wave, extra);
    const uint32_t s1 = s0 + base + (wave < extra ? 1u : 0u);
    const SlabGeom g = slab_geom(T, a.cols);
    const uint8_t* slab0 = a.w0 + (uint64_t)blockIdx.x * g.slab_bytes;
    float acc0[NV], acc1[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc0[v] = acc1[v] = 0.0f;
    if constexpr (PAIR) {
        const uint8_t* slab1 = a.w1 + (uint64_t)blockIdx.x * g.slab_bytes;
#pragma unroll 2
        for (uint32_t s = s0; s < s1; ++s) {
            slab_slot_gemv<T, NV>(slab0, g, lane, s, x, a.x_stride, xsum, S, acc0);
            slab_slot_gemv<T, NV>(slab1, g, lane, s, x, a.x_stride, xsum, S, acc1);
        }
    } else {
#pragma unroll 4
        for (uint32_t s = s0; s < s1; ++s) slab_slot_gemv<T, NV>(slab0, g, lane, s, x, a.x_stride, xsum, S, acc0);
    }
    constexpr int NA = PAIR ? 2 * NV : NV;
    if (nw > 1) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            red[(wave * NA + v) * 64 + lane] = acc0[v];
            if constexpr (PAIR) red[(wave * NA + NV + v) * 64 + lane] = acc1[v];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            float s = red[v * 64 + lane], u = PAIR ? red[(NV + v) * 64 + lane] : 0.0f;
            for (uint32_t w = 1; w < nw; ++w) {
                s += red[(w * NA + v) * 64 + lane];
                if constexpr (PAIR) u += red[(w * NA + NV + v) * 64 + lane];
            }
            acc0[v] = s;
            acc1[v] = u;
        }
    }
    const uint32_t row = blockIdx.x * kSlabRows + lane;
    if (row >= a.rows) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        if ((uint32_t)v >= a.n_vec) break;
        a.y[(uint64_t)v * a.y_stride + row] = PAIR ? silu_f(acc0[v]) * acc1[v] : acc0[v];
    }
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

uint32_t pick_waves(uint32_t slabs, uint32_t S) {
    // Aim for about 2048 waves in flight over the chip (256 CUs), at most 16 per workgroup.
    uint32_t nw = (2048u + slabs - 1) / std::max(slabs, 1u);
    nw = std::clamp(nw, 1u, kMaxWaves);
    return std::min(nw, std::max(S, 1u));
}

template <uint32_t T, int NV, bool PAIR>
int launch_gemv_slab_t(const GemvSlabArgs& a, uint32_t slabs, hipStream_t st) {
    const uint32_t S = a.cols / kSlot;
    const uint32_t nw = pick_waves(slabs, S);
    const size_t lds = ((size_t)NV * S * 2 + (size_t)nw * NV * (PAIR ? 2 : 1) * 64) * sizeof(float);
    if (lds > 160 * 1024) return set_error(HALO_MI_E_UNSUPPORTED, "gemv_slab: %u columns need %zu B of LDS", a.cols, lds);
    hipLaunchKernelGGL((k_gemv_slab<T, NV, PAIR>), dim3(slabs), dim3(64 * nw), lds, st, a);
    return hip_status(hipGetLastError(), "gemv_slab launch");
}

template <uint32_t T, bool PAIR>
int launch_gemv_slab_nv(const GemvSlabArgs& a, uint32_t slabs, hipStream_t st) {
    switch (a.n_vec) {
        case 1: return launch_gemv_slab_t<T, 1, PAIR>(a, slabs, st);
        case 2: return launch_gemv_slab_t<T, 2, PAIR>(a, slabs, st);
        case 3: return launch_gemv_slab_t<T, 3, PAIR>(a, slabs, st);
        default: return launch_gemv_slab_t<T, 4, PAIR>(a, slabs, st);
    }
}

template <bool PAIR>
int launch_gemv_slab(uint32_t type, GemvSlabArgs a, hipStream_t st) {
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    const uint32_t total = a.n_vec;
    for (uint32_t t0 = 0; t0 < total; t0 += kMaxGemvVec) {
        GemvSlabArgs c = a;
        c.n_vec = std::min(kMaxGemvVec, total - t0);
        c.x = a.x + (uint64_t)t0 * a.x_stride;
        c.y = a.y + (uint64_t)t0 * a.y_stride;
        int rc;
        switch (type) {
            case kQ4_0: rc = launch_gemv_slab_nv<kQ4_0, PAIR>(c, slabs, st); break;
            case kQ8_0: rc = launch_gemv_slab_nv<kQ8_0, PAIR>(c, slabs, st); break;
            case kQ4_K: rc = launch_gemv_slab_nv<kQ4_K, PAIR>(c, slabs, st); break;
            default: rc = launch_gemv_slab_nv<kQ6_K, PAIR>(c, slabs, st); break;
        }
        if (rc) return rc;
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
    return launch_gemm_slab<false>(p->type, a, st);
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
        variant = p->n_vec <= 8 ? HALO_MI_GEMV_SLAB : HALO_MI_GEMM_SLAB_BF16;
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
    return launch_gemm_slab<true>(p->type, a, st);
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
