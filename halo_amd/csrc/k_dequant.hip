// gfx950 kernels of the halo_mi355x library: GGUF <-> SLAB repack, exact dequantization
// (bit-identical to tensor::dequantize_row, src/tensor/quant.cpp:430-435 of the reference) and
// a fill kernel for workspace initialisation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "device.h"
#include "launch.h"

namespace halo_mi {
namespace {

using namespace dev;

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

// The table row of output row r: first_row + r, or ids[r] (GET_ROWS). An id outside the table
// returns false, and the thread of the row's first element reports it in *status.
__device__ __forceinline__ bool table_row(const int32_t* ids, uint32_t table_rows, uint32_t first_row, uint64_t r,
                                          bool first, uint32_t* status, uint64_t& row) {
    if (!ids) {
        row = first_row + r;
        return true;
    }
    const int32_t id = ids[r];
    if (id < 0 || (uint32_t)id >= table_rows) {
        if (first && status) atomicOr(status, kStatusBadIndex);
        return false;
    }
    row = (uint64_t)id;
    return true;
}

__global__ void k_dequant_gguf(uint32_t type, const uint8_t* __restrict__ w, uint64_t w_stride, uint32_t cols,
                               uint32_t first_row, uint32_t n_rows, float* __restrict__ out, uint64_t out_stride,
                               const int32_t* __restrict__ ids, uint32_t table_rows, uint32_t* status) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)n_rows * cols) return;
    const uint64_t r = idx / cols;
    const uint32_t i = (uint32_t)(idx % cols);
    uint64_t row;
    if (!table_row(ids, table_rows, first_row, r, i == 0, status, row)) return;
    out[r * out_stride + i] = gguf_elem(type, w + row * w_stride, i);
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
    } else if constexpr (T == kQ5_K) {
        const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + r) * 16);
        const uint32_t qh = *reinterpret_cast<const uint32_t*>(slab + g.aux_off + ((uint64_t)s * 64 + r) * 4);
        const uint4 hdr = *reinterpret_cast<const uint4*>(slab + g.sc_off + ((uint64_t)(s / 8) * 64 + r) * 16);
        float d1, m1;
        q4k_scales(hdr, s % 8, d1, m1);
        const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (Q[i] & 0x0F0F0F0Fu) | ((qh << (4 - i)) & 0x10101010u);
            const uint32_t hi = ((Q[i] >> 4) & 0x0F0F0F0Fu) | ((qh >> i) & 0x10101010u);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w[4 * i + k] = d1 * ubyte(lo, k) - m1;
                w[16 + 4 * i + k] = d1 * ubyte(hi, k) - m1;
            }
        }
    } else if constexpr (T == kIQ4_XS) {
        const uint4 q = *reinterpret_cast<const uint4*>(slab + g.q_off + ((uint64_t)s * 64 + r) * 16);
        const uint2 hdr = *reinterpret_cast<const uint2*>(slab + g.aux_off + ((uint64_t)(s / 8) * 64 + r) * 8);
        const float dl = h2f((uint16_t)(hdr.x & 0xFFFFu)) * (float)iq4xs_ls(hdr.x >> 16, hdr.y, s % 8);
        const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = iq4_lookup4(Q[i]), hi = iq4_lookup4(Q[i] >> 4);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w[4 * i + k] = dl * (ubyte(lo, k) - 128.0f);
                w[16 + 4 * i + k] = dl * (ubyte(hi, k) - 128.0f);
            }
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
                               float* __restrict__ out, uint64_t out_stride, const int32_t* __restrict__ ids,
                               uint32_t table_rows, uint32_t* status) {
    const SlabGeom g = slab_geom(T, cols);
    const uint32_t S = cols / kSlot;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)n_rows * S) return;
    const uint32_t s = (uint32_t)(idx % S);
    uint64_t row;
    if (!table_row(ids, table_rows, first_row, idx / S, s == 0, status, row)) return;
    float wv[32];
    slab_slot_weights<T>(w + (row / kSlabRows) * g.slab_bytes, g, (uint32_t)(row % kSlabRows), s, wv);
    float* o = out + (idx / S) * out_stride + (uint64_t)s * 32;
    for (int i = 0; i < 32; ++i) o[i] = wv[i];
}

__global__ void k_fill_u32(uint32_t* p, uint64_t n, uint32_t v) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// The read floor: a plain stream over n16 16-byte words, U nontemporal loads in flight per
// thread, grid-stride. The words are folded into one value per thread that is stored only if it
// equals a constant no input here produces, so the loads stay and nothing is written.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const u32x4_t* __restrict__ p, uint64_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * 256 * U;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 * U + threadIdx.x; i < n16; i += stride) {
        u32x4_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t k = i + (uint64_t)u * 256;
            v[u] = __builtin_nontemporal_load(p + (k < n16 ? k : n16 - 1));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x * 256 + threadIdx.x] = acc;
}
}  // namespace

int launch_stream_read(const void* p, uint64_t bytes, uint32_t workgroups, uint32_t unroll, uint32_t* sink, hipStream_t st) {
    const uint64_t n16 = bytes / 16;
    const dim3 grid(workgroups), block(256);
    switch (unroll) {
        case 2: hipLaunchKernelGGL(k_stream_read<2>, grid, block, 0, st, static_cast<const u32x4_t*>(p), n16, sink); break;
        case 4: hipLaunchKernelGGL(k_stream_read<4>, grid, block, 0, st, static_cast<const u32x4_t*>(p), n16, sink); break;
        case 8: hipLaunchKernelGGL(k_stream_read<8>, grid, block, 0, st, static_cast<const u32x4_t*>(p), n16, sink); break;
        default: hipLaunchKernelGGL(k_stream_read<16>, grid, block, 0, st, static_cast<const u32x4_t*>(p), n16, sink); break;
    }
    return hip_status(hipGetLastError(), "stream_read launch");
}

int launch_repack_slab(uint32_t type, const uint8_t* src, uint64_t src_stride, uint32_t rows, uint32_t cols,
                       uint8_t* dst, hipStream_t st) {
    const uint64_t n = (uint64_t)(rows + kSlabRows - 1) / kSlabRows * kSlabRows * (cols / block_elems(type));
    hipLaunchKernelGGL(k_repack_slab, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, type, src, src_stride, rows,
                       cols, dst);
    return hip_status(hipGetLastError(), "repack_slab launch");
}

int launch_unpack_slab(uint32_t type, const uint8_t* src, uint32_t rows, uint32_t cols, uint8_t* dst,
                       uint64_t dst_stride, hipStream_t st) {
    const uint64_t n = (uint64_t)rows * (cols / block_elems(type));
    hipLaunchKernelGGL(k_unpack_slab, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, type, src, rows, cols, dst,
                       dst_stride);
    return hip_status(hipGetLastError(), "unpack_slab launch");
}

int launch_dequant_gguf(uint32_t type, const uint8_t* w, uint64_t w_stride, uint32_t cols, uint32_t first_row,
                        uint32_t n_rows, float* out, uint64_t out_stride, hipStream_t st, const int32_t* ids,
                        uint32_t table_rows, uint32_t* status) {
    const uint64_t n = (uint64_t)n_rows * cols;
    hipLaunchKernelGGL(k_dequant_gguf, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, type, w, w_stride, cols,
                       first_row, n_rows, out, out_stride, ids, table_rows, status);
    return hip_status(hipGetLastError(), "dequant_gguf launch");
}

int launch_dequant_slab(uint32_t type, const uint8_t* w, uint32_t cols, uint32_t first_row, uint32_t n_rows, float* out,
                        uint64_t out_stride, hipStream_t st, const int32_t* ids, uint32_t table_rows, uint32_t* status) {
    const uint64_t n = (uint64_t)n_rows * (cols / kSlot);
    const dim3 grid((uint32_t)((n + 255) / 256)), block(256);
#define HALO_MI_DQ(T) hipLaunchKernelGGL(k_dequant_slab<T>, grid, block, 0, st, w, cols, first_row, n_rows, out, out_stride, ids, table_rows, status)
    switch (type) {
        case kQ4_0: HALO_MI_DQ(kQ4_0); break;
        case kQ8_0: HALO_MI_DQ(kQ8_0); break;
        case kQ4_K: HALO_MI_DQ(kQ4_K); break;
        case kQ5_K: HALO_MI_DQ(kQ5_K); break;
        case kIQ4_XS: HALO_MI_DQ(kIQ4_XS); break;
        default: HALO_MI_DQ(kQ6_K); break;
    }
#undef HALO_MI_DQ
    return hip_status(hipGetLastError(), "dequant_slab launch");
}

int launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t st) {
    hipLaunchKernelGGL(k_fill_u32, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, p, n, v);
    return hip_status(hipGetLastError(), "fill launch");
}

}  // namespace halo_mi
