// gfx950 kernels of the RMS norm in front of the matmul (cpu::rms_norm,
// backends/cpu/ops_basic.cpp:18-33 of the reference):
//   mean = dot(x, x) / cols   (cpu::detail::dot, backends/cpu/kernel_common.h:16-27)
//   inv  = 1 / sqrt(mean + eps)
//   out  = (x * inv) * w
// Both kernels compute the sum of squares in the CPU's order, so the results are bitwise the
// CPU's: k_rms_norm_rows writes the normalized rows (the reference-order GEMV's input, and the
// RMS_NORM op itself); k_rms_inv_rows writes only inv per row, for the GEMM's x staging.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device.h"
#include "launch.h"
#include "norm_device.h"

namespace halo_mi {
namespace {

constexpr uint32_t kNormBlock = 256;
constexpr uint32_t kNormChunk = 8192;               // floats of a row staged in LDS at a time
constexpr uint32_t kPerThread = kNormChunk / kNormBlock;
constexpr uint32_t kChainStride = dev::norm_chain_stride(kNormChunk);  // LDS floats per chain row (padded)
constexpr uint32_t kNormLds = dev::norm_lds_floats(kNormChunk);        // the chain rows, then the result

// 1 / sqrt(dot(x, x) / cols + eps) of one row, for the whole block, in cpu::detail::dot's order
// (norm_device.h): each chunk's squares are staged in LDS transposed (every load of the chunk is
// issued before the first is used: one memory round trip per chunk), lanes 0..7 of wave 0 carry
// the 8 chain sums across the chunks, then wave 0 combines them and thread 0 finishes.
__device__ float row_rms_inv(const float* __restrict__ x, uint32_t cols, float eps, float* lds) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x;
    const uint32_t full = cols - cols % 8u;
    float p = 0.0f;
    for (uint32_t c0 = 0; c0 < full; c0 += kNormChunk) {
        const uint32_t n = min(kNormChunk, full - c0);  // a multiple of 8
        float v[kPerThread];
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) {
            const uint32_t e = tid + i * kNormBlock;
            v[i] = x[c0 + min(e, n - 1)];  // clamped: the value past n is never stored
        }
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) {
            const uint32_t e = tid + i * kNormBlock;
            if (e < n) lds[(e % 8) * kChainStride + e / 8] = v[i] * v[i];
        }
        __syncthreads();
        if (tid < 8) p = dev::norm_chain(lds + tid * kChainStride, n / 8, p);
        __syncthreads();
    }
    if (tid < 64) {
        const float inv = dev::norm_finish(p, x, full, cols, eps, tid);
        if (tid == 0) lds[8 * kChainStride] = inv;
    }
    __syncthreads();
    return lds[8 * kChainStride];
}

// grid rows, block kNormBlock. out may be x (each element is read before it is written, by
// the same thread, after the whole row has been summed).
__global__ __launch_bounds__(kNormBlock) void k_rms_norm_rows(const float* x, uint64_t x_stride,
                                                              const float* __restrict__ w, float* out,
                                                              uint64_t out_stride, uint32_t cols, float eps) {
#pragma clang fp contract(off)
    __shared__ float lds[kNormLds];
    const float* xr = x + (uint64_t)blockIdx.x * x_stride;
    const float inv = row_rms_inv(xr, cols, eps, lds);
    float* o = out + (uint64_t)blockIdx.x * out_stride;
    // every load of a chunk before the first store: one memory round trip per chunk
    for (uint32_t c0 = 0; c0 < cols; c0 += kNormChunk) {
        const uint32_t n = min(kNormChunk, cols - c0);
        float xv[kPerThread], wv[kPerThread];
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) {
            const uint32_t e = c0 + min(threadIdx.x + i * kNormBlock, n - 1);
            xv[i] = xr[e];
            wv[i] = w[e];
        }
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) {
            const uint32_t e = threadIdx.x + i * kNormBlock;
            if (e < n) {
                const float t = xv[i] * inv;
                o[c0 + e] = t * wv[i];
            }
        }
    }
}

__global__ __launch_bounds__(kNormBlock) void k_rms_inv_rows(const float* __restrict__ x, uint64_t x_stride,
                                                             uint32_t cols, float eps, float* __restrict__ inv) {
    __shared__ float lds[kNormLds];
    const float v = row_rms_inv(x + (uint64_t)blockIdx.x * x_stride, cols, eps, lds);
    if (threadIdx.x == 0) inv[blockIdx.x] = v;
}

}  // namespace

int launch_rms_norm(const float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride, uint32_t rows,
                    uint32_t cols, float eps, hipStream_t st) {
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    hipLaunchKernelGGL(k_rms_norm_rows, dim3(rows), dim3(kNormBlock), 0, st, x, x_stride, w, out, out_stride, cols, eps);
    return hip_status(hipGetLastError(), "rms_norm launch");
}

int launch_rms_inv(const float* x, uint64_t x_stride, uint32_t rows, uint32_t cols, float eps, float* inv,
                   hipStream_t st) {
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    hipLaunchKernelGGL(k_rms_inv_rows, dim3(rows), dim3(kNormBlock), 0, st, x, x_stride, cols, eps, inv);
    return hip_status(hipGetLastError(), "rms_inv launch");
}

}  // namespace halo_mi
