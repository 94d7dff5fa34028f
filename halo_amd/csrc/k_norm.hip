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

namespace halo_mi {
namespace {

constexpr uint32_t kNormBlock = 256;
constexpr uint32_t kNormChunk = 8192;               // floats of a row staged in LDS at a time
constexpr uint32_t kPerThread = kNormChunk / kNormBlock;
constexpr uint32_t kChainStride = kNormChunk / 8 + 4;  // LDS floats per chain row (padded)
constexpr uint32_t kNormLds = 8 * kChainStride + 4;     // the chain rows, then the result

// 1 / sqrt(dot(x, x) / cols + eps) of one row, for the whole block. The block stages the squares
// of a chunk of the row in LDS transposed, element e in chain row e % 8 at e / 8 (every load of
// the chunk is issued before the first is used: one memory round trip per chunk); lanes 0..7 of
// wave 0 run the dot's 8 interleaved sequential sums over their rows (16-byte LDS reads), then
// combine them as ((p0+p4)+(p1+p5))+((p2+p6)+(p3+p7)) and add the sequential tail of the last
// cols % 8 elements. The squares are rounded as the CPU's products are, so every sum is the
// CPU's bitwise.
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
        if (tid < 8) {
            // batches of 8 16-byte reads issued before their 32 additions (the LDS latency is
            // paid once per batch, not once per read)
            const float* r = lds + tid * kChainStride;
            const uint32_t m = n / 8;
            uint32_t k = 0;
            for (; k + 32 <= m; k += 32) {
                float4 q[8];
#pragma unroll
                for (int b = 0; b < 8; ++b) q[b] = *reinterpret_cast<const float4*>(r + k + 4 * b);
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    p = p + q[b].x;
                    p = p + q[b].y;
                    p = p + q[b].z;
                    p = p + q[b].w;
                }
            }
            for (; k < m; ++k) p = p + r[k];
        }
        __syncthreads();
    }
    if (tid < 64) {
        const float q = p + __shfl_down(p, 4, 8);  // lanes 0..3: p_j + p_{j+4}
        const float r = q + __shfl_down(q, 1, 8);  // lane 0: left, lane 2: right
        float s = r + __shfl_down(r, 2, 8);        // lane 0: left + right
        if (tid == 0) {
            float tail = 0.0f;
            for (uint32_t i = full; i < cols; ++i) {
                const float q2 = x[i] * x[i];
                tail = tail + q2;
            }
            s = s + tail;
            // sqrtf and / are correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt, set
            // by the build); __fsqrt_rn would be the native approximation in this toolchain
            const float mean = s / (float)cols;
            lds[8 * kChainStride] = 1.0f / sqrtf(mean + eps);
        }
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
