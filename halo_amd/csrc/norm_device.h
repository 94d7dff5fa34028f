// Device pieces of the RMS norm shared by the RMS_NORM kernels (k_norm.hip) and the GEMV's fused
// prologue (gemv_device.h), so that both compute 1 / rms in one and the same order:
// cpu::rms_norm (backends/cpu/ops_basic.cpp:18-33 of the reference) takes
//   mean = dot(x, x) / cols   (cpu::detail::dot, backends/cpu/kernel_common.h:16-27)
//   inv  = 1 / sqrt(mean + eps)
// where dot keeps 8 interleaved sequential sums p_j over the elements j, j + 8, j + 16, ... of
// the first cols - cols % 8, combines them as ((p0 + p4) + (p1 + p5)) + ((p2 + p6) + (p3 + p7))
// and adds the last cols % 8 products one at a time. A block stages the squares of the row in
// LDS transposed (element e in chain row e % 8, at e / 8), lanes 0..7 of wave 0 run the chains,
// and the squares are rounded as the CPU's products are, so every sum is the CPU's bitwise.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace halo_mi {
namespace dev {

// LDS floats of a chain row holding n squares (padded: rows start on different banks)
__host__ __device__ constexpr uint32_t norm_chain_stride(uint32_t n) { return n / 8 + 4; }
// LDS floats of the 8 chain rows for n squares, then one word for the result
__host__ __device__ constexpr uint32_t norm_lds_floats(uint32_t n) { return 8 * norm_chain_stride(n) + 4; }

// Continues chain sum p over m squares of one chain row r (LDS), in order. Batches of B 16-byte
// reads are issued before their 4 B additions, so the LDS latency is paid once per batch; the
// batch's 4 B registers count towards the caller's register budget. (Reading one batch ahead, in
// a second register set, measured slower in the GEMV's prologue.)
template <int B = 8>
__device__ __forceinline__ float norm_chain(const float* r, uint32_t m, float p) {
#pragma clang fp contract(off)
    uint32_t k = 0;
    for (; k + 4 * B <= m; k += 4 * B) {
        float4 q[B];
#pragma unroll
        for (int b = 0; b < B; ++b) q[b] = *reinterpret_cast<const float4*>(r + k + 4 * b);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            p = p + q[b].x;
            p = p + q[b].y;
            p = p + q[b].z;
            p = p + q[b].w;
        }
    }
    for (; k < m; ++k) p = p + r[k];
    return p;
}

// norm_chain with the reads of the next batch in flight while a batch is added (two register
// sets used in turn, so no copies between them), so the LDS latency overlaps the additions: for a
// chain that runs alone on the critical path (the GEMV's publishing workgroup). The additions are
// norm_chain's, in the same order.
template <int B = 4>
__device__ __forceinline__ float norm_chain_ahead(const float* r, uint32_t m, float p) {
#pragma clang fp contract(off)
    constexpr uint32_t N = 4 * B;  // floats per batch
    auto add = [&](const float4 (&q)[B]) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            p = p + q[b].x;
            p = p + q[b].y;
            p = p + q[b].z;
            p = p + q[b].w;
        }
    };
    auto load = [&](float4 (&q)[B], uint32_t k) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < B; ++b) q[b] = *reinterpret_cast<const float4*>(r + k + 4 * b);
    };
    uint32_t k = 0;
    if (m >= 2 * N) {
        // c0 holds r[k, k + N), c1 r[k + N, k + 2 N)
        float4 c0[B], c1[B];
        load(c0, 0);
        load(c1, N);
        for (; k + 4 * N <= m; k += 2 * N) {
            // (the scheduling barriers keep each batch's reads where they are issued here)
            add(c0);
            __builtin_amdgcn_sched_barrier(0);
            load(c0, k + 2 * N);
            __builtin_amdgcn_sched_barrier(0);
            add(c1);
            __builtin_amdgcn_sched_barrier(0);
            load(c1, k + 3 * N);
            __builtin_amdgcn_sched_barrier(0);
        }
        add(c0);
        add(c1);
        k += 2 * N;
    }
    for (; k + N <= m; k += N) {
        float4 q[B];
        load(q, k);
        add(q);
    }
    for (; k < m; ++k) p = p + r[k];
    return p;
}

// Wave 0 (all 64 lanes, p: lane j < 8 holds chain sum p_j): the dot's combine, the sequential
// tail of x[full .. cols) and 1 / sqrt(mean + eps), returned in lane 0 (other lanes: unspecified).
// sqrtf and / are correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt, set by the build;
// __fsqrt_rn would be the native approximation in this toolchain).
__device__ __forceinline__ float norm_finish(float p, const float* __restrict__ x, uint32_t full, uint32_t cols, float eps,
                                             uint32_t lane) {
#pragma clang fp contract(off)
    const float q = p + __shfl_down(p, 4, 8);  // lanes 0..3: p_j + p_{j+4}
    const float r = q + __shfl_down(q, 1, 8);  // lane 0: left, lane 2: right
    float s = r + __shfl_down(r, 2, 8);        // lane 0: left + right
    float inv = 0.0f;
    if (lane == 0) {
        float tail = 0.0f;
        for (uint32_t i = full; i < cols; ++i) {
            const float q2 = x[i] * x[i];
            tail = tail + q2;
        }
        s = s + tail;
        const float mean = s / (float)cols;
        inv = 1.0f / sqrtf(mean + eps);
    }
    return inv;
}

}  // namespace dev
}  // namespace halo_mi
