// gfx950 kernels of the LM head's argmax (Backend::lm_head, include/halo/backend/backend.h:433-460
// of the reference; semantics of CpuBackend::lm_head, src/backend/cpu_backend.cpp:669-770):
//   stage 1: one ArgPart per 64 rows and vector, from a logits buffer (the slab GEMV writes the
//            same parts in its epilogue, so the fused path skips this stage);
//   stage 2: each vector's parts -> its result words {index, value bits, poisoned}, and the
//            optional dense ids and scattered ids.
// The ranking is a total order on (value, index) (higher value, then lower index), so neither
// stage depends on the reduction order: the result is the CPU's argmax over the same values.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device.h"
#include "launch.h"

namespace halo_mi {
namespace {

using namespace dev;

// grid (parts, n_vec), block 64: part p of vector v covers rows [64 p, 64 p + 64)
__global__ __launch_bounds__(64) void k_argmax_parts(const float* __restrict__ logits, uint64_t stride, uint32_t rows,
                                                     uint32_t valid_rows, ArgPart* __restrict__ parts) {
    const uint32_t p = blockIdx.x, v = blockIdx.y, lane = threadIdx.x;
    const uint32_t row = p * 64 + lane;
    const bool live = row < rows;
    const float val = live ? logits[(uint64_t)v * stride + row] : 0.0f;
    const bool nan = live && val != val;
    const bool rank = live && !nan && (valid_rows == 0 || row < valid_rows);
    float bv;
    uint32_t bi, any_nan;
    wave_argmax(val, row, rank, nan, bv, bi, any_nan);
    if (lane == 0) parts[(uint64_t)v * gridDim.x + p] = ArgPart{bv, bi, any_nan, 0u};
}

// grid n_vec, block 256. A poisoned vector (any NaN logit) reports {kNoIndex, quiet NaN, 1}
// (cpu_backend.cpp:745-747); one with no ranked row {kNoIndex, 0, 0} (TopKEntry's default,
// include/halo/backends/cpu/ops.h:351-355). ids: the winning index, 0 for either of those
// (cpu_backend.cpp:756-760); ids_scatter[ids_slots[v]] likewise, a slot past the end dropped.
__global__ __launch_bounds__(256) void k_argmax_finish(const ArgPart* __restrict__ parts, uint32_t n_parts,
                                                       uint32_t* __restrict__ result, int32_t* ids,
                                                       const uint32_t* ids_slots, int32_t* ids_scatter,
                                                       uint64_t scatter_len) {
    __shared__ float sv[256];
    __shared__ uint32_t si[256], sn[256];
    const uint32_t v = blockIdx.x, tid = threadIdx.x;
    float bv = 0.0f;
    uint32_t bi = kNoIndex, nan = 0;
    for (uint32_t i = tid; i < n_parts; i += 256) {
        const ArgPart q = parts[(uint64_t)v * n_parts + i];
        nan |= q.nan;
        if (ranks_before(q.value, q.index, bv, bi)) {
            bv = q.value;
            bi = q.index;
        }
    }
    sv[tid] = bv;
    si[tid] = bi;
    sn[tid] = nan;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            if (ranks_before(sv[tid + s], si[tid + s], sv[tid], si[tid])) {
                sv[tid] = sv[tid + s];
                si[tid] = si[tid + s];
            }
            sn[tid] |= sn[tid + s];
        }
        __syncthreads();
    }
    if (tid != 0) return;
    const bool poisoned = sn[0] != 0;
    const uint32_t idx = poisoned ? kNoIndex : si[0];
    result[3 * v] = idx;
    result[3 * v + 1] = poisoned ? 0x7FC00000u : __float_as_uint(sv[0]);
    result[3 * v + 2] = poisoned ? 1u : 0u;
    const int32_t id = idx == kNoIndex ? 0 : (int32_t)idx;
    if (ids) ids[v] = id;
    if (ids_scatter) {
        const uint32_t slot = ids_slots[v];
        if (slot < scatter_len) ids_scatter[slot] = id;
    }
}

}  // namespace

int launch_argmax_parts(const float* logits, uint64_t stride, uint32_t rows, uint32_t n_vec, uint32_t valid_rows,
                        ArgPart* parts, hipStream_t st) {
    const uint32_t n_parts = (rows + 63) / 64;
    hipLaunchKernelGGL(k_argmax_parts, dim3(n_parts, n_vec), dim3(64), 0, st, logits, stride, rows, valid_rows, parts);
    return hip_status(hipGetLastError(), "argmax_parts launch");
}

int launch_argmax_finish(const ArgPart* parts, uint32_t n_parts, uint32_t n_vec, uint32_t* result, int32_t* ids,
                         const uint32_t* ids_slots, int32_t* ids_scatter, uint64_t scatter_len, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_finish, dim3(n_vec), dim3(256), 0, st, parts, n_parts, result, ids, ids_slots, ids_scatter,
                       scatter_len);
    return hip_status(hipGetLastError(), "argmax_finish launch");
}

}  // namespace halo_mi
