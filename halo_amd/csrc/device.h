// Device helpers shared by the kernel files of the halo_mi355x library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "decode.h"
#include "slab_layout.h"

namespace halo_mi::dev {

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ float ubyte(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sbyte(uint32_t v, int k) { return (float)(int)(int8_t)((v >> (8 * k)) & 0xFFu); }

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


// Value of the fp8 (e4m3) code 1 on this device: every code c < 16 converts to exactly
// c * fp8_unit(), so v_cvt_pk_f32_fp8 turns two 4-bit quants into two exact floats.
__device__ __forceinline__ float fp8_unit() { return __builtin_amdgcn_cvt_pk_f32_fp8(1u, false)[0]; }

// The CPU argmax's order (cpu_backend.cpp:738-739 of the reference: a row replaces the best only
// when strictly greater, so ties go to the lower index): (va, ia) ranks before (vb, ib).
// Index 0xFFFFFFFF (no row) ranks after everything.
__device__ __forceinline__ bool ranks_before(float va, uint32_t ia, float vb, uint32_t ib) {
    if (ia == 0xFFFFFFFFu) return false;
    if (ib == 0xFFFFFFFFu) return true;
    return va > vb || (va == vb && ia < ib);
}

// Wave-wide argmax of one value per lane: rank (lane's value and index take part) or not, any
// NaN flag. Every lane returns the wave's best; the order is total, so the result does not
// depend on the reduction order.
__device__ __forceinline__ void wave_argmax(float v, uint32_t idx, bool rank, bool is_nan, float& bv, uint32_t& bi,
                                            uint32_t& any_nan) {
    bv = rank ? v : 0.0f;
    bi = rank ? idx : 0xFFFFFFFFu;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, off);
        if (ranks_before(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    any_nan = __ballot(is_nan) != 0 ? 1u : 0u;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

}  // namespace halo_mi::dev
