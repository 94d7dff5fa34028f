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

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

}  // namespace halo_mi::dev
