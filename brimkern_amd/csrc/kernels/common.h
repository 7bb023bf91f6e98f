// Shared device helpers for the .brik quantized matmul kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define BRIK_GROUP 32

// Plane formats: the value is the code's bit width, as in the reference's q8web/q4web/q3web.
enum { FMT_Q8 = 8, FMT_Q4 = 4, FMT_Q3 = 3 };

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// IEEE binary16 -> f32 (v_cvt_f32_f16). Exact for every finite half, including subnormals;
// e == 31 decodes to +-Inf / NaN like the reference's CPU decoder (src/lib/brik/f16.ts:31).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Weights are streamed once per launch: load them non-temporally so they do not evict the
// activation vector and the scale planes from the caches.
template <typename T>
__device__ __forceinline__ T ld_stream(const T* p)
{
    return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int b) { return (w >> (8 * b)) & 0xffu; }
