// Shared device helpers for the .brik quantized matmul kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define BRIK_GROUP 32

// Plane formats: the value is the code's bit width, as in the reference's q8web/q4web/q3web.
enum { FMT_Q8 = 8, FMT_Q4 = 4, FMT_Q3 = 3, FMT_F16 = 16 };   // F16: IEEE half weights (the MFMA GEMM only)

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

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

// ---- buffer addressing ------------------------------------------------------------------------
// A raw buffer resource over [p, p + bytes): loads take a 32-bit VGPR offset, a uniform SGPR offset
// and an immediate, so per-load address arithmetic is free, and reads past `bytes` return 0
// instead of faulting. Planes are limited to < 4 GiB per resource (checked on the host).
typedef __amdgpu_buffer_rsrc_t brsrc_t;
#define BRIK_BUF_DWORD3 0x00020000   // raw (untyped) buffer, 32-bit data format, gfx9 family

__device__ __forceinline__ brsrc_t make_rsrc(const void* p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, BRIK_BUF_DWORD3);
}

// Order-preserving map of f32 to u32 (larger float -> larger key); NaN -> 0 (ranks below every
// number). The top-k passes compare logits through it.
__device__ __forceinline__ uint32_t order_key(float v)
{
    if (v != v) return 0u;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// p, with its provenance hidden from the compiler (an empty asm on a uniform value). Loads through a
// restrict-qualified const pointer are treated as reads of constant memory, which the compiler may
// reorder freely; through the laundered pointer they stay in program order relative to other memory
// operations and compiler barriers, where the order in which loads are issued matters.
template <typename T>
__device__ __forceinline__ T* launder_uniform(T* p)
{
    asm volatile("" : "+s"(p));
    return p;
}

// Cache policy of streamed weight loads: non-temporal (nt).
#define BRIK_AUX_STREAM 2

// ---- DPP cross-lane sums (within 16-lane rows) ---------------------------------------------------

#define BRIK_DPP_ADD(v, CTRL) \
    ((v) + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (CTRL), 0xF, 0xF, false)))
#define BRIK_DPP_MAX(v, CTRL) \
    fmaxf((v), __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (CTRL), 0xF, 0xF, false)))
#define DPP_QUAD_1032 0xB1      // quad_perm [1,0,3,2]
#define DPP_QUAD_2301 0x4E      // quad_perm [2,3,0,1]
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_ROR4 0x124
#define DPP_ROW_ROR8 0x128

// Sum / max over aligned groups of 8 lanes; every lane of the group receives the result.
__device__ __forceinline__ float sum8(float v)
{
    v = BRIK_DPP_ADD(v, DPP_QUAD_1032);
    v = BRIK_DPP_ADD(v, DPP_QUAD_2301);
    return BRIK_DPP_ADD(v, DPP_ROW_HALF_MIRROR);
}
__device__ __forceinline__ float max8(float v)
{
    v = BRIK_DPP_MAX(v, DPP_QUAD_1032);
    v = BRIK_DPP_MAX(v, DPP_QUAD_2301);
    return BRIK_DPP_MAX(v, DPP_ROW_HALF_MIRROR);
}
// Sum over aligned groups of 16 lanes (one DPP row); every lane receives the result.
__device__ __forceinline__ float sum16(float v)
{
    v = BRIK_DPP_ADD(v, DPP_QUAD_1032);
    v = BRIK_DPP_ADD(v, DPP_QUAD_2301);
    v = BRIK_DPP_ADD(v, DPP_ROW_ROR4);
    return BRIK_DPP_ADD(v, DPP_ROW_ROR8);
}

// Unsigned maximum over aligned groups of 16 lanes (one DPP row); every lane receives the result.
__device__ __forceinline__ uint32_t max16u(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_QUAD_1032, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_QUAD_2301, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_ROW_ROR4, 0xF, 0xF, false));
    return max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_ROW_ROR8, 0xF, 0xF, false));
}

// Wait until at most N vector-memory loads of this wave are in flight (direct global->LDS loads count;
// the compiler does not track those as writers of LDS, so their completion is waited for explicitly).
namespace brik {
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
typedef __attribute__((address_space(3))) void lds_void_t;
}  // namespace brik
