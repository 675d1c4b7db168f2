#pragma once
// bf16 <-> fp32 for the RMSNorm consumers (HIP sources only).  A 32-bit word
// holds two bf16 values, the lower address in the low half.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace gfd {
namespace bf16 {

__device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Round-to-nearest-even fp32 -> bf16 (finite values).
__device__ __forceinline__ uint32_t from_f32(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 values to one word of two bf16 (lo in the low half) with the
// hardware conversion (v_cvt_pk_bf16_f32 on gfx950), rounding to nearest
// even as from_f32 does, in one instruction instead of ten.
__device__ __forceinline__ uint32_t pack(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

}  // namespace bf16
}  // namespace gfd
