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

}  // namespace bf16
}  // namespace gfd
