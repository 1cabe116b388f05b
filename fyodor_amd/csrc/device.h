// Device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fy {

// IEEE binary16 bits -> f32 with v_cvt_f32_f16; exact for every encoding,
// subnormals included (backend/core/llm_quant.c:5-39 decodes the same value).
__device__ __forceinline__ float f16_to_f32(uint32_t bits)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits)
{
    return __builtin_bit_cast(float, bits << 16);
}

// Byte b of v as a float; selects v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float ubyte_f32(uint32_t v, int b)
{
    return (float)((v >> (8 * b)) & 0xFFu);
}

__device__ __forceinline__ uint32_t word_of(const uint4 &v, int j)
{
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

}  // namespace fy
