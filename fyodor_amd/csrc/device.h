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
// DPP only, no LDS traffic: quad and row rotations give every lane its
// 16-lane row sum, row_bcast:15 / row_bcast:31 fold rows 0-2 into row 3,
// and lane 63 is broadcast. All 64 lanes must be active.
__device__ __forceinline__ float dpp_term(float v, int step)
{
    const int b = __builtin_bit_cast(int, v);
    int s;
    switch (step) {
    case 0: s = __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
    case 1: s = __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false); break;   // quad_perm [2,3,0,1]
    case 2: s = __builtin_amdgcn_update_dpp(0, b, 0x124, 0xF, 0xF, false); break;  // row_ror:4
    case 3: s = __builtin_amdgcn_update_dpp(0, b, 0x128, 0xF, 0xF, false); break;  // row_ror:8
    case 4: s = __builtin_amdgcn_update_dpp(0, b, 0x142, 0xA, 0xF, false); break;  // row_bcast:15 into rows 1, 3
    default: s = __builtin_amdgcn_update_dpp(0, b, 0x143, 0xC, 0xF, false); break; // row_bcast:31 into rows 2, 3
    }
    return __builtin_bit_cast(float, s);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int step = 0; step < 6; ++step) v += dpp_term(v, step);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

}  // namespace fy
