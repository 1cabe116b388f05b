// Device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fy {

// Cross-lane reductions without LDS: DPP moves inside a row of 16 lanes
// (gfx9 controls 0xB1 quad_perm [1,0,3,2], 0x4E quad_perm [2,3,0,1], 0x141
// row_half_mirror, 0x140 row_mirror; each lane reads a lane of its own
// row), then v_readlane across the four rows of a wavefront. (A __shfl_xor
// is a ds_bpermute: one LDS round trip per step, each waited for before the
// next.) Every lane of the row, or of the wavefront for the wave forms,
// must be active.
template <int CTRL>
__device__ __forceinline__ float row_lane(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ double row_lane(double v)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}

// The sum (MAX: the maximum) over the 16 lanes of an aligned row, the same
// bits in each of them: pairs, quads, half rows, the row (each step adds two
// values in either order, which is the same sum).
template <bool MAX>
__device__ __forceinline__ float row16_reduce(float v)
{
    if constexpr (MAX) {
        v = fmaxf(v, row_lane<0xB1>(v));
        v = fmaxf(v, row_lane<0x4E>(v));
        v = fmaxf(v, row_lane<0x141>(v));
        return fmaxf(v, row_lane<0x140>(v));
    } else {
        v += row_lane<0xB1>(v);
        v += row_lane<0x4E>(v);
        v += row_lane<0x141>(v);
        return v + row_lane<0x140>(v);
    }
}

__device__ __forceinline__ double row16_sum(double v)
{
    v += row_lane<0xB1>(v);
    v += row_lane<0x4E>(v);
    v += row_lane<0x141>(v);
    return v + row_lane<0x140>(v);
}

__device__ __forceinline__ float lane_value(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ double lane_value(double v, int lane)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}

// Over the wavefront, the same value in every lane: each row's, then the
// rows' as (r0 . r1) . (r2 . r3).
template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v)
{
    v = row16_reduce<MAX>(v);
    const float r0 = lane_value(v, 0), r1 = lane_value(v, 16), r2 = lane_value(v, 32), r3 = lane_value(v, 48);
    return MAX ? fmaxf(fmaxf(r0, r1), fmaxf(r2, r3)) : (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ double wave_sum(double v)
{
    v = row16_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

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
