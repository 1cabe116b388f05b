// Block dot products on gfx950 int8 MFMA, shared by the small-N path
// (smalln.hip) and the prefill GEMM (prefill.hip): activation digits, the
// tiled weight stages of one 256-column group, and the digit recombination.
//
// Activations. Each 32-column group of a token's x is scaled by 2^(22-e)
// (2^(e-1) <= max |x| < 2^e over the group) and rounded to integers X with
// |X| <= 2^22, split into signed 8-bit digits X = a0 + 2^8 a1 + 2^16 a2. A
// non-finite value makes its whole group NaN. Block dot products sum q * X are
// then exact in int32: the MFMA unit forms sum q * a_d for each digit d and the
// three sums are recombined. Digits of group g (32 columns) sit at
// dig + g * 128 * np, slot 4t + d (32 bytes; slot 4t + 3 is zero), with
// meta[g * np + t] = {2^(e-22), (float)sum(X) * 2^(e-22)}.
#pragma once
#include "device.h"
#include "formats.h"

namespace fy {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kSlotBytes = 32;      // one digit of one token over a 32-column group

__device__ __forceinline__ i32x4 as_i32x4(u32x4 v) { return __builtin_bit_cast(i32x4, v); }

// ---- activation digits ---------------------------------------------------
// Group g (32 columns) of a chunk: digits at dig + g * 128 * np, slot 4t + d
// (32 bytes), meta[g * np + t] = {2^(e-22), (float)sum(X) * 2^(e-22)}.

// Byte b of each of four words, packed into one word.
__device__ __forceinline__ uint32_t gather_byte(const int (&v)[8], int k, int b)
{
    const uint32_t sel = 0x0c0c0000u | (uint32_t)(4 + b) << 8 | (uint32_t)b;
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)v[k + 1], (uint32_t)v[k], sel);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)v[k + 3], (uint32_t)v[k + 2], sel);
    return lo | hi << 16;
}

// Item `item` = 8 consecutive values of token t (4 items per group). The four
// lanes of a group are consecutive and must call this together. The signed
// digits of X are byte 0 of X, byte 1 of X + 2^7 and byte 2 of X + 2^7 + 2^15
// (a1 = sext8((X + 128) >> 8), a2 = (X + 32896) >> 16).
__device__ __forceinline__ void quantize8(float4 v0, float4 v1, int np, int t, int item, uint8_t *dig, float2 *meta)
{
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.f, z = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        m = fmaxf(m, fabsf(v[j]));
        z = __builtin_fmaf(v[j], 0.f, z);   // NaN iff some value is inf or NaN
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    z += __shfl_xor(z, 1, 64);
    z += __shfl_xor(z, 2, 64);
    int ex = 0;
    (void)__builtin_frexpf(m, &ex);
    const bool finite = z == z;
    const int shift = m > 0.f && finite ? 22 - ex : 0;
    const float scale = !finite ? __builtin_nanf("") : m > 0.f ? __builtin_ldexpf(1.f, ex - 22) : 0.f;
    int X[8], X1[8], X2[8];
    int sx = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // A non-finite group's digits are never used: its scale is NaN.
        X[j] = (int)__builtin_rintf(__builtin_ldexpf(v[j], shift));
        X1[j] = X[j] + 128;
        X2[j] = X[j] + 32896;
        sx += X[j];
    }
    sx += __shfl_xor(sx, 1, 64);
    sx += __shfl_xor(sx, 2, 64);
    const int g = item >> 2, part = item & 3;
    uint8_t *dst = dig + (size_t)g * 4 * kSlotBytes * np + kSlotBytes * 4 * t + 8 * part;
    *(uint2 *)dst = make_uint2(gather_byte(X, 0, 0), gather_byte(X, 4, 0));
    *(uint2 *)(dst + kSlotBytes) = make_uint2(gather_byte(X1, 0, 1), gather_byte(X1, 4, 1));
    *(uint2 *)(dst + 2 * kSlotBytes) = make_uint2(gather_byte(X2, 0, 2), gather_byte(X2, 4, 2));
    *(uint2 *)(dst + 3 * kSlotBytes) = make_uint2(0, 0);
    if (part == 0) meta[(size_t)g * np + t] = make_float2(scale, (float)sx * scale);
}

// ---- weight stages -------------------------------------------------------
template <unsigned T> struct WStage;
template <> struct WStage<Q4_K> { u32x4 q[4]; u32x4 sl; };
template <> struct WStage<Q6_K> { u32x4 ql[4], qh[4]; u32x4 sc; uint32_t d; };
template <> struct WStage<Q8_0> { u32x4 q[8]; uint32_t d[8]; };
template <> struct WStage<Q4_0> { u32x4 q[8]; uint32_t d[8]; };

// The lane's place in the tile.
struct Lane {
    const uint8_t *tile;
    int R, r, h, slot;
    int groups, blocks;   // per row: 256-column groups, 32-column blocks
};

// Blocks in group g (Q8_0/Q4_0 last group may be short).
__device__ __forceinline__ int group_blocks(const Lane &L, int g)
{
    const int nb = L.blocks - 8 * g;
    return nb < 8 ? nb : 8;
}

// One 16-byte weight load; NT marks it non-temporal (weights are streamed
// once; the callers choose where that measured faster).
template <bool NT>
__device__ __forceinline__ u32x4 load16(const uint8_t *p)
{
    if constexpr (NT) return __builtin_nontemporal_load((const u32x4 *)p);
    else return *(const u32x4 *)p;
}

template <unsigned T, bool NT = false>
__device__ __forceinline__ void load_weights(WStage<T> &w, const Lane &L, int g)
{
    const int R = L.R, r = L.r, h = L.h;
    if constexpr (T == Q4_K) {
        const uint8_t *b = L.tile + (size_t)144 * R * g;
#pragma unroll
        for (int p = 0; p < 4; ++p) w.q[p] = load16<NT>(b + 32 * R * p + 16 * R * h + 16 * r);
        w.sl = load16<NT>(b + 128 * R + 16 * r);
    } else if constexpr (T == Q6_K) {
        const uint8_t *b = L.tile + (size_t)208 * R * g;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            w.ql[p] = load16<NT>(b + 48 * R * p + 16 * R * h + 16 * r);
            w.qh[p] = load16<NT>(b + 48 * R * p + 32 * R + 16 * r);
        }
        w.sc = load16<NT>(b + 192 * R + 16 * r);
        w.d = *(const uint16_t *)(L.tile + (size_t)208 * R * L.groups + 2 * R * g + 2 * r);
    } else {
        // A full group: Q4_0 units of two blocks (q[0..3]) or Q8_0 blocks, and
        // the row's eight scales as one 16-byte load (d[0..3], two per word).
        // A short last group: block by block, one scale per word.
        constexpr int quant = T == Q8_0 ? 32 : 16;
        const int nb = group_blocks(L, g);
        const uint8_t *b = L.tile + (size_t)(quant + 2) * 8 * R * g;
        if (nb == 8) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (T == Q4_0 && j >= 4) w.q[j] = (u32x4){};
                else w.q[j] = load16<NT>(b + 32 * R * j + 16 * R * h + 16 * r);
            }
            const u32x4 d = load16<NT>(b + 8 * quant * R + 16 * r);
#pragma unroll
            for (int k = 0; k < 8; ++k) w.d[k] = k < 4 ? d[k] : 0u;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int jj = j < nb ? j : nb - 1;
                w.q[j] = load16<NT>(b + quant * R * jj + (T == Q8_0 ? 16 * R * h : 0) + 16 * r);
                w.d[j] = *(const uint16_t *)(b + quant * R * nb + 2 * R * jj + 2 * r);
            }
        }
    }
}

// fp16 bits of the scale of block j of a Q8_0/Q4_0 stage (FULL: a full group,
// two scales per word; else one per word).
template <bool FULL, unsigned T>
__device__ __forceinline__ uint32_t block_d(const WStage<T> &w, int j)
{
    if constexpr (FULL) return (w.d[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    else return w.d[j];
}

// sum q * X of one 32-column block from its three digit sums. Q4_K
// (q <= 15): |D2| <= 32 * 15 * 64, so the whole sum fits int32. Q8_0, and
// Q6_K and Q4_0 in their scaled forms (|q| <= 128, see block_operand), can
// reach 2^34: the low two digits (below 2^27) combine in int32, the top one
// in float.
// The int32 form is evaluated as (d2 * 2^8 + d1) * 2^8 + d0, two shift-adds;
// the empty asm keeps the compiler from re-associating it into two shifts
// and a three-input add. (It touches no register the MFMA writes: those are
// read only by compiler-visible code, which keeps the MFMA result hazards
// under the compiler's control.)
template <unsigned T>
__device__ __forceinline__ float recombine(int d0, int d1, int d2)
{
    if constexpr (T == Q4_K) {
        int u = d2 * 256 + d1;
        asm("" : "+v"(u));
        return (float)(u * 256 + d0);
    } else {
        return (float)d2 * 65536.f + (float)(d1 * 256 + d0);
    }
}

// Block j (32 columns) of one group for this lane (half h): the B operand
// (signed 8-bit weights), the multipliers of q.x (sc) and of sum x (mn, Q4_K
// minimums; 0 otherwise), and which of the group's eight 32-column x groups
// the lane's A-rows cover. K-quant superblock scales are left to
// group_scales (backend/core/llm_quant.c:70-142).
//
// The offset weights enter the MFMA scaled so that a byte needs no per-byte
// subtraction: Q6_K as 4 (q6 - 32) = (q6 << 2) ^ 0x80 (the 6-bit value in
// bits 2..7, its top bit flipped), Q4_0 as 16 (q - 8) = (q << 4) ^ 0x80; the
// factor returns through the scale (exactly: a power of two).
template <unsigned T, bool FULL = true>
__device__ __forceinline__ i32x4 block_operand(const WStage<T> &w, int j, int h, float &sc, float &mn, int &xgl)
{
    mn = 0.f;
    if constexpr (T == Q4_K) {
        const int p = j >> 1, nib = j & 1;
        const uint32_t own = w.sl[p];
        sc = (float)((own >> (12 * nib)) & 63u);
        mn = (float)((own >> (12 * nib + 6)) & 63u);
        xgl = j;
        return as_i32x4((w.q[p] >> (4 * nib)) & 0x0F0F0F0Fu);
    } else if constexpr (T == Q6_K) {
        const int p = j >> 1, m = j & 1, q = 2 * m + h;
        u32x4 u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = m ? w.ql[p][k] >> 2 : w.ql[p][k] << 2;   // nibble to bits 2..5
            const uint32_t hi = w.qh[p][k] << (6 - 2 * q);                // two bits to 6..7
            u[k] = (lo & 0x3C3C3C3Cu) | ((hi & 0xC0C0C0C0u) ^ 0x80808080u);
        }
        sc = (float)(int8_t)((w.sc[p] >> (8 * q)) & 0xFFu);
        xgl = 4 * (p >> 1) + q;
        return as_i32x4(u);
    } else if constexpr (T == Q8_0) {
        sc = f16_to_f32(block_d<FULL>(w, j));
        xgl = j;
        return as_i32x4(w.q[j]);
    } else {
        // Full group: nibble j & 1 of unit j >> 1 (this lane's 16 columns);
        // short group: nibble h of block j. The nibble goes to bits 4..7.
        u32x4 u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t v = FULL ? w.q[j >> 1][k] << (4 - 4 * (j & 1)) : w.q[j][k] << (4 - 4 * h);
            u[k] = (v & 0xF0F0F0F0u) ^ 0x80808080u;
        }
        sc = f16_to_f32(block_d<FULL>(w, j)) * 0.0625f;
        xgl = j;
        return as_i32x4(u);
    }
}

// Superblock scales of a K-quant group: d and dmin (Q4_K), d (Q6_K).
template <unsigned T>
__device__ __forceinline__ void group_scales(const WStage<T> &w, float &d, float &dmin)
{
    d = dmin = 0.f;
    if constexpr (T == Q4_K) {
        const uint32_t dd = (w.sl.x >> 24) | ((w.sl.y >> 24) << 8) | ((w.sl.z >> 24) << 16) | ((w.sl.w >> 24) << 24);
        d = f16_to_f32(dd & 0xFFFFu);
        dmin = f16_to_f32(dd >> 16);
    } else if constexpr (T == Q6_K) {
        d = f16_to_f32(w.d) * 0.25f;   // the weights entered as 4 (q6 - 32)
    }
}

}  // namespace fy
