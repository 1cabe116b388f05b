// Small-N matmul Y[n][row] = sum_k W[row][k] * X[n][k] for batches 1..8
// (batch-1 decode and speculative-decode verification) over the tiled weight
// layout of formats.h, with every block dot product on gfx950 int8 MFMA.
//
// Activations. Each 32-column group of a token's x is scaled by 2^(22-e)
// (2^(e-1) <= max |x| < 2^e over the group) and rounded to integers X with
// |X| <= 2^22, split into signed 8-bit digits X = a0 + 2^8 a1 + 2^16 a2. A
// non-finite value makes its whole group NaN. Block dot products sum q * X are
// then exact in int32: the MFMA unit forms sum q * a_d for each digit d and the
// three sums are recombined in integers. Per (row, token, 32-column group) the
// float work applies the block scales as the reference decodes them
// (backend/core/llm_quant.c:70-142): Q4_K (d*sc)*q - dmin*m, Q6_K
// (d*sc)*(q6-32), Q8_0 d*q, Q4_0 d*(q-8); the Q6_K and Q4_0 offsets are folded
// into signed 8-bit weights before the MFMA.
//
// MFMA mapping (v_mfma_i32_32x32x32_i8). A = activation digits, 32 rows:
// row 4t + d holds digit d of token t (row 4t + 3 is zero). B = 32 weight
// rows of the tile x 32 columns of the group: lane l supplies weight row l%32,
// columns 16(l/32)..+15. D lane l, register r holds A-row 8(r/4) + 4(l/32) +
// r%4 for weight row l%32, so each lane holds all three digit sums of its
// tokens 2(r/4) + l/32 and recombines them without crossing lanes. Q6_K scale
// groups are 16 columns: its A-row 8t + 4c + d carries digit d of token t in
// the 16 columns of half c only (zeros elsewhere), so lane half c sees the sums
// of its own scale group for tokens 0..3 (a second MFMA covers tokens 4..7).
//
// Work split. One workgroup per 32-row tile. Its KS wavefronts split the
// tile's 256-column groups; each streams its groups through a two-stage
// register ring, all loads of a stage issued one stage ahead (vector loads
// retire in order, so activations are requested before weights), and the
// partial sums meet in LDS at the end. N = 1 quantizes each wavefront's own
// columns of x into LDS; N >= 2 reads digits written once per call by
// quantize_x into the workspace. Columns beyond kChunkCols run as further
// launches that add into y.
#include "device.h"
#include "formats.h"
#include "kernels.h"

namespace fy {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunkCols = 16384;   // columns per launch (bounds the LDS copy of x)
constexpr int kSlotBytes = 32;      // one digit of one token over a 32-column group

__device__ __forceinline__ int sext8(int v) { return (int)(int8_t)(v & 0xFF); }

// Bytes v < 128 minus c (c <= 64) as signed 8-bit values, four at once.
__device__ __forceinline__ uint32_t bytes_minus(uint32_t v, uint32_t c4)
{
    return ((v | 0x80808080u) - c4) ^ 0x80808080u;
}

__device__ __forceinline__ i32x4 as_i32x4(u32x4 v) { return __builtin_bit_cast(i32x4, v); }

// ---- activation digits ---------------------------------------------------
// Group g (32 columns) of a chunk: digits at dig + g * 128 * np, slot 4t + d
// (32 bytes), meta[g * np + t] = {2^(e-22), (float)sum(X) * 2^(e-22)}.

// Item `item` = 8 consecutive values of token t (4 items per group). The four
// lanes of a group are consecutive and must call this together.
__device__ __forceinline__ void quantize8(float4 v0, float4 v1, int np, int t, int item, uint8_t *dig, float2 *meta)
{
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.f;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        m = fmaxf(m, fabsf(v[j]));
        bad |= !(fabsf(v[j]) <= 3.4028235e38f);   // inf or NaN
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    int ex = 0;
    (void)__builtin_frexpf(m, &ex);
    const bool finite = !bad;
    const int shift = m > 0.f && finite ? 22 - ex : 0;
    const float scale = !finite ? __builtin_nanf("") : m > 0.f ? __builtin_ldexpf(1.f, ex - 22) : 0.f;
    uint32_t pk[3][2] = {{0, 0}, {0, 0}, {0, 0}};
    int sx = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int X = finite ? (int)__builtin_rintf(__builtin_ldexpf(v[j], shift)) : 0;
        const int a0 = sext8(X), r1 = (X - a0) >> 8, a1 = sext8(r1), a2 = (r1 - a1) >> 8;
        sx += X;
        pk[0][j >> 2] |= (uint32_t)(a0 & 0xFF) << (8 * (j & 3));
        pk[1][j >> 2] |= (uint32_t)(a1 & 0xFF) << (8 * (j & 3));
        pk[2][j >> 2] |= (uint32_t)(a2 & 0xFF) << (8 * (j & 3));
    }
    sx += __shfl_xor(sx, 1, 64);
    sx += __shfl_xor(sx, 2, 64);
    const int g = item >> 2, part = item & 3;
    uint8_t *dst = dig + (size_t)g * 4 * kSlotBytes * np + kSlotBytes * 4 * t + 8 * part;
#pragma unroll
    for (int d = 0; d < 3; ++d) *(uint2 *)(dst + kSlotBytes * d) = make_uint2(pk[d][0], pk[d][1]);
    *(uint2 *)(dst + kSlotBytes * 3) = make_uint2(0, 0);
    if (part == 0) meta[(size_t)g * np + t] = make_float2(scale, (float)sx * scale);
}

// Digits of n tokens x cols columns (row stride ldx) for a batch of np slots.
__global__ __launch_bounds__(256) void quantize_x(const float *__restrict__ x, int ldx, int cols, int n, int np,
    uint8_t *__restrict__ dig, float2 *__restrict__ meta)
{
    const int per = cols / 8, total = n * per;   // a multiple of 4: whole groups
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int t = i / per, item = i % per;
    const float4 *src = (const float4 *)(x + (size_t)t * ldx) + 2 * item;
    quantize8(src[0], src[1], np, t, item, dig, meta);
}

// ---- weight stages -------------------------------------------------------
template <unsigned T> struct WStage;
template <> struct WStage<Q4_K> { u32x4 q[4]; u32x4 sl; };
template <> struct WStage<Q6_K> { u32x4 ql[4], qh[4]; u32x4 sc; uint32_t d; };
template <> struct WStage<Q8_0> { u32x4 q[8]; uint32_t d[8]; };
template <> struct WStage<Q4_0> { u32x4 q[8]; uint32_t d[8]; };

// MFMAs per 256-column group, and how many activation operands each needs.
template <unsigned T, int NP> constexpr int kTokenHalves = (T == Q6_K && NP > 4) ? 2 : 1;

template <unsigned T, int NP, bool G>
struct Stage {
    WStage<T> w;
    i32x4 a[G ? 8 * kTokenHalves<T, NP> : 1];
};

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

template <unsigned T>
__device__ __forceinline__ void load_weights(WStage<T> &w, const Lane &L, int g)
{
    const int R = L.R, r = L.r, h = L.h;
    if constexpr (T == Q4_K) {
        const uint8_t *b = L.tile + (size_t)144 * R * g;
#pragma unroll
        for (int p = 0; p < 4; ++p) w.q[p] = *(const u32x4 *)(b + 32 * R * p + 16 * R * h + 16 * r);
        w.sl = *(const u32x4 *)(b + 128 * R + 16 * r);
    } else if constexpr (T == Q6_K) {
        const uint8_t *b = L.tile + (size_t)208 * R * g;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            w.ql[p] = *(const u32x4 *)(b + 48 * R * p + 16 * R * h + 16 * r);
            w.qh[p] = *(const u32x4 *)(b + 48 * R * p + 32 * R + 16 * r);
        }
        w.sc = *(const u32x4 *)(b + 192 * R + 16 * r);
        w.d = *(const uint16_t *)(L.tile + (size_t)208 * R * L.groups + 2 * R * g + 2 * r);
    } else {
        constexpr int quant = T == Q8_0 ? 32 : 16;
        const int nb = group_blocks(L, g);
        const uint8_t *b = L.tile + (size_t)(quant + 2) * 8 * R * g;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int jj = j < nb ? j : nb - 1;
            w.q[j] = *(const u32x4 *)(b + quant * R * jj + quant * r + (T == Q8_0 ? 16 * h : 0));
            w.d[j] = *(const uint16_t *)(b + quant * R * nb + 2 * R * jj + 2 * r);
        }
    }
}

// Activation operand of MFMA j (token half th) of chunk-local group gl:
// returns the byte offset into the digit array, and whether the lane's
// A-row is live for n tokens.
template <unsigned T, int NP>
__device__ __forceinline__ int a_offset(const Lane &L, int gl, int j, int th, int n, int nb, bool &live)
{
    const int row_bytes = 4 * kSlotBytes * NP;
    if constexpr (T == Q6_K) {
        const int p = j >> 1, m = j & 1;
        const int t = (L.slot >> 3) + 4 * th, c = (L.slot >> 2) & 1, d = L.slot & 3;
        live = c == L.h && d < 3 && t < n;
        const int xg = 8 * gl + 4 * (p >> 1) + 2 * m + L.h;
        return xg * row_bytes + kSlotBytes * (4 * (t < NP ? t : 0) + d) + 16 * (p & 1);
    } else {
        const int jj = j < nb ? j : nb - 1;
        const int t = L.slot >> 2;
        live = t < n;
        return (8 * gl + jj) * row_bytes + kSlotBytes * (t < NP ? L.slot : 0) + 16 * L.h;
    }
}

template <unsigned T, int NP, bool G>
__device__ __forceinline__ void load_stage(Stage<T, NP, G> &st, const Lane &L, int g, int g0c,
    const uint8_t *__restrict__ dig, int n)
{
    if constexpr (G) {
        const int nb = (T == Q8_0 || T == Q4_0) ? group_blocks(L, g) : 8;
#pragma unroll
        for (int th = 0; th < kTokenHalves<T, NP>; ++th)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                bool live;
                const int off = a_offset<T, NP>(L, g - g0c, j, th, n, nb, live);
                st.a[8 * th + j] = *(const i32x4 *)(dig + off);
            }
    }
    load_weights<T>(st.w, L, g);
}

// sum q * X of one 32-column block from its three digit sums. Q4_K (q <= 15)
// and Q4_0 (|q| <= 8): |D2| <= 32 * 15 * 64, so the whole sum fits int32.
// Q8_0 (|q| <= 128) and Q6_K (|q| <= 32) can reach 2^34: the low two digits
// (below 2^27) combine in int32, the top one in float.
template <unsigned T>
__device__ __forceinline__ float recombine(int d0, int d1, int d2)
{
    if constexpr (T == Q4_K || T == Q4_0) return (float)(d2 * 65536 + d1 * 256 + d0);
    else return (float)d2 * 65536.f + (float)(d1 * 256 + d0);
}

// The block dot products of one stage (group g) into acc. Q4_K/Q8_0/Q4_0:
// acc[k] belongs to token 2k + h; Q6_K: acc[t] to token t (this lane half's
// scale groups).
template <unsigned T, int NP, bool G>
__device__ __forceinline__ void compute_stage(float (&acc)[8], const Stage<T, NP, G> &st, const Lane &L, int g,
    int g0c, const uint8_t *dig, const float2 *meta, int n)
{
    const int h = L.h;
    const int nb = (T == Q8_0 || T == Q4_0) ? group_blocks(L, g) : 8;
    float d = 0.f, dmin = 0.f;
    if constexpr (T == Q4_K) {
        const uint32_t dd = (st.w.sl.x >> 24) | ((st.w.sl.y >> 24) << 8) | ((st.w.sl.z >> 24) << 16) |
            ((st.w.sl.w >> 24) << 24);
        d = f16_to_f32(dd & 0xFFFFu);
        dmin = f16_to_f32(dd >> 16);
    } else if constexpr (T == Q6_K) {
        d = f16_to_f32(st.w.d);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if ((T == Q8_0 || T == Q4_0) && j >= nb) break;
        i32x4 b;
        float factor, bias = 0.f;
        int xg;
        if constexpr (T == Q4_K) {
            const int p = j >> 1, nib = j & 1;
            b = as_i32x4((st.w.q[p] >> (4 * nib)) & 0x0F0F0F0Fu);
            const uint32_t own = st.w.sl[p];
            factor = d * (float)((own >> (12 * nib)) & 63u);
            bias = dmin * (float)((own >> (12 * nib + 6)) & 63u);
            xg = 8 * (g - g0c) + j;
        } else if constexpr (T == Q6_K) {
            const int p = j >> 1, m = j & 1, q = 2 * m + h;
            u32x4 u;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                u[k] = bytes_minus(((st.w.ql[p][k] >> (4 * m)) & 0x0F0F0F0Fu) |
                    (((st.w.qh[p][k] >> (2 * q)) & 0x03030303u) << 4), 0x20202020u);
            b = as_i32x4(u);
            factor = d * (float)(int8_t)((st.w.sc[p] >> (8 * q)) & 0xFFu);
            xg = 8 * (g - g0c) + 4 * (p >> 1) + q;
        } else if constexpr (T == Q8_0) {
            b = as_i32x4(st.w.q[j]);
            factor = f16_to_f32(st.w.d[j]);
            xg = 8 * (g - g0c) + j;
        } else {
            u32x4 u;
#pragma unroll
            for (int k = 0; k < 4; ++k) u[k] = bytes_minus((st.w.q[j][k] >> (4 * h)) & 0x0F0F0F0Fu, 0x08080808u);
            b = as_i32x4(u);
            factor = f16_to_f32(st.w.d[j]);
            xg = 8 * (g - g0c) + j;
        }
#pragma unroll
        for (int th = 0; th < kTokenHalves<T, NP>; ++th) {
            bool live;
            const int off = a_offset<T, NP>(L, g - g0c, j, th, n, nb, live);
            i32x4 a;
            if constexpr (G) a = st.a[8 * th + j];
            else a = *(const i32x4 *)(dig + off);
            if (!live) a = (i32x4){0, 0, 0, 0};
            const i32x16 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, (i32x16){}, 0, 0, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float Gs = recombine<T>(D[4 * k], D[4 * k + 1], D[4 * k + 2]);
                if constexpr (T == Q6_K) {
                    const int t = k + 4 * th;
                    if (t < NP) {
                        const float2 mt = meta[xg * NP + t];
                        acc[t] += mt.x * (factor * Gs);
                    }
                } else if (2 * k < NP) {
                    const int t = 2 * k + h < NP ? 2 * k + h : 0;
                    const float2 mt = meta[xg * NP + t];
                    if constexpr (T == Q4_K) acc[k] += mt.x * (factor * Gs) - bias * mt.y;
                    else acc[k] += mt.x * (factor * Gs);
                }
            }
        }
        // Keep each sub-block's MFMA next to its epilogue (bounds the live
        // accumulator registers).
        __builtin_amdgcn_sched_barrier(0);
    }
}

// One workgroup per 32-row tile; groups [g0c, g0c + ngc) of every row (one
// column chunk). N = 1 (G false): x is this chunk's columns of the single
// token; otherwise dig/meta hold the chunk's digits for np = NP slots.
template <unsigned T, int NP, int KS, bool G>
__global__ __launch_bounds__(64 * KS) void smalln_mfma(const uint8_t *__restrict__ w, const float *__restrict__ x,
    const uint8_t *__restrict__ gdig, const float2 *__restrict__ gmeta, float *__restrict__ y, int rows, int cols,
    int g0c, int ngc, int n, int accumulate)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[KS][8][64];
    const int ccols = (g0c + ngc) * kGroupCols < cols ? ngc * kGroupCols : cols - g0c * kGroupCols;
    const int xgroups = ccols / 32;
    float2 *smeta = (float2 *)lds;                               // [xgroup][NP]
    uint8_t *sdig = lds + (size_t)8 * NP * ((xgroups + 1) & ~1); // N = 1: [xgroup][4 slots][32 B]

    const size_t row_bytes = tiled_row_bytes<T>(cols);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x, R = rows - kTileRows * t < kTileRows ? rows - kTileRows * t : kTileRows;
    Lane L;
    L.tile = w + (size_t)kTileRows * t * row_bytes;
    L.R = R;
    L.r = (lane & 31) < R ? (lane & 31) : R - 1;
    L.h = lane >> 5;
    L.slot = lane & 31;
    L.groups = (cols + kGroupCols - 1) / kGroupCols;
    L.blocks = cols / 32;
    // This wave's groups [s0, s1) of the chunk.
    const int s0 = g0c + wave * ngc / KS, s1 = g0c + (wave + 1) * ngc / KS, ns = s1 - s0;
    const int last = ns > 0 ? s1 - 1 : g0c;
    auto clamp = [&](int g) { return g <= last ? g : last; };

    // 1. Activations first.
    constexpr int kPre = 2;   // x items (8 values) per lane issued ahead (N = 1)
    const int i0 = 32 * (s0 - g0c);
    const int items = ns > 0 ? (32 * s1 < 4 * xgroups + 32 * g0c ? 32 * ns : 4 * xgroups - i0) : 0;
    float4 px[kPre][2];
    float2 pm[2];
    if constexpr (!G) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int it = i0 + (lane + 64 * k < items ? lane + 64 * k : 0);
            const float4 *src = (const float4 *)x + 2 * (it < 4 * xgroups ? it : 0);
            px[k][0] = src[0];
            px[k][1] = src[1];
        }
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = threadIdx.x + 64 * KS * k;
            pm[k] = gmeta[i < xgroups * NP ? i : 0];
        }
    }
    asm volatile("" ::: "memory");
    // 2. Both weight stages.
    Stage<T, NP, G> st0, st1;
    load_stage<T, NP, G>(st0, L, clamp(s0), g0c, gdig, n);
    load_stage<T, NP, G>(st1, L, clamp(s0 + 1), g0c, gdig, n);
    // 3. Activations into LDS (waits for them only).
    if constexpr (!G) {
#pragma unroll
        for (int k = 0; k < kPre; ++k)
            asm volatile("" : "+v"(px[k][0].x), "+v"(px[k][0].y), "+v"(px[k][0].z), "+v"(px[k][0].w),
                         "+v"(px[k][1].x), "+v"(px[k][1].y), "+v"(px[k][1].z), "+v"(px[k][1].w) :: "memory");
        // Items are whole 4-lane groups: lanes of one group share validity.
#pragma unroll
        for (int k = 0; k < kPre; ++k)
            if (lane + 64 * k < items) quantize8(px[k][0], px[k][1], 1, 0, i0 + lane + 64 * k, sdig, smeta);
        for (int k = 64 * kPre; k < items; k += 64)
            if (lane + k < items) {
                const float4 *src = (const float4 *)x + 2 * (i0 + lane + k);
                quantize8(src[0], src[1], 1, 0, i0 + lane + k, sdig, smeta);
            }
        // Each wave reads back only the groups it wrote.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        asm volatile("" : "+v"(pm[0].x), "+v"(pm[0].y), "+v"(pm[1].x), "+v"(pm[1].y) :: "memory");
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = threadIdx.x + 64 * KS * k;
            if (i < xgroups * NP) smeta[i] = pm[k];
        }
        for (int i = threadIdx.x + 128 * KS; i < xgroups * NP; i += 64 * KS) smeta[i] = gmeta[i];
        __syncthreads();
    }
    const uint8_t *dig = G ? gdig : sdig;

    // 4. Two-stage ring, branch-free: an odd count computes its last stage
    //    twice and drops the copy.
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < ns; i += 2) {
        float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        compute_stage<T, NP, G>(part, st0, L, clamp(s0 + i), g0c, dig, smeta, n);
        load_stage<T, NP, G>(st0, L, clamp(s0 + i + 2), g0c, gdig, n);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += part[k];
        float part1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        compute_stage<T, NP, G>(part1, st1, L, clamp(s0 + i + 1), g0c, dig, smeta, n);
        load_stage<T, NP, G>(st1, L, clamp(s0 + i + 3), g0c, gdig, n);
        const float keep = i + 1 < ns ? 1.f : 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += keep * part1[k];
    }

    // 5. Partial sums of the KS waves, added in wave order.
#pragma unroll
    for (int k = 0; k < 8; ++k) red[wave][k][lane] = acc[k];
    __syncthreads();
    if (wave != 0) return;
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        v[k] = red[0][k][lane];
        for (int q = 1; q < KS; ++q) v[k] += red[q][k][lane];
    }
    const int row = kTileRows * t + (lane & 31);
    const bool own = (lane & 31) < R;
    if constexpr (T == Q6_K) {
        // The two lane halves hold the two scale groups of each 32 columns.
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] += __shfl_xor(v[k], 32, 64);
#pragma unroll
        for (int k = 0; k < NP; ++k)
            if (own && k < n && (k & 1) == L.h) {
                float *dst = y + (size_t)k * rows + row;
                *dst = accumulate ? *dst + v[k] : v[k];
            }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int tok = 2 * k + L.h;
            if (own && 2 * k < NP && tok < n) {
                float *dst = y + (size_t)tok * rows + row;
                *dst = accumulate ? *dst + v[k] : v[k];
            }
        }
    }
}

// LDS bytes for a chunk of `ccols` columns.
size_t smalln_lds(int np, bool g, int ccols)
{
    const size_t xgroups = (size_t)ccols / 32;
    return 8 * np * ((xgroups + 1) & ~(size_t)1) + (g ? 0 : xgroups * 4 * kSlotBytes);
}

template <unsigned T, int NP, int KS>
hipError_t launch_chunk(const uint8_t *w, const float *x, const uint8_t *dig, const float2 *meta, float *y,
    int rows, int cols, int g0, int ng, int ccols, int n, int accumulate, hipStream_t s)
{
    constexpr bool G = NP > 1;
    const unsigned tiles = (unsigned)((rows + kTileRows - 1) / kTileRows);
    hipLaunchKernelGGL((smalln_mfma<T, NP, KS, G>), dim3(tiles), dim3(64 * KS), smalln_lds(NP, G, ccols), s,
        w, x, dig, meta, y, rows, cols, g0, ng, n, accumulate);
    return hipGetLastError();
}

template <unsigned T, int NP>
hipError_t launch_np(const uint8_t *w, const float *x, const uint8_t *dig, const float2 *meta, float *y,
    int rows, int cols, int g0, int ng, int ccols, int n, int accumulate, hipStream_t s)
{
    // Fewer than 256 tiles: more wavefronts per tile.
    if ((rows + kTileRows - 1) / kTileRows >= 256)
        return launch_chunk<T, NP, 4>(w, x, dig, meta, y, rows, cols, g0, ng, ccols, n, accumulate, s);
    return launch_chunk<T, NP, 8>(w, x, dig, meta, y, rows, cols, g0, ng, ccols, n, accumulate, s);
}

template <unsigned T>
hipError_t launch_type(int np, const uint8_t *w, const float *x, const uint8_t *dig, const float2 *meta, float *y,
    int rows, int cols, int g0, int ng, int ccols, int n, int accumulate, hipStream_t s)
{
    switch (np) {
    case 1: return launch_np<T, 1>(w, x, dig, meta, y, rows, cols, g0, ng, ccols, n, accumulate, s);
    case 2: return launch_np<T, 2>(w, x, dig, meta, y, rows, cols, g0, ng, ccols, n, accumulate, s);
    case 4: return launch_np<T, 4>(w, x, dig, meta, y, rows, cols, g0, ng, ccols, n, accumulate, s);
    default: return launch_np<T, 8>(w, x, dig, meta, y, rows, cols, g0, ng, ccols, n, accumulate, s);
    }
}

int padded_tokens(int n)
{
    return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8;
}

}  // namespace

size_t smalln_workspace(int cols, int batch)
{
    const int np = padded_tokens(batch);
    if (np == 1) return 0;
    const size_t ccols = (size_t)(cols < kChunkCols ? cols : kChunkCols);
    return ccols / 32 * (size_t)(4 * kSlotBytes + 8) * np;
}

hipError_t launch_smalln(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, int batch,
    void *workspace, hipStream_t s)
{
    const int np = padded_tokens(batch);
    const int groups = (cols + kGroupCols - 1) / kGroupCols;
    for (int g0 = 0; g0 < groups; g0 += kChunkCols / kGroupCols) {
        const int ng = groups - g0 < kChunkCols / kGroupCols ? groups - g0 : kChunkCols / kGroupCols;
        const int c0 = g0 * kGroupCols, ccols = cols - c0 < ng * kGroupCols ? cols - c0 : ng * kGroupCols;
        uint8_t *dig = (uint8_t *)workspace;
        float2 *meta = dig ? (float2 *)(dig + (size_t)ccols / 32 * 4 * kSlotBytes * np) : nullptr;
        if (np > 1) {
            const int total = batch * ccols / 8;
            hipLaunchKernelGGL(quantize_x, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                x + c0, cols, ccols, batch, np, dig, meta);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        hipError_t e;
        switch (type) {
        case Q4_K: e = launch_type<Q4_K>(np, w, x + c0, dig, meta, y, rows, cols, g0, ng, ccols, batch, g0 > 0, s); break;
        case Q6_K: e = launch_type<Q6_K>(np, w, x + c0, dig, meta, y, rows, cols, g0, ng, ccols, batch, g0 > 0, s); break;
        case Q8_0: e = launch_type<Q8_0>(np, w, x + c0, dig, meta, y, rows, cols, g0, ng, ccols, batch, g0 > 0, s); break;
        case Q4_0: e = launch_type<Q4_0>(np, w, x + c0, dig, meta, y, rows, cols, g0, ng, ccols, batch, g0 > 0, s); break;
        default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace fy
