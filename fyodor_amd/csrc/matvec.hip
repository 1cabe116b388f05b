// Batch 1..8 products of GGUF block-quantized weights with fp32 activations:
// the decode matvec (batch 1) and the small-N path (batch 2..8).
//
// Arithmetic. Each 32-element group of an activation column is written
// exactly as x_k = X_k * 2^e with one power-of-two scale per group and
// integers |X_k| <= 2^22 (X_k = rint(x_k * 2^-e), e chosen from the group's
// largest magnitude), and X_k is split into three signed 8-bit digits,
// X = a2*2^16 + a1*2^8 + a0. A block dot sum_k q_k x_k then becomes
//     2^e * (2^16 sum q a2 + 2^8 sum q a1 + sum q a0),
// three v_dot4_i32_i8 chains over the unpacked quants that are exact in
// int32. Only the per-block scales (d*sc, dmin*m) and the sum over blocks
// use fp32. The representation error of x is at most 2^-23 of the group's
// largest magnitude, below the rounding of an fp32 sum of the same terms;
// the block formulas are those of backend/core/llm_quant.c:206-311:
//   Q8_0  d * sum q x                      (q signed)
//   Q4_0  d * sum (q - 8) x                (-8 * sum X folded into the chain)
//   Q4_K  d*sc * sum q x - dmin*m * sum x  (per 32-element sub-block)
//   Q6_K  d*sc * sum (q6 - 32) x           (per 16-element sub-block)
//
// Work split. A 512-thread workgroup (8 wavefronts) first quantizes the
// activation columns of one column chunk into LDS, then each wavefront owns
// R consecutive rows and its 64 lanes own one unit of columns each (64
// elements of a K-quant superblock or one 32-element Q8_0/Q4_0 block): a
// lane issues the 16-byte loads of its unit for all R rows before the
// workgroup quantizes x, so the weight stream is in flight from the first
// cycles; it then unpacks in registers, runs the dot chains for each column
// and finally the wavefront reduces the per-lane sums of each row.
#include "device.h"
#include "formats.h"
#include "kernels.h"

namespace fy {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;

// Per 32-element activation group: the scale 2^e, sum_k X_k * 2^e, and the
// digit sums of each 16-element half (for the -8 / -32 quant offsets).
struct XGroup {
    float scale;
    float sx;
    int s16[2][3];
};
static_assert(sizeof(XGroup) == 32, "XGroup is 32 bytes");

template <unsigned T> struct Unit { static constexpr int elems = 64, runs = 4; };
template <> struct Unit<Q8_0> { static constexpr int elems = 32, runs = 2; };
template <> struct Unit<Q4_0> { static constexpr int elems = 32, runs = 2; };

// Unit and 16-element run of chunk-local element e: the run order is the
// order in which a lane's quants meet the activations.
template <unsigned T>
__device__ __forceinline__ void locate(int e, int &unit, int &run)
{
    if constexpr (T == Q4_K) {
        unit = e >> 6;                 // (superblock, nibble pair)
        run = (e >> 4) & 3;            // low group halves, then high group halves
    } else if constexpr (T == Q6_K) {
        const int w = e & 255;         // 128h + 32q + 16*l16 + i
        unit = 4 * (e >> 8) + 2 * (w >> 7) + ((w >> 4) & 1);
        run = (w >> 5) & 3;            // quarter q
    } else {
        unit = e >> 5;
        run = (e >> 4) & 1;
    }
}

// LDS layout for one column chunk of kc elements and `units` units:
//   digits: for each column n, plane p (0 = a0, 1 = a1, 2 = a2), run r,
//           unit u: 16 bytes at ((n*3 + p)*runs + r)*units + u (x16),
//           so the lanes of a wavefront read consecutive 16-byte slots;
//   groups: XGroup[n][kc/32] after all digits.
template <unsigned T>
__device__ __forceinline__ int digit_slot(int n, int plane, int run, int unit, int units)
{
    return ((n * 3 + plane) * Unit<T>::runs + run) * units + unit;
}

__device__ __forceinline__ int sext8(int v) { return (int)(int8_t)(v & 0xFF); }

// Quantize 8 consecutive activations (elements e0..e0+7 of column n of a
// chunk of kc elements) into LDS. Four consecutive lanes hold the four
// quarters of one 32-element group and must call this together.
template <unsigned T>
__device__ __forceinline__ void quantize_item(const float (&val)[8], int n, int e0, int kc,
    uint4 *digits, XGroup *groups, bool store = true)
{
    const int units = kc / Unit<T>::elems;
    float m = 0.f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        m = fmaxf(m, fabsf(val[i]));
        bad |= !(fabsf(val[i]) <= 3.4028235e38f);   // inf or NaN
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    int ex = 0;
    (void)__builtin_frexpf(m, &ex);          // m in [2^(ex-1), 2^ex)
    // A non-finite activation makes its whole group NaN, so every output
    // that depends on it is NaN.
    const bool finite = !bad;
    const int shift = m > 0.f && finite ? 22 - ex : 0;
    const float scale = !finite ? __builtin_nanf("") : m > 0.f ? __builtin_ldexpf(1.f, ex - 22) : 0.f;
    int sx = 0, s[3] = {0, 0, 0};
    uint32_t packed[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int X = finite ? (int)__builtin_rintf(__builtin_ldexpf(val[i], shift)) : 0;
        const int a0 = sext8(X);
        const int r1 = (X - a0) >> 8;
        const int a1 = sext8(r1);
        const int a2 = (r1 - a1) >> 8;
        sx += X;
        s[0] += a0; s[1] += a1; s[2] += a2;
        packed[0][i >> 2] |= (uint32_t)(a0 & 0xFF) << (8 * (i & 3));
        packed[1][i >> 2] |= (uint32_t)(a1 & 0xFF) << (8 * (i & 3));
        packed[2][i >> 2] |= (uint32_t)(a2 & 0xFF) << (8 * (i & 3));
    }
    int unit, run;
    locate<T>(e0, unit, run);
    uint8_t *bytes = (uint8_t *)digits;
    if (store) {
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            uint2 *dst = (uint2 *)(bytes + 16 * digit_slot<T>(n, p, run, unit, units) + (e0 & 15));
            *dst = make_uint2(packed[p][0], packed[p][1]);
        }
    }
    // Digit sums per 16-element half (lane pairs), X sums per group (quads).
#pragma unroll
    for (int p = 0; p < 3; ++p) s[p] += __shfl_xor(s[p], 1, 64);
    sx += __shfl_xor(sx, 1, 64);
    sx += __shfl_xor(sx, 2, 64);
    int hi[3];
#pragma unroll
    for (int p = 0; p < 3; ++p) hi[p] = __shfl_down(s[p], 2, 64);
    if (store && (threadIdx.x & 3) == 0) {
        XGroup g;
        g.scale = scale;
        g.sx = (float)sx * scale;
#pragma unroll
        for (int p = 0; p < 3; ++p) { g.s16[0][p] = s[p]; g.s16[1][p] = hi[p]; }
        groups[n * (kc / 32) + (e0 >> 5)] = g;
    }
}

__device__ __forceinline__ void load_item(float (&val)[8], const float *__restrict__ x, int cols, int k0,
    int per_col, int t)
{
    const int n = t / per_col, e0 = 8 * (t - n * per_col);
    const float4 *src = (const float4 *)(x + (size_t)n * cols + k0 + e0);
    const float4 u = src[0], v = src[1];
    val[0] = u.x; val[1] = u.y; val[2] = u.z; val[3] = u.w;
    val[4] = v.x; val[5] = v.y; val[6] = v.z; val[7] = v.w;
}

// Quantize columns [k0, k0 + kc) of the N activation columns into LDS, 8
// elements per thread and item; the first PRE items of each thread come
// from `pre`, loaded by prefetch_x before the weight loads were issued.
template <int PRE>
struct XPrefetch { float v[PRE][8]; };

// Loads are issued unconditionally (surplus items reload item 0) so the
// number of outstanding vector loads is the same on every path and the
// waits that follow can be exact.
// Orders the activation prefetch before the weight loads and the
// quantization after them: the asm consumes the prefetched registers (so the
// wait inserted before it covers exactly the older activation loads), and its
// memory clobber keeps the weight loads above it.
template <int PRE>
__device__ __forceinline__ void after_weight_loads(XPrefetch<PRE> &pre)
{
#pragma unroll
    for (int i = 0; i < PRE; ++i)
        asm volatile("" : "+v"(pre.v[i][0]), "+v"(pre.v[i][1]), "+v"(pre.v[i][2]), "+v"(pre.v[i][3]),
                          "+v"(pre.v[i][4]), "+v"(pre.v[i][5]), "+v"(pre.v[i][6]), "+v"(pre.v[i][7])
                     :: "memory");
}

template <int N, int PRE>
__device__ __forceinline__ void prefetch_x(XPrefetch<PRE> &pre, const float *__restrict__ x, int cols, int k0, int kc)
{
    const int per_col = kc / 8, items = N * per_col;
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
        const int t = threadIdx.x + i * blockDim.x;
        load_item(pre.v[i], x, cols, k0, per_col, t < items ? t : 0);
    }
}

template <unsigned T, int N, int PRE>
__device__ __forceinline__ void prepare_x(const XPrefetch<PRE> &pre, const float *__restrict__ x, int cols,
    int k0, int kc, uint4 *digits, XGroup *groups)
{
    const int per_col = kc / 8, items = N * per_col;
    // Every thread quantizes its PRE prefetched items (surplus ones compute
    // item 0 and store nothing): no branch lets the compiler sink the
    // prefetch loads below the weight loads.
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
        const int t = threadIdx.x + i * blockDim.x;
        const bool valid = t < items;
        const int tv = valid ? t : 0;
        quantize_item<T>(pre.v[i], tv / per_col, 8 * (tv % per_col), kc, digits, groups, valid);
    }
    for (int t = threadIdx.x + PRE * blockDim.x; t < items; t += blockDim.x) {
        float val[8];
        load_item(val, x, cols, k0, per_col, t);
        quantize_item<T>(val, t / per_col, 8 * (t % per_col), kc, digits, groups);
    }
}

// ---- per-format weight units -------------------------------------------

struct RawQ4K { uint4 qa, qb; uint32_t slice; };
struct RawQ6K { uint4 la, lb, qh; uint32_t sc, d; };
struct RawQ8 { uint4 qa, qb; uint32_t d; };
struct RawQ4 { uint4 q; uint32_t d; };

template <unsigned T> struct RawOf;
template <> struct RawOf<Q4_K> { using type = RawQ4K; };
template <> struct RawOf<Q6_K> { using type = RawQ6K; };
template <> struct RawOf<Q8_0> { using type = RawQ8; };
template <> struct RawOf<Q4_0> { using type = RawQ4; };

// Load unit `unit` (row-global index) of row `row` from the field planes of
// the device layout (formats.h): consecutive lanes read consecutive slices.
template <unsigned T>
__device__ __forceinline__ void load_unit(typename RawOf<T>::type &raw, const uint8_t *__restrict__ w,
    int rows, int cols, int row, int unit)
{
    const size_t U = (size_t)(cols / Unit<T>::elems), n = (size_t)rows * U, at = (size_t)row * U + unit;
    if constexpr (T == Q4_K) {
        raw.qa = ((const uint4 *)w)[at];
        raw.qb = ((const uint4 *)(w + 16 * n))[at];
        raw.slice = ((const uint32_t *)(w + 32 * n))[at];
    } else if constexpr (T == Q6_K) {
        raw.la = ((const uint4 *)w)[at];
        raw.lb = ((const uint4 *)(w + 16 * n))[at];
        raw.qh = ((const uint4 *)(w + 32 * n))[at];
        raw.sc = ((const uint32_t *)(w + 48 * n))[at];
        raw.d = ((const uint16_t *)(w + 52 * n))[at >> 2];
    } else if constexpr (T == Q8_0) {
        raw.qa = ((const uint4 *)w)[at];
        raw.qb = ((const uint4 *)(w + 16 * n))[at];
        raw.d = ((const uint16_t *)(w + 32 * n))[at];
    } else {
        raw.q = ((const uint4 *)w)[at];
        raw.d = ((const uint16_t *)(w + 16 * n))[at];
    }
}

// `top` of lane i of this lane's quad (DPP quad broadcast).
__device__ __forceinline__ uint32_t quad_byte(uint32_t top, int i)
{
    switch (i) {
    case 0: return (uint32_t)__builtin_amdgcn_mov_dpp((int)top, 0x00, 0xF, 0xF, false);
    case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)top, 0x55, 0xF, 0xF, false);
    case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)top, 0xAA, 0xF, 0xF, false);
    default: return (uint32_t)__builtin_amdgcn_mov_dpp((int)top, 0xFF, 0xF, 0xF, false);
    }
}

__device__ __forceinline__ int dot4(uint32_t q, uint32_t a, int acc)
{
    return __builtin_amdgcn_sdot4((int)q, (int)a, acc, false);
}

// Dot of one unit of one row with one activation column whose digit slots
// (dg[plane][run]) and groups are given. `unit` is chunk-local.
template <unsigned T>
__device__ __forceinline__ float unit_dot(const typename RawOf<T>::type &raw, const uint4 (&dg)[3][Unit<T>::runs],
    const XGroup *groups, int unit);

template <>
__device__ __forceinline__ float unit_dot<Q4_K>(const RawQ4K &raw, const uint4 (&dg)[3][4], const XGroup *groups, int unit)
{
    // Sub-blocks 2p and 2p+1 (backend/core/llm_quant.c:249-251): the
    // unit's slice holds their 6-bit scales and minimums; d and dmin are
    // spread one byte per lane over the superblock's four lanes.
    const uint32_t sc0 = raw.slice & 63u, m0 = (raw.slice >> 6) & 63u;
    const uint32_t sc1 = (raw.slice >> 12) & 63u, m1 = (raw.slice >> 18) & 63u;
    const uint32_t top = raw.slice >> 24;
    const uint32_t dd = quad_byte(top, 0) | quad_byte(top, 1) << 8 | quad_byte(top, 2) << 16 | quad_byte(top, 3) << 24;
    const float d = f16_to_f32(dd & 0xFFFFu), dmin = f16_to_f32(dd >> 16);
    int l0 = 0, l1 = 0, l2 = 0, h0 = 0, h1 = 0, h2 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t dw = j < 4 ? word_of(raw.qa, j) : word_of(raw.qb, j - 4);
        const uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
        const int rl = j >> 2, rh = 2 + (j >> 2), c = j & 3;
        l0 = dot4(lo, word_of(dg[0][rl], c), l0);
        l1 = dot4(lo, word_of(dg[1][rl], c), l1);
        l2 = dot4(lo, word_of(dg[2][rl], c), l2);
        h0 = dot4(hi, word_of(dg[0][rh], c), h0);
        h1 = dot4(hi, word_of(dg[1][rh], c), h1);
        h2 = dot4(hi, word_of(dg[2][rh], c), h2);
    }
    // |l2| <= 32*15*64, so the combined sums stay inside int32.
    const int gl = l2 * 65536 + l1 * 256 + l0, gh = h2 * 65536 + h1 * 256 + h0;
    const XGroup &g0 = groups[2 * unit], &g1 = groups[2 * unit + 1];
    const float lo_part = g0.scale * ((d * (float)sc0) * (float)gl) - (dmin * (float)m0) * g0.sx;
    const float hi_part = g1.scale * ((d * (float)sc1) * (float)gh) - (dmin * (float)m1) * g1.sx;
    return lo_part + hi_part;
}

template <>
__device__ __forceinline__ float unit_dot<Q6_K>(const RawQ6K &raw, const uint4 (&dg)[3][4], const XGroup *groups, int unit)
{
    // Elements 128h + 32q + 16*l16 + i; quarter q uses sc[8h + 2q + l16]
    // (backend/core/llm_quant.c:256-270) and group 8s + 4h + q of x.
    const int h = (unit >> 1) & 1, l16 = unit & 1;
    const XGroup *g = groups + 8 * (unit >> 2) + 4 * h;
    const float d = f16_to_f32(raw.d);
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int8_t sc = (int8_t)((raw.sc >> (8 * q)) & 0xFFu);
        int c0 = -32 * g[q].s16[l16][0], c1 = -32 * g[q].s16[l16][1], c2 = -32 * g[q].s16[l16][2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t ql = word_of((q & 1) ? raw.lb : raw.la, j);
            const uint32_t v = ((ql >> (4 * (q >> 1))) & 0x0F0F0F0Fu) |
                (((word_of(raw.qh, j) >> (2 * q)) & 0x03030303u) << 4);
            c0 = dot4(v, word_of(dg[0][q], j), c0);
            c1 = dot4(v, word_of(dg[1][q], j), c1);
            c2 = dot4(v, word_of(dg[2][q], j), c2);
        }
        const float G = (float)c2 * 65536.f + ((float)c1 * 256.f + (float)c0);
        sum += g[q].scale * ((d * (float)sc) * G);
    }
    return sum;
}

template <>
__device__ __forceinline__ float unit_dot<Q8_0>(const RawQ8 &raw, const uint4 (&dg)[3][2], const XGroup *groups, int unit)
{
    int c0 = 0, c1 = 0, c2 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t q = j < 4 ? word_of(raw.qa, j) : word_of(raw.qb, j - 4);
        const int r = j >> 2, c = j & 3;
        c0 = dot4(q, word_of(dg[0][r], c), c0);
        c1 = dot4(q, word_of(dg[1][r], c), c1);
        c2 = dot4(q, word_of(dg[2][r], c), c2);
    }
    const float G = (float)c2 * 65536.f + ((float)c1 * 256.f + (float)c0);
    return groups[unit].scale * (f16_to_f32(raw.d) * G);
}

template <>
__device__ __forceinline__ float unit_dot<Q4_0>(const RawQ4 &raw, const uint4 (&dg)[3][2], const XGroup *groups, int unit)
{
    const XGroup &g = groups[unit];
    int c0 = -8 * (g.s16[0][0] + g.s16[1][0]);
    int c1 = -8 * (g.s16[0][1] + g.s16[1][1]);
    int c2 = -8 * (g.s16[0][2] + g.s16[1][2]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t dw = word_of(raw.q, j);
        const uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
        c0 = dot4(lo, word_of(dg[0][0], j), c0);
        c1 = dot4(lo, word_of(dg[1][0], j), c1);
        c2 = dot4(lo, word_of(dg[2][0], j), c2);
        c0 = dot4(hi, word_of(dg[0][1], j), c0);
        c1 = dot4(hi, word_of(dg[1][1], j), c1);
        c2 = dot4(hi, word_of(dg[2][1], j), c2);
    }
    // |c2| <= 32*8*64, so the combined sum stays inside int32.
    const int G = c2 * 65536 + c1 * 256 + c0;
    return g.scale * (f16_to_f32(raw.d) * (float)G);
}

template <unsigned T, int N, int R>
__global__ __launch_bounds__(kThreads) void quant_chunked(const uint8_t *__restrict__ w,
    const float *__restrict__ x, float *__restrict__ y, int rows, int cols, int chunk)
{
    using Raw = typename RawOf<T>::type;
    constexpr int UE = Unit<T>::elems, RUNS = Unit<T>::runs;
    extern __shared__ __align__(16) uint4 lds[];
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
    const int nrow = rows - row0 < R ? rows - row0 : R;
    float acc[R][N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < N; ++n) acc[r][n] = 0.f;

    Raw raw[R];
    const int first_units = (cols < chunk ? cols : chunk) / UE;
    if (lane < first_units) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r < nrow) load_unit<T>(raw[r], w, rows, cols, row0 + r, lane);
    }
    for (int k0 = 0; k0 < cols; k0 += chunk) {
        const int kc = cols - k0 < chunk ? cols - k0 : chunk;
        const int units = kc / UE, base_unit = k0 / UE;
        uint4 *digits = lds;
        XGroup *groups = (XGroup *)(lds + N * 3 * RUNS * units);
        __syncthreads();
        XPrefetch<1> pre;
        prefetch_x<N, 1>(pre, x, cols, k0, kc);
        prepare_x<T, N, 1>(pre, x, cols, k0, kc, digits, groups);
        __syncthreads();
        for (int u = lane; u < units; u += 64) {
            if (k0 != 0 || u != lane) {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (r < nrow) load_unit<T>(raw[r], w, rows, cols, row0 + r, base_unit + u);
            }
#pragma unroll
            for (int n = 0; n < N; ++n) {
                uint4 dg[3][RUNS];
#pragma unroll
                for (int p = 0; p < 3; ++p)
#pragma unroll
                    for (int q = 0; q < RUNS; ++q) dg[p][q] = digits[digit_slot<T>(n, p, q, u, units)];
                const XGroup *gn = groups + n * (kc / 32);
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (r < nrow) acc[r][n] += unit_dot<T>(raw[r], dg, gn, u);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const float v = wave_sum(acc[r][n]);
            if (lane == 0 && r < nrow) y[(size_t)n * rows + row0 + r] = v;
        }
}

// One pass: each lane owns at most one unit of each of its R rows, so all of
// a wavefront's weight loads are in flight before the activations are
// quantized. The workgroup's wavefronts form `split` column slices (split-K)
// of (waves / split) row groups; slices of a row group add their per-wave
// sums through LDS in a fixed order.
template <unsigned T, int N, int R, int PRE, int D>
__global__ __launch_bounds__(kThreads) void quant_rows(const uint8_t *__restrict__ w,
    const float *__restrict__ x, float *__restrict__ y, int rows, int cols, int split)
{
    using Raw = typename RawOf<T>::type;
    constexpr int UE = Unit<T>::elems, RUNS = Unit<T>::runs;
    extern __shared__ __align__(16) uint4 lds[];
    const int units = cols / UE;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slice = wave % split, group = wave / split;
    const int groups_per_block = (int)(blockDim.x >> 6) / split;
    const int row0 = (blockIdx.x * groups_per_block + group) * R;
    const int nrow = rows - row0 < R ? (rows - row0 > 0 ? rows - row0 : 0) : R;
    const int unit = slice * 64 + lane;
    const bool owns = unit < units;

    // Activation loads first: vector loads retire in order, so the
    // quantization below waits only for these, not for the weight stream.
    // Every lane loads R units; lanes past the row end and rows past the
    // matrix end reload a valid unit whose result is discarded, which keeps
    // the load count static (see prefetch_x).
    XPrefetch<PRE> pre;
    prefetch_x<N, PRE>(pre, x, cols, 0, cols);
    uint4 *digits = lds;
    XGroup *groups = (XGroup *)(lds + N * 3 * RUNS * units);
    float *partial = (float *)(groups + N * (cols / 32));
    float acc[R][N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < N; ++n) acc[r][n] = 0.f;
    auto row_of = [&](int r) { return row0 + r < rows ? row0 + r : rows - 1; };

    if constexpr (N == 1) {
        // Decode: a ring of D rows in flight per wavefront. Row r+D is
        // requested before row r is computed, so each wavefront alternates
        // between waiting on memory and computing instead of queueing all
        // its requests up front (which blocks instruction issue until most
        // of them have returned).
        Raw ring[D];
#pragma unroll
        for (int i = 0; i < D && i < R; ++i) load_unit<T>(ring[i], w, rows, cols, row_of(i), owns ? unit : 0);
        after_weight_loads(pre);
        prepare_x<T, N, PRE>(pre, x, cols, 0, cols, digits, groups);
        __syncthreads();
        uint4 dg[3][RUNS];
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int q = 0; q < RUNS; ++q) dg[p][q] = digits[digit_slot<T>(0, p, q, owns ? unit : 0, units)];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const Raw cur = ring[r % D];
            if (r + D < R) load_unit<T>(ring[r % D], w, rows, cols, row_of(r + D), owns ? unit : 0);
            const float v = unit_dot<T>(cur, dg, groups, owns ? unit : 0);
            acc[r][0] = owns && r < nrow ? v : 0.f;
            // Row r is finished here and row r+D+1 is requested only after:
            // the asm consumes the result and no load may cross it.
            asm volatile("" : "+v"(acc[r][0]) :: "memory");
        }
    } else {
        // Small N: all R rows resident, activation columns in the outer loop
        // so each column's digits are read from LDS once per R rows.
        Raw raw[R];
#pragma unroll
        for (int r = 0; r < R; ++r) load_unit<T>(raw[r], w, rows, cols, row_of(r), owns ? unit : 0);
        after_weight_loads(pre);
        prepare_x<T, N, PRE>(pre, x, cols, 0, cols, digits, groups);
        __syncthreads();
        if (owns) {
#pragma unroll
            for (int n = 0; n < N; ++n) {
                uint4 dg[3][RUNS];
#pragma unroll
                for (int p = 0; p < 3; ++p)
#pragma unroll
                    for (int q = 0; q < RUNS; ++q) dg[p][q] = digits[digit_slot<T>(n, p, q, unit, units)];
                const XGroup *gn = groups + n * (cols / 32);
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (r < nrow) acc[r][n] = unit_dot<T>(raw[r], dg, gn, unit);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const float v = wave_sum(acc[r][n]);
            if (lane == 0) {
                if (split == 1) {
                    if (r < nrow) y[(size_t)n * rows + row0 + r] = v;
                } else {
                    partial[(wave * R + r) * N + n] = v;
                }
            }
        }
    if (split > 1) {
        __syncthreads();
        if (slice == 0 && lane < R * N) {
            const int r = lane / N, n = lane - r * N;
            float sum = 0.f;
            for (int k = 0; k < split; ++k) sum += partial[((group * split + k) * R + r) * N + n];
            if (r < nrow) y[(size_t)n * rows + row0 + r] = sum;
        }
    }
}

// Largest LDS a workgroup may use, from the device (64 KiB if unknown).
int lds_limit()
{
    static int limit = 0;
    if (!limit) {
        int device = 0, value = 0;
        if (hipGetDevice(&device) != hipSuccess ||
            hipDeviceGetAttribute(&value, hipDeviceAttributeMaxSharedMemoryPerBlock, device) != hipSuccess ||
            value < 65536)
            value = 65536;
        limit = value;
    }
    return limit;
}

hipError_t allow_lds(const void *kernel, size_t shared)
{
    if (shared <= 65536) return hipSuccess;
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shared);
}

// Fallback for rows wider than 8 x 64 units or activations larger than LDS:
// the activations are quantized one LDS-sized column chunk at a time.
template <unsigned T, int N, int R>
hipError_t launch_chunked(const uint8_t *w, const float *x, float *y, int rows, int cols, hipStream_t s)
{
    constexpr int UE = Unit<T>::elems;
    // 4 bytes of LDS per element and column (3 digit planes + one 32-byte
    // group record per 32 elements); chunks are multiples of 256 columns.
    int chunk = lds_limit() / (4 * N) / 256 * 256;
    if (chunk > cols) chunk = cols;
    if (chunk < UE) return hipErrorInvalidValue;
    const size_t shared = (size_t)4 * N * chunk;
    auto kernel = quant_chunked<T, N, R>;
    hipError_t e = allow_lds((const void *)kernel, shared);
    if (e != hipSuccess) return e;
    const int per_block = kWaves * R;
    const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), shared, s, w, x, y, rows, cols, chunk);
    return hipGetLastError();
}

template <unsigned T, int N, int R, int PRE, int D = 3>
hipError_t launch_one_pass(const uint8_t *w, const float *x, float *y, int rows, int cols, int split,
    hipStream_t s)
{
    const int groups = kWaves / split, threads = 64 * split * groups;
    const size_t shared = (size_t)4 * N * cols + sizeof(float) * (size_t)(threads / 64) * R * N;
    auto kernel = quant_rows<T, N, R, PRE, D>;
    hipError_t e = allow_lds((const void *)kernel, shared);
    if (e != hipSuccess) return e;
    const int per_block = groups * R;
    const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
    hipLaunchKernelGGL(kernel, grid, dim3(threads), shared, s, w, x, y, rows, cols, split);
    return hipGetLastError();
}

// Shape policy: one pass when a row fits 8 wavefronts of units and the
// quantized activations fit LDS; rows per wavefront so that one round of
// workgroups covers the 256 CUs with as many bytes in flight as registers
// allow.
template <unsigned T, int N>
hipError_t launch_rows(const uint8_t *w, const float *x, float *y, int rows, int cols, hipStream_t s)
{
    constexpr int UE = Unit<T>::elems;
    const int units = cols / UE, split = (units + 63) / 64;
    const int groups = split <= kWaves ? kWaves / split : 0;
    const size_t shared = (size_t)4 * N * cols + sizeof(float) * 8 * 8 * N;
    if (groups == 0 || shared > (size_t)lds_limit()) {
        if (rows >= kWaves * 2 * 256) return launch_chunked<T, N, 2>(w, x, y, rows, cols, s);
        return launch_chunked<T, N, 1>(w, x, y, rows, cols, s);
    }
    const int threads = 64 * split * groups;
    const bool many = N * cols / 8 > threads;   // more than one activation item per thread
    const int per = rows / (groups * 256);
    if constexpr (N == 1) {
        // One round of workgroups over the 256 CUs (up to 8 rows per
        // wavefront), two rows in flight per wavefront; measured best for the
        // 14336 x 4096 decode projection against deeper rings, more
        // wavefronts per CU and fewer rows per wavefront.
        const int rpw = (rows + groups * 256 - 1) / (groups * 256);
        if (many) {
            if (rpw >= 4) return launch_one_pass<T, N, 4, 4, 2>(w, x, y, rows, cols, split, s);
            if (rpw >= 2) return launch_one_pass<T, N, 2, 4, 2>(w, x, y, rows, cols, split, s);
            return launch_one_pass<T, N, 1, 4, 1>(w, x, y, rows, cols, split, s);
        }
        switch (rpw) {
        case 1: return launch_one_pass<T, N, 1, 1, 1>(w, x, y, rows, cols, split, s);
        case 2: return launch_one_pass<T, N, 2, 1, 2>(w, x, y, rows, cols, split, s);
        case 3: return launch_one_pass<T, N, 3, 1, 2>(w, x, y, rows, cols, split, s);
        case 4: return launch_one_pass<T, N, 4, 1, 2>(w, x, y, rows, cols, split, s);
        case 5: return launch_one_pass<T, N, 5, 1, 2>(w, x, y, rows, cols, split, s);
        case 6: return launch_one_pass<T, N, 6, 1, 2>(w, x, y, rows, cols, split, s);
        case 7: return launch_one_pass<T, N, 7, 1, 2>(w, x, y, rows, cols, split, s);
        default: return launch_one_pass<T, N, 8, 1, 2>(w, x, y, rows, cols, split, s);
        }
    } else if constexpr (N <= 4) {
        if (per >= 4) return launch_one_pass<T, N, 4, N>(w, x, y, rows, cols, split, s);
        if (per >= 2) return launch_one_pass<T, N, 2, N>(w, x, y, rows, cols, split, s);
        return launch_one_pass<T, N, 1, N>(w, x, y, rows, cols, split, s);
    } else {
        if (per >= 2) return launch_one_pass<T, N, 2, N>(w, x, y, rows, cols, split, s);
        return launch_one_pass<T, N, 1, N>(w, x, y, rows, cols, split, s);
    }
}

template <unsigned T>
hipError_t launch_type(const uint8_t *w, const float *x, float *y, int rows, int cols, int batch, hipStream_t s)
{
    switch (batch) {
    case 1: return launch_rows<T, 1>(w, x, y, rows, cols, s);
    case 2: return launch_rows<T, 2>(w, x, y, rows, cols, s);
    case 3: return launch_rows<T, 3>(w, x, y, rows, cols, s);
    case 4: return launch_rows<T, 4>(w, x, y, rows, cols, s);
    case 5: return launch_rows<T, 5>(w, x, y, rows, cols, s);
    case 6: return launch_rows<T, 6>(w, x, y, rows, cols, s);
    case 7: return launch_rows<T, 7>(w, x, y, rows, cols, s);
    case 8: return launch_rows<T, 8>(w, x, y, rows, cols, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

const char *quant_matvec_kernel(unsigned type, int rows, int cols, int batch)
{
    (void)rows;
    const int elems = type == Q8_0 || type == Q4_0 ? 32 : 64;
    const int split = (cols / elems + 63) / 64;
    const size_t shared = (size_t)4 * batch * cols + sizeof(float) * 8 * 8 * batch;
    return split <= kWaves && shared <= (size_t)lds_limit() ? "quant_rows" : "quant_chunked";
}

hipError_t launch_quant_matvec(unsigned type, const uint8_t *w, const float *x, float *y,
    int rows, int cols, int batch, hipStream_t s)
{
    switch (type) {
    case Q4_0: return launch_type<Q4_0>(w, x, y, rows, cols, batch, s);
    case Q8_0: return launch_type<Q8_0>(w, x, y, rows, cols, batch, s);
    case Q4_K: return launch_type<Q4_K>(w, x, y, rows, cols, batch, s);
    case Q6_K: return launch_type<Q6_K>(w, x, y, rows, cols, batch, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace fy
