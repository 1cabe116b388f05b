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
// into signed 8-bit weights before the MFMA (scaled by 4 and 16, which the
// block scales take back).
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
// tile's 256-column groups; each streams its groups' weights through a
// two-stage register ring (a stage's loads issued two groups ahead), and the
// partial sums meet in LDS at the end. N = 1 quantizes each wavefront's own
// columns of x into LDS; N >= 2 reads digits written once per call by
// quantize_x into the workspace, one group ahead: the operand registers of a
// block are reloaded with the next group's as soon as the block's MFMA has
// issued (L2 hits need less lead than HBM weights, and one set of operand
// registers instead of one per stage keeps the wavefront within its register
// budget). Columns beyond kChunkCols run as further launches that add into y.
#include "blockdot.h"
#include "kernels.h"

namespace fy {
namespace {

constexpr int kChunkCols = 16384;   // columns per launch (bounds the LDS copy of x)

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

// MFMAs per 256-column group, and how many activation operands each needs.
template <unsigned T, int NP> constexpr int kTokenHalves = (T == Q6_K && NP > 4) ? 2 : 1;
// Weight stages in flight per wavefront (a third one measured slower).
template <unsigned T, int NP> constexpr int kRing = 2;
// Accumulators per lane: Q6_K lanes hold every token, the others every
// second one.
template <unsigned T, int NP> constexpr int kAcc = T == Q6_K ? NP : (NP + 1) / 2;
// Non-temporal weight loads: measured faster for the batch-1 matvec of Q4_K,
// Q6_K and Q4_0 (Q4_K 14336 x 4096: 8.5 -> 8.1 us), slower for Q8_0 (4096^2:
// 6.55 -> 7.4 us) and for batches of 2..8.
template <unsigned T, bool G> constexpr bool kStreamWeights = !G && T != Q8_0;

// Activation operands of one group (N >= 2): MFMA j, token half th at
// 8 th + j.
template <unsigned T, int NP, bool G> constexpr int kActs = G ? 8 * kTokenHalves<T, NP> : 1;

// Byte offset of the activation operand of MFMA j (token half th) of
// chunk-local group gl in the digit array. Lanes whose A-row is not live for
// n tokens read slot 3 of token 0, which is always zero.
template <unsigned T, int NP>
__device__ __forceinline__ int a_offset(const Lane &L, int gl, int j, int th, int n, int nb)
{
    const int row_bytes = 4 * kSlotBytes * NP;
    if constexpr (T == Q6_K) {
        const int p = j >> 1, m = j & 1;
        const int t = (L.slot >> 3) + 4 * th, c = (L.slot >> 2) & 1, d = L.slot & 3;
        const bool live = c == L.h && d < 3 && t < n;
        const int xg = 8 * gl + 4 * (p >> 1) + 2 * m + L.h;
        return xg * row_bytes + kSlotBytes * (live ? 4 * t + d : 3) + 16 * (p & 1);
    } else {
        const int jj = j < nb ? j : nb - 1;
        const bool live = (L.slot >> 2) < n;
        return (8 * gl + jj) * row_bytes + kSlotBytes * (live ? L.slot : 3) + 16 * L.h;
    }
}

// Activation operands j0 .. j0 + cnt - 1 (every token half) of group g.
template <unsigned T, int NP, bool G>
__device__ __forceinline__ void load_acts(i32x4 (&a)[(kActs<T, NP, G>)], const Lane &L, int g, int g0c, int j0,
    int cnt, const uint8_t *__restrict__ dig, int n)
{
    if constexpr (G) {
        const int nb = (T == Q8_0 || T == Q4_0) ? group_blocks(L, g) : 8;
#pragma unroll
        for (int th = 0; th < kTokenHalves<T, NP>; ++th)
#pragma unroll
            for (int j = j0; j < j0 + cnt; ++j)
                a[8 * th + j] = *(const i32x4 *)(dig + a_offset<T, NP>(L, g - g0c, j, th, n, nb));
    }
}

// The block dot products of one stage (group g) into acc. Q4_K/Q8_0/Q4_0:
// acc[k] belongs to token 2k + h; Q6_K: acc[t] to token t (this lane half's
// scale groups). The K-quant superblock scales d and dmin multiply the
// group's sums once: sum_j (d sc_j q - dmin m_j) x = d sum_j sc_j (q.x)_j -
// dmin sum_j m_j (sum x)_j. N >= 2: a holds group g's activation operands;
// each is reloaded with group gn's as soon as its MFMA has issued, so one set
// of operand registers serves the whole ring.
template <unsigned T, int NP, bool G, bool FULL>
__device__ __forceinline__ void compute_stage(float (&acc)[(kAcc<T, NP>)], const WStage<T> &w,
    i32x4 (&acts)[(kActs<T, NP, G>)], const Lane &L, int g, int gn, int g0c, const uint8_t *dig, const float2 *meta,
    int n)
{
    constexpr int NA = kAcc<T, NP>;
    const int h = L.h;
    const int nb = (T == Q8_0 || T == Q4_0) && !FULL ? group_blocks(L, g) : 8;
    float sum_s[NA], sum_m[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) sum_s[k] = sum_m[k] = 0.f;
    // PAIR blocks at a time: both MFMAs issue before either epilogue reads a
    // result, so the second covers the first's latency (one at a time when a
    // block already takes two MFMAs).
    constexpr int PAIR = kTokenHalves<T, NP> == 1 ? 2 : 1;
#pragma unroll
    for (int j0 = 0; j0 < 8; j0 += PAIR) {
        // A short last Q8_0/Q4_0 group skips its missing blocks (their
        // operands are still reloaded for the next group).
        if ((T == Q8_0 || T == Q4_0) && !FULL && j0 >= nb) {
            load_acts<T, NP, G>(acts, L, gn, g0c, j0, PAIR, dig, n);
            continue;
        }
        i32x16 D[PAIR][kTokenHalves<T, NP>];
        float sc[PAIR], mn[PAIR];   // per-block multipliers of q.x and of sum x
        int xg[PAIR];
#pragma unroll
        for (int jj = 0; jj < PAIR; ++jj) {
            const int j = j0 + jj;
            int xgl;
            const i32x4 b = block_operand<T, FULL>(w, j, h, sc[jj], mn[jj], xgl);
            xg[jj] = 8 * (g - g0c) + xgl;
#pragma unroll
            for (int th = 0; th < kTokenHalves<T, NP>; ++th) {
                i32x4 a;
                if constexpr (G) a = acts[8 * th + j];
                else a = *(const i32x4 *)(dig + a_offset<T, NP>(L, g - g0c, j, th, n, nb));
                D[jj][th] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, (i32x16){}, 0, 0, 0);
            }
        }
        load_acts<T, NP, G>(acts, L, gn, g0c, j0, PAIR, dig, n);
#pragma unroll
        for (int jj = 0; jj < PAIR; ++jj) {
            // A short last Q8_0/Q4_0 group drops its padding block.
            if ((T == Q8_0 || T == Q4_0) && j0 + jj >= nb) break;
#pragma unroll
            for (int th = 0; th < kTokenHalves<T, NP>; ++th)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int t = T == Q6_K ? k + 4 * th : 2 * k + h;
                    const int slot = T == Q6_K ? k + 4 * th : k;   // accumulator
                    if (slot >= NA) continue;
                    const float Gs = recombine<T>(D[jj][th][4 * k], D[jj][th][4 * k + 1], D[jj][th][4 * k + 2]);
                    const float2 mt = meta[xg[jj] * NP + (t < NP ? t : 0)];
                    if constexpr (T == Q8_0 || T == Q4_0) {
                        acc[slot] += mt.x * (sc[jj] * Gs);
                    } else {
                        sum_s[slot] += sc[jj] * (Gs * mt.x);
                        if constexpr (T == Q4_K) sum_m[slot] += mn[jj] * mt.y;
                    }
                }
        }
        // Bounds the live result registers to one pair.
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (T == Q4_K || T == Q6_K) {
        float d, dmin;
        group_scales<T>(w, d, dmin);
#pragma unroll
        for (int k = 0; k < NA; ++k) acc[k] += T == Q4_K ? d * sum_s[k] - dmin * sum_m[k] : d * sum_s[k];
    }
}

// One workgroup per 32-row tile; groups [g0c, g0c + ngc) of every row (one
// column chunk). N = 1 (G false): x is this chunk's columns of the single
// token; otherwise dig/meta hold the chunk's digits for np = NP slots.
template <unsigned T, int NP, int KS, bool G>
__global__ __launch_bounds__(64 * KS) __attribute__((amdgpu_waves_per_eu(2))) void smalln_mfma(const uint8_t *__restrict__ w, const float *__restrict__ x,
    const uint8_t *__restrict__ gdig, const float2 *__restrict__ gmeta, float *__restrict__ y, int rows, int cols,
    int g0c, int ngc, int n, int accumulate)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[KS][(kAcc<T, NP>)][64];
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
    // This wave's groups: g0c + wave + KS k for k < ns (the workgroup's
    // wavefronts read adjacent groups at the same time). Past the last one a
    // stage repeats it.
    const int ns = wave < ngc ? (ngc - wave + KS - 1) / KS : 0;
    auto group_of = [&](int k) { return g0c + (ns > 0 ? wave + KS * (k < ns ? k : ns - 1) : 0); };
    // N = 1: item idx (8 values) of this wave's columns of x, as a chunk
    // item, or -1 past the end (whole 4-lane groups agree).
    auto item_of = [&](int idx) {
        const int k = idx >> 5, it = 32 * (wave + KS * k) + (idx & 31);
        return k < ns && it < 4 * xgroups ? it : -1;
    };

    // 1. Activations first.
    constexpr int kPre = 2;   // x items (8 values) per lane issued ahead (N = 1)
    float4 px[kPre][2];
    float2 pm[2];
    if constexpr (!G) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int it = item_of(lane + 64 * k);
            const float4 *src = (const float4 *)x + 2 * (it >= 0 ? it : 0);
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
    // 2. The first group's activation operands (N >= 2), then the first RING
    //    weight stages.
    constexpr int RING = kRing<T, NP>;
    i32x4 acts[kActs<T, NP, G>];
    load_acts<T, NP, G>(acts, L, group_of(0), g0c, 0, 8, gdig, n);
    WStage<T> st[RING];
#pragma unroll
    for (int k = 0; k < RING; ++k) load_weights<T, kStreamWeights<T, G>>(st[k], L, group_of(k));
    // 3. Activations into LDS (waits for them only).
    if constexpr (!G) {
#pragma unroll
        for (int k = 0; k < kPre; ++k)
            asm volatile("" : "+v"(px[k][0].x), "+v"(px[k][0].y), "+v"(px[k][0].z), "+v"(px[k][0].w),
                         "+v"(px[k][1].x), "+v"(px[k][1].y), "+v"(px[k][1].z), "+v"(px[k][1].w) :: "memory");
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int it = item_of(lane + 64 * k);
            if (it >= 0) quantize8(px[k][0], px[k][1], 1, 0, it, sdig, smeta);
        }
        for (int k = 64 * kPre; k < 32 * ns; k += 64) {
            const int it = item_of(lane + k);
            if (it >= 0) {
                const float4 *src = (const float4 *)x + 2 * it;
                quantize8(src[0], src[1], 1, 0, it, sdig, smeta);
            }
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

    // 4. The ring, branch-free: past the wave's last group a stage repeats
    //    that group and its sums are dropped.
    constexpr int NA = kAcc<T, NP>;
    float acc[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) acc[k] = 0.f;
    for (int i = 0; i < ns; i += RING) {
#pragma unroll
        for (int k = 0; k < RING; ++k) {
            float part[NA];
#pragma unroll
            for (int q = 0; q < NA; ++q) part[q] = 0.f;
            // A short last Q8_0/Q4_0 group has its own layout (formats.h).
            const int gk = group_of(i + k), gn = group_of(i + k + 1);
            if ((T == Q8_0 || T == Q4_0) && group_blocks(L, gk) < 8)
                compute_stage<T, NP, G, false>(part, st[k], acts, L, gk, gn, g0c, dig, smeta, n);
            else
                compute_stage<T, NP, G, true>(part, st[k], acts, L, gk, gn, g0c, dig, smeta, n);
            load_weights<T, kStreamWeights<T, G>>(st[k], L, group_of(i + k + RING));
            const float keep = i + k < ns ? 1.f : 0.f;
#pragma unroll
            for (int q = 0; q < NA; ++q) acc[q] += keep * part[q];
        }
    }

    // 5. Partial sums of the KS waves, added in wave order.
#pragma unroll
    for (int k = 0; k < NA; ++k) red[wave][k][lane] = acc[k];
    __syncthreads();
    if (wave != 0) return;
    float v[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) {
        v[k] = red[0][k][lane];
        for (int q = 1; q < KS; ++q) v[k] += red[q][k][lane];
    }
    const int row = kTileRows * t + (lane & 31);
    const bool own = (lane & 31) < R;
    if constexpr (T == Q6_K) {
        // The two lane halves hold the two scale groups of each 32 columns.
#pragma unroll
        for (int k = 0; k < NA; ++k) v[k] += __shfl_xor(v[k], 32, 64);
#pragma unroll
        for (int k = 0; k < NP; ++k)
            if (own && k < n && (k & 1) == L.h) {
                float *dst = y + (size_t)k * rows + row;
                *dst = accumulate ? *dst + v[k] : v[k];
            }
    } else {
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            const int tok = 2 * k + L.h;
            if (own && tok < n) {
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

hipError_t launch_quantize_x(const float *x, int ldx, int cols, int batch, int np, uint8_t *dig, float2 *meta,
    hipStream_t s)
{
    const int total = batch * (cols / 8);
    hipLaunchKernelGGL(quantize_x, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, ldx, cols, batch, np,
        dig, meta);
    return hipGetLastError();
}

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
            const hipError_t e = launch_quantize_x(x + c0, cols, ccols, batch, np, dig, meta, s);
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
