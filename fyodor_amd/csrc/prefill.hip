// Prefill GEMM Y[m][row] = sum_k W[row][k] * X[m][k] for batches above 8, on
// gfx950 int8 MFMA with the exact block dot products of blockdot.h: the same
// activation digits and integer block sums as the small-N path, so outputs
// differ from it only by the order of the fp32 sum over blocks.
//
// Work split. A workgroup of four wavefronts owns 128 weight rows (wavefront
// w: the 32-row tile 4 * blockIdx.x + w) and 32 tokens (four MFMA token
// blocks of 8; Q6_K, whose blocks take two MFMAs each, 16). K advances one
// 256-column group per step. The group's activation digits for those tokens
// (8 blocks x 128 B per token) and their scales are staged in LDS,
// double-buffered (68 KiB per workgroup, Q6_K 36 KiB; one barrier per step):
// after the MFMAs of group g each thread stores group g+1's digits (fetched
// one step earlier) into the other buffer and fetches g+2. The weights of
// each wavefront's tile stream through the same two-stage register ring as
// the small-N kernel and feed one MFMA per token block (Q6_K two) per
// 32-column block.
#include "blockdot.h"
#include "kernels.h"

namespace fy {
namespace {

constexpr int kRowTiles = 4;   // 32-row tiles per workgroup (one per wavefront)

// Tokens per workgroup: 32 (four MFMA token blocks of 8); Q6_K, whose blocks
// take two MFMAs and eight accumulators per lane, 16.
template <unsigned T> constexpr int kTokens = T == Q6_K ? 16 : 32;
template <unsigned T> constexpr int kTokenBlocks = kTokens<T> / 8;
template <unsigned T> constexpr int kBlockDigits = kTokens<T> * 4 * kSlotBytes;   // one 32-column block
template <unsigned T> constexpr int kGroupDigits = 8 * kBlockDigits<T>;
template <unsigned T> constexpr int kGroupMeta = 8 * kTokens<T>;                   // float2 per group
template <unsigned T> constexpr int kDigitLoads = kGroupDigits<T> / (16 * 256);     // 16-byte loads per thread

template <unsigned T> constexpr int kHalves = T == Q6_K ? 2 : 1;   // MFMAs per token block
template <unsigned T> constexpr int kLaneTokens = T == Q6_K ? 8 : 4; // accumulators per token block

// Every thread stores one scale pair per group (branch-free); entries past
// kGroupMeta are duplicates nobody reads.
template <unsigned T>
struct Staging {
    uint8_t dig[2][kGroupDigits<T>];
    float2 meta[2][kGroupMeta<T> > 256 ? kGroupMeta<T> : 256];
};

// This thread's share of group g's digits and scales.
template <unsigned T>
struct AFetch {
    u32x4 d[kDigitLoads<T>];
    float2 m;
};

template <unsigned T>
__device__ __forceinline__ void fetch_group(AFetch<T> &f, const uint8_t *__restrict__ dig,
    const float2 *__restrict__ meta, size_t np, int m0, int groups_x, int g)
{
    const int tid = threadIdx.x;
    // Load k covers block k * 8 / kDigitLoads + (tid * 16) / kBlockDigits.
    constexpr int per = kBlockDigits<T> / (16 * 256) > 0 ? kBlockDigits<T> / (16 * 256) : 1;   // loads per block
    constexpr int blocks_per_load = (16 * 256) / kBlockDigits<T> > 0 ? (16 * 256) / kBlockDigits<T> : 1;
#pragma unroll
    for (int k = 0; k < kDigitLoads<T>; ++k) {
        const int j = blocks_per_load == 1 ? k / per : k * blocks_per_load + (16 * tid) / kBlockDigits<T>;
        const int in = blocks_per_load == 1 ? 16 * tid + (k % per) * 16 * 256 : (16 * tid) % kBlockDigits<T>;
        const int xg = 8 * g + j < groups_x ? 8 * g + j : groups_x - 1;
        f.d[k] = *(const u32x4 *)(dig + (size_t)xg * 4 * kSlotBytes * np + (size_t)m0 * 4 * kSlotBytes + in);
    }
    const int e = tid % kGroupMeta<T>;
    const int xg = 8 * g + e / kTokens<T> < groups_x ? 8 * g + e / kTokens<T> : groups_x - 1;
    f.m = meta[(size_t)xg * np + m0 + e % kTokens<T>];
}

template <unsigned T>
__device__ __forceinline__ void store_group(Staging<T> &s, int buf, const AFetch<T> &f)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < kDigitLoads<T>; ++k) *(u32x4 *)(s.dig[buf] + 16 * (tid + 256 * k)) = f.d[k];
    s.meta[buf][tid] = f.m;
}

// LDS offset of the A operand of block j, token block tb, token half th for
// this lane (chunk-local: x group xgl of the group), or of token 0's zero
// slot when the lane's A-row is not live for the n tokens left.
template <unsigned T>
__device__ __forceinline__ int a_lds(const Lane &L, int xgl, int j, int tb, int th, int n)
{
    if constexpr (T == Q6_K) {
        const int p = j >> 1;
        const int t = (L.slot >> 3) + 4 * th, c = (L.slot >> 2) & 1, d = L.slot & 3;
        const bool live = c == L.h && d < 3 && 8 * tb + t < n;
        return kBlockDigits<T> * xgl + (live ? 128 * (8 * tb + t) + kSlotBytes * d : kSlotBytes * 3) + 16 * (p & 1);
    } else {
        const bool live = 8 * tb + (L.slot >> 2) < n;
        return kBlockDigits<T> * xgl + (live ? 1024 * tb + kSlotBytes * L.slot : kSlotBytes * 3) + 16 * L.h;
    }
}

template <unsigned T>
__global__ __launch_bounds__(256) void prefill_mfma(const uint8_t *__restrict__ w, const uint8_t *__restrict__ dig,
    const float2 *__restrict__ meta, float *__restrict__ y, int rows, int cols, int batch, int np)
{
    __shared__ __align__(16) Staging<T> S;
    constexpr int TOK = kTokens<T>, TBN = kTokenBlocks<T>;
    constexpr int NL = kLaneTokens<T>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const int tile_raw = kRowTiles * blockIdx.x + wave;
    const int tile = tile_raw < tiles ? tile_raw : tiles - 1;
    const int m0 = TOK * blockIdx.y, n = batch - m0;   // tokens left (> 0)
    const int R = rows - kTileRows * tile < kTileRows ? rows - kTileRows * tile : kTileRows;
    Lane L;
    L.tile = w + (size_t)kTileRows * tile * tiled_row_bytes<T>(cols);
    L.R = R;
    L.r = (lane & 31) < R ? (lane & 31) : R - 1;
    L.h = lane >> 5;
    L.slot = lane & 31;
    L.groups = (cols + kGroupCols - 1) / kGroupCols;
    L.blocks = cols / 32;
    const int groups = L.groups, groups_x = cols / 32;
    auto clampg = [&](int g) { return g < groups ? g : groups - 1; };

    // Prologue: group 0's activations into LDS, weights of groups 0 and 1 and
    // activations of group 1 in flight.
    AFetch<T> af;
    fetch_group(af, dig, meta, (size_t)np, m0, groups_x, 0);
    WStage<T> st[2];
    load_weights<T>(st[0], L, 0);
    store_group(S, 0, af);
    fetch_group(af, dig, meta, (size_t)np, m0, groups_x, clampg(1));
    load_weights<T>(st[1], L, clampg(1));
    __syncthreads();

    float acc[TBN][NL];
#pragma unroll
    for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
        for (int k = 0; k < NL; ++k) acc[tb][k] = 0.f;

    for (int g = 0; g < groups; ++g) {
        const uint8_t *sd = S.dig[g & 1];
        const float2 *sm = S.meta[g & 1];
        const int nb = (T == Q8_0 || T == Q4_0) ? group_blocks(L, g) : 8;
        float sum_s[TBN][NL], sum_m[TBN][NL];
#pragma unroll
        for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
            for (int k = 0; k < NL; ++k) sum_s[tb][k] = sum_m[tb][k] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if ((T == Q8_0 || T == Q4_0) && j >= nb) break;
            float sc, mn;
            int xgl;
            const i32x4 b = block_operand<T>(st[0], j, L.h, sc, mn, xgl);
            // Two MFMAs issue before their epilogues read them: two token
            // blocks, or one Q6_K token block's two halves.
            constexpr int TBS = kHalves<T> == 1 ? 2 : 1;
#pragma unroll
            for (int tb0 = 0; tb0 < TBN; tb0 += TBS) {
                i32x16 D[TBS][kHalves<T>];
#pragma unroll
                for (int q = 0; q < TBS; ++q)
#pragma unroll
                    for (int th = 0; th < kHalves<T>; ++th) {
                        const i32x4 a = *(const i32x4 *)(sd + a_lds<T>(L, xgl, j, tb0 + q, th, n));
                        D[q][th] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, (i32x16){}, 0, 0, 0);
                    }
#pragma unroll
                for (int q = 0; q < TBS; ++q)
#pragma unroll
                    for (int th = 0; th < kHalves<T>; ++th)
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int tb = tb0 + q;
                            const int t = T == Q6_K ? k + 4 * th : 2 * k + L.h;   // token within the block
                            const int slot = T == Q6_K ? k + 4 * th : k;
                            const float Gs = recombine<T>(D[q][th][4 * k], D[q][th][4 * k + 1], D[q][th][4 * k + 2]);
                            const float2 mt = sm[TOK * xgl + 8 * tb + t];
                            if constexpr (T == Q8_0 || T == Q4_0) {
                                sum_s[tb][slot] += mt.x * (sc * Gs);
                            } else {
                                sum_s[tb][slot] += sc * (Gs * mt.x);
                                if constexpr (T == Q4_K) sum_m[tb][slot] += mn * mt.y;
                            }
                        }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        float d, dmin;
        group_scales<T>(st[0], d, dmin);
#pragma unroll
        for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
            for (int k = 0; k < NL; ++k)
                acc[tb][k] += T == Q4_K ? d * sum_s[tb][k] - dmin * sum_m[tb][k]
                            : T == Q6_K ? d * sum_s[tb][k] : sum_s[tb][k];
        // Group g + 1's activations into the other buffer (its readers passed
        // the last barrier), fetch group g + 2, and rotate the weight ring.
        store_group(S, (g + 1) & 1, af);
        fetch_group(af, dig, meta, (size_t)np, m0, groups_x, clampg(g + 2));
        st[0] = st[1];
        load_weights<T>(st[1], L, clampg(g + 2));
        __syncthreads();
    }

    // Q6_K: the two lane halves hold the two scale groups of every 32
    // columns (all lanes take part in the exchange).
    if constexpr (T == Q6_K) {
#pragma unroll
        for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
            for (int k = 0; k < NL; ++k) acc[tb][k] += __shfl_xor(acc[tb][k], 32, 64);
    }
    if (tile_raw >= tiles || (lane & 31) >= R) return;
    const int row = kTileRows * tile + (lane & 31);
#pragma unroll
    for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            const int t = T == Q6_K ? 8 * tb + k : 8 * tb + 2 * k + L.h;
            const bool mine = T == Q6_K ? (k & 1) == L.h : true;
            if (mine && t < n) y[(size_t)(m0 + t) * rows + row] = acc[tb][k];
        }
}

}  // namespace

size_t prefill_workspace(int cols, int batch)
{
    const size_t np = ((size_t)batch + 31) / 32 * 32;   // a multiple of every kTokens
    return (size_t)(cols / 32) * (4 * kSlotBytes + 8) * np;
}

hipError_t launch_prefill(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, int batch,
    void *workspace, hipStream_t s)
{
    const int np = (batch + 31) / 32 * 32;
    uint8_t *dig = (uint8_t *)workspace;
    float2 *meta = (float2 *)(dig + (size_t)(cols / 32) * 4 * kSlotBytes * np);
    hipError_t e = launch_quantize_x(x, cols, cols, batch, np, dig, meta, s);
    if (e != hipSuccess) return e;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const unsigned gx = (unsigned)((tiles + kRowTiles - 1) / kRowTiles);
    // Token blocks that hold at least one token.
    auto gy = [&](int tok) { return (unsigned)((batch + tok - 1) / tok); };
    switch (type) {
    case Q4_K: hipLaunchKernelGGL(prefill_mfma<Q4_K>, dim3(gx, gy(32)), dim3(256), 0, s, w, dig, meta, y, rows, cols, batch, np); break;
    case Q6_K: hipLaunchKernelGGL(prefill_mfma<Q6_K>, dim3(gx, gy(16)), dim3(256), 0, s, w, dig, meta, y, rows, cols, batch, np); break;
    case Q8_0: hipLaunchKernelGGL(prefill_mfma<Q8_0>, dim3(gx, gy(32)), dim3(256), 0, s, w, dig, meta, y, rows, cols, batch, np); break;
    case Q4_0: hipLaunchKernelGGL(prefill_mfma<Q4_0>, dim3(gx, gy(32)), dim3(256), 0, s, w, dig, meta, y, rows, cols, batch, np); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fy
