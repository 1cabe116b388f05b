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

typedef float f32x16 __attribute__((ext_vector_type(16)));

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

// LDS staging of one group, double-buffered. Every thread stores one digit
// chunk per load and one scale pair (branch-free; for Q6_K the entries past
// kGroupMeta are duplicates nobody reads).
//
// 32-token types: token block tb, digit slot s (= 4 * token + digit within
// the block) and column half h of block j sit at
// 4096 j + 1024 tb + 512 h + 16 (s ^ 8 h): the sixteen lanes that one LDS
// cycle serves read 256 contiguous bytes, and the staging stores (h
// alternating with the thread index) land on both halves of the banks.
// Activation scales are stored token-permuted, mx[32 j + i] for token tau(i),
// tau(i) = 8 (i / 8) + 2 (i % 4) + (i / 4) % 2: lane half h reads its four
// tokens 8 tb + 2 k + h (k = 0..3) as one 16-byte load at 32 j + 8 tb + 4 h.
// Q4_K also stores the block sums of x as the A operand of the min-term MFMA:
// my[4 l + s] = sum x of block 2 s + l / 32 for token tau(l % 32).
// Q6_K keeps tokens in order: mx[kTokens * j + t].
template <unsigned T>
struct Staging {
    uint8_t dig[2][kGroupDigits<T>];
    float mx[2][256];
    float my[T == Q4_K ? 2 : 1][T == Q4_K ? 256 : 1];
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

// Position of token t (0..31) in the permuted scale order (used by the
// 32-token formats; only Q6_K is launched on this kernel now).
[[maybe_unused]] __device__ __forceinline__ int tau_inv(int t) { return 8 * (t >> 3) + 4 * (t & 1) + ((t >> 1) & 3); }

template <unsigned T>
__device__ __forceinline__ void store_group(Staging<T> &s, int buf, const AFetch<T> &f)
{
    const int tid = threadIdx.x;
    if constexpr (T == Q6_K) {
#pragma unroll
        for (int k = 0; k < kDigitLoads<T>; ++k) *(u32x4 *)(s.dig[buf] + 16 * (tid + 256 * k)) = f.d[k];
        s.mx[buf][tid] = f.m.x;
    } else {
        // Chunk tid of block k: slot tid / 2 (token block tid / 64), half tid % 2.
        const int slot = (tid >> 1) & 31, h = tid & 1;
        const int at = 1024 * (tid >> 6) + 512 * h + 16 * (slot ^ (8 * h));
#pragma unroll
        for (int k = 0; k < kDigitLoads<T>; ++k) *(u32x4 *)(s.dig[buf] + kBlockDigits<T> * k + at) = f.d[k];
        const int j = tid >> 5, i = tau_inv(tid & 31);
        s.mx[buf][32 * j + i] = f.m.x;
        if constexpr (T == Q4_K) s.my[buf][4 * (32 * (j & 1) + i) + (j >> 1)] = f.m.y;
    }
}

// LDS offset of the A operand of block j, token block tb, token half th for
// this lane (chunk-local: x group xgl of the group), or of a zero slot when
// the lane's A-row is not live for the n tokens left.
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
        const int slot = live ? L.slot : 3;   // token 0's zero slot
        return kBlockDigits<T> * xgl + (live ? 1024 * tb : 0) + 512 * L.h + 16 * (slot ^ (8 * L.h));
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
        const float *smx = S.mx[g & 1];
        const int nb = (T == Q8_0 || T == Q4_0) ? group_blocks(L, g) : 8;
        float sum_s[TBN][NL];
#pragma unroll
        for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
            for (int k = 0; k < NL; ++k) sum_s[tb][k] = 0.f;
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
                for (int q = 0; q < TBS; ++q) {
                    const int tb = tb0 + q;
                    if constexpr (T == Q6_K) {
#pragma unroll
                        for (int th = 0; th < kHalves<T>; ++th)
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const float Gs = recombine<T>(D[q][th][4 * k], D[q][th][4 * k + 1], D[q][th][4 * k + 2]);
                                sum_s[tb][k + 4 * th] += sc * (Gs * smx[TOK * xgl + 8 * tb + k + 4 * th]);
                            }
                    } else {
                        // Scales of tokens 8 tb + 2 k + h, k = 0..3.
                        const float4 mx = *(const float4 *)(smx + 32 * xgl + 8 * tb + 4 * L.h);
                        const float m4[4] = {mx.x, mx.y, mx.z, mx.w};
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float Gs = recombine<T>(D[q][0][4 * k], D[q][0][4 * k + 1], D[q][0][4 * k + 2]);
                            if constexpr (T == Q4_K) sum_s[tb][k] += sc * (Gs * m4[k]);
                            else sum_s[tb][k] += m4[k] * (sc * Gs);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            (void)mn;
        }
        float d, dmin;
        group_scales<T>(st[0], d, dmin);
        if constexpr (T == Q4_K) {
            // Min term sum_j m_j * (sum x over block j) for the 32 rows x 32
            // tokens: A = block sums (lane l: blocks 2s + l / 32 of token
            // tau(l % 32)), B = the rows' 6-bit minimums; D row i is token
            // tau(i), the token of acc[i / 8][i % 4] in lane half (i / 4) % 2.
            const float4 ys = *(const float4 *)(S.my[g & 1] + 4 * lane);
            const float ya[4] = {ys.x, ys.y, ys.z, ys.w};
            f32x16 M = {};
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                const float m = (float)((st[0].sl[s2] >> (12 * L.h + 6)) & 63u);
                M = __builtin_amdgcn_mfma_f32_32x32x2f32(ya[s2], m, M, 0, 0, 0);
            }
#pragma unroll
            for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
                for (int k = 0; k < NL; ++k) acc[tb][k] += d * sum_s[tb][k] - dmin * M[4 * tb + k];
        } else {
#pragma unroll
            for (int tb = 0; tb < TBN; ++tb)
#pragma unroll
                for (int k = 0; k < NL; ++k) acc[tb][k] += T == Q6_K ? d * sum_s[tb][k] : sum_s[tb][k];
        }
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

size_t prefill_workspace(unsigned type, int cols, int batch)
{
    if (prefill_f16_supported(type)) return prefill_f16_workspace(cols, batch);
    const size_t np = ((size_t)batch + 31) / 32 * 32;   // a multiple of every kTokens
    return (size_t)(cols / 32) * (4 * kSlotBytes + 8) * np;
}

const char *prefill_kernel(unsigned type) { return prefill_f16_supported(type) ? "prefill_f16" : "prefill_mfma"; }

hipError_t launch_prefill(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, int batch,
    void *workspace, hipStream_t s)
{
    if (prefill_f16_supported(type)) return launch_prefill_f16(type, w, x, y, rows, cols, batch, workspace, s);
    const int np = (batch + 31) / 32 * 32;
    uint8_t *dig = (uint8_t *)workspace;
    float2 *meta = (float2 *)(dig + (size_t)(cols / 32) * 4 * kSlotBytes * np);
    hipError_t e = launch_quantize_x(x, cols, cols, batch, np, dig, meta, s);
    if (e != hipSuccess) return e;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const unsigned gx = (unsigned)((tiles + kRowTiles - 1) / kRowTiles);
    // Token blocks that hold at least one token.
    auto gy = [&](int tok) { return (unsigned)((batch + tok - 1) / tok); };
    if (type != Q6_K) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prefill_mfma<Q6_K>, dim3(gx, gy(16)), dim3(256), 0, s, w, dig, meta, y, rows, cols, batch, np);
    return hipGetLastError();
}

}  // namespace fy
