// Prefill GEMM Y[m][row] = sum_k W[row][k] * X[m][k] for batches above 8 on
// gfx950 fp16 MFMA (v_mfma_f32_32x32x16_f16), Q4_K / Q8_0 / Q4_0 weights.
//
// Numbers. The weights enter the MFMA as exact fp16 integers: Q4_K sc * q
// (<= 63 * 15 = 945), Q8_0 q, Q4_0 q - 8. Each token's activations are scaled
// by one power of two s = 2^(14 - E) (2^(E-1) <= max |x| < 2^E over the
// token) and split into two fp16 pieces, x s = hi + lo + e with hi = fp16(x s)
// and lo = fp16(x s - hi): |e| <= 2^-22 |x s|, or 2^-25 absolute where lo is
// subnormal. The MFMA multiplies fp16 pairs exactly and accumulates in fp32,
// so a block dot is sum (sc q)(hi + lo) with fp32 accumulation error only.
// What remains for the VALU is the superblock scales d and dmin per 256
// columns (Q4_K; the 6-bit minimums meet the per-block sums of x s on one
// more fp16 MFMA, the sums split into two pieces like x) or the fp16 block
// scale per 32 columns (Q8_0, Q4_0), and 1/s once per output. A token holding a non-finite value gets NaN pieces: its outputs are
// NaN.
//
// Column order. A lane of the weight tile holds 16 consecutive columns of a
// block (tiled layout, formats.h); the cheapest fp16 conversion of its bytes
// yields columns in the order c0 c2 c1 c3 per 4 bytes. The MFMA sums over its
// 16 K slots in any order, so the activation pieces are stored in the same
// order: within every 8 columns, position s holds column pi(s),
// pi = 0 2 1 3 4 6 5 7.
//
// Work split. A workgroup of eight wavefronts (four for Q8_0/Q4_0 and for
// grids too small to fill the chip twice) owns 256 weight rows (one 32-row
// tile per wavefront) and 32 tokens (the A rows of the MFMA); the token block
// varies fastest over the grid, so workgroups that share a row group run
// side by side on one XCD and its L2. K advances one 256-column group per
// step. Both pieces of the 32 tokens (32 KiB) go straight from global memory
// into LDS (global_load_lds, no staging registers), double-buffered: step g
// issues group g + 1's copies and weights, computes group g, waits for its
// own copies and meets the others at one barrier. LDS rows are paired: the
// 1 KiB copy of tokens 2q and 2q + 1 interleaves them per 16 bytes at a
// 1056-byte pair pitch, so the sixteen lanes of one LDS cycle (tokens r..r+15,
// same columns) hit distinct banks with immediate offsets only.
#include <type_traits>

#include "blockdot.h"
#include "kernels.h"

namespace fy {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kTokens = 32;       // tokens per token tile = MFMA A rows
constexpr int kPairPitch = 1056;  // LDS bytes per token pair of one piece (1 KiB + 32)
constexpr int kPieceBytes = kTokens / 2 * kPairPitch;
constexpr int kSumBytes = 1024;   // Q4_K block sums of one group: 32 tokens x 2 halves x 16 bytes
constexpr int kTileBytes = 2 * kPieceBytes + kSumBytes;   // one token tile of one group
// One LDS buffer holds a group for the workgroup's TW token tiles.
template <int TW> constexpr int kBufBytes = TW * kTileBytes;

// ---- activation pieces ---------------------------------------------------
// Workspace for np tokens (np a multiple of 32): hi[np][cols], lo[np][cols]
// (fp16, permuted as above), bsum[np][cols / 256][2][8] (the sum of x s over
// 32-column block j of each 256-column group, times 2^-5, as two fp16
// pieces: [0][j] hi, [1][j] lo; |sum| < 2^19, so the scaled sum is below the
// fp16 range limit; written when cols % 256 == 0) and inv[np] (1 / s, or
// NaN).
struct Pieces {
    _Float16 *hi, *lo, *bsum;
    float *inv;
};

__host__ __device__ inline Pieces pieces_of(void *ws, int cols, int np)
{
    Pieces p;
    p.hi = (_Float16 *)ws;
    p.lo = p.hi + (size_t)np * cols;
    p.bsum = p.lo + (size_t)np * cols;
    p.inv = (float *)(p.bsum + (size_t)np * (cols / 16));
    return p;
}

__device__ __forceinline__ float block_max(float v, float *red)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

// One workgroup per token; cols % 32 == 0.
__global__ __launch_bounds__(256) void split_x(const float *__restrict__ x, int cols, Pieces out)
{
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float *row = x + (size_t)t * cols;
    const int chunks = cols / 8;
    float m = 0.f, z = 0.f;
    for (int c = threadIdx.x; c < chunks; c += 256) {
        const float4 a = *(const float4 *)(row + 8 * c), b = *(const float4 *)(row + 8 * c + 4);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        m = fmaxf(m, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        // NaN iff some value is inf or NaN.
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) z = __builtin_fmaf(v[i], 0.f, z);
    }
    m = block_max(m, red);
    z = block_max(z != z ? 1.f : 0.f, red);
    const bool finite = z == 0.f;
    int e = 0;
    (void)__builtin_frexpf(m, &e);
    const int shift = m > 0.f ? 14 - e : 0;
    if (threadIdx.x == 0)
        out.inv[t] = finite ? __builtin_ldexpf(1.f, -shift) : __builtin_nanf("");
    for (int c = threadIdx.x; c < chunks; c += 256) {
        const float4 a = *(const float4 *)(row + 8 * c), b = *(const float4 *)(row + 8 * c + 4);
        float v[8] = {a.x, a.z, a.y, a.w, b.x, b.z, b.y, b.w};   // columns in pi order
        float s = 0.f;
        h8 hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] = finite ? __builtin_ldexpf(v[i], shift) : __builtin_nanf("");
            s += v[i];
            hi[i] = (_Float16)v[i];
            lo[i] = (_Float16)(v[i] - (float)hi[i]);
        }
        *(h8 *)(out.hi + (size_t)t * cols + 8 * c) = hi;
        *(h8 *)(out.lo + (size_t)t * cols + 8 * c) = lo;
        // Four consecutive chunks form a 32-column block (256 is a multiple of 4).
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((c & 3) == 0 && cols % 256 == 0) {
            const int b = c / 4, j = b & 7;
            const float sv = s * 0.03125f;
            const _Float16 shi = (_Float16)sv;
            _Float16 *dst = out.bsum + (size_t)t * (cols / 16) + 2 * (b & ~7) + j;
            dst[0] = shi;
            dst[8] = (_Float16)(sv - (float)shi);
        }
    }
}

// ---- GEMM ---------------------------------------------------------------
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Workgroup barrier without the memory-model fences of __syncthreads (whose
// release side waits for every outstanding vector load): the kernel orders
// its LDS traffic itself (explicit s_waitcnt before each barrier); the empty
// asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier()
{
    asm volatile("" : : : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" : : : "memory");
}

// 16 bytes per lane from a buffer straight into LDS: lane l's bytes (at
// voff + soff in the buffer) land at dst + 16 l (dst uniform over the
// wavefront). Buffer loads take a per-lane 32-bit offset fixed for the kernel
// and a scalar one: no vector address arithmetic per copy (global_load_lds
// needed four to five VALU instructions of 64-bit address math each).
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, int voff, int soff, lds_u8 *dst)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)dst, 16, voff, soff, 0, 0);
}

// Buffer resource over `bytes` bytes at p (out-of-range reads return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// Copies of group g into LDS buffer `buf` issued by this wavefront (one of
// RT), for each of the TW token tiles (tile tt at buf + kTileBytes tt):
// token pairs 16 TW / RT per wavefront of both pieces (lane l: token
// 2q + (l & 1), 16-byte chunk l >> 1 of the group's row, to byte 16 l of the
// pair), and for Q4_K tile (wavefront % TW)'s block sums (lane l: token
// l % 32, half l / 32). Each copy reads through a resource over its own two
// token rows (rebased in scalar registers, so every offset stays far below
// 2^31 at the widest rows the library accepts); past a short last Q8_0/Q4_0
// group a lane reads the next row's columns or zeros, into LDS slots of
// blocks that are skipped.
template <int RT, int TW>
__device__ __forceinline__ void copy_group(lds_u8 *__restrict__ buf, const Pieces &p, int cols, int m0, int g, bool sums)
{
    constexpr int kPairs = 16 * TW / RT;   // token pairs per wavefront, over all token tiles
    static_assert(kPairs >= 1 && 16 * TW % RT == 0, "whole token pairs per wavefront");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int vpair = 2 * ((lane & 1) * cols + 8 * (lane >> 1));   // bytes within the pair's two rows
#pragma unroll
    for (int piece = 0; piece < 2; ++piece)
#pragma unroll
        for (int k = 0; k < kPairs; ++k) {
            const int q = kPairs * wave + k, tt = q / 16, qq = q % 16;   // pair qq of token tile tt
            const _Float16 *rows2 = (piece ? p.lo : p.hi) + (size_t)(m0 + 32 * tt + 2 * qq) * cols;
            lds_copy16(rsrc_of(rows2, 4u * (uint32_t)cols), vpair, 512 * g,
                       buf + kTileBytes * tt + piece * kPieceBytes + qq * kPairPitch);
        }
    if (sums) {
        // Every wavefront copies (wavefronts past TW the same bytes to the
        // same place again): a copy under a wavefront condition leaves a
        // branch after which the compiler waits for every load.
        const int tt = wave % TW, gs = cols / 256;
        const _Float16 *first = p.bsum + ((size_t)(m0 + 32 * tt) * gs + g) * 16;   // token 0 of the tile
        lds_copy16(rsrc_of(first, 1024u * (uint32_t)gs), 2 * (16 * gs * (lane & 31) + 8 * (lane >> 5)), 0,
                   buf + kTileBytes * tt + 2 * kPieceBytes);
    }
}

__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// fp16 pairs 1024 + (byte 0, byte 2) and 1024 + (byte 1, byte 3) of v (bytes
// below 2^10 - 1024 = 0x3ff: the byte becomes the low mantissa bits under
// the exponent byte 0x64).
__device__ __forceinline__ h2 pair02(uint32_t v) { return as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04020400u)); }
__device__ __forceinline__ h2 pair13(uint32_t v) { return as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04030401u)); }

// B operand of block j, K slice kappa (columns 16h + 8 kappa .. of the block,
// in pi order) for this lane. Q4_K folds the 6-bit sub-block scale in:
// (1024 + q) sc - 1024 sc = q sc exactly (one fused rounding of an integer
// below 2^11), with sc2 = (sc, sc) and nsc2 = (-1024 sc, -1024 sc).
template <unsigned T, bool FULL = true>
__device__ __forceinline__ h8 b_operand(const WStage<T> &w, int j, int kappa, int h, h2 sc2, h2 nsc2)
{
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (T == Q4_K) {
            const uint32_t word = w.q[j >> 1][2 * kappa + i];
            const uint32_t nib = ((j & 1) ? word >> 4 : word) & 0x0F0F0F0Fu;
            v[2 * i] = as_u32(__builtin_elementwise_fma(pair02(nib), sc2, nsc2));
            v[2 * i + 1] = as_u32(__builtin_elementwise_fma(pair13(nib), sc2, nsc2));
        } else if constexpr (T == Q4_0) {
            // Full group: nibble j & 1 of unit j >> 1; short group: nibble h of
            // block j (formats.h).
            const uint32_t nib = (FULL ? w.q[j >> 1][2 * kappa + i] >> (4 * (j & 1)) : w.q[j][2 * kappa + i] >> (4 * h)) &
                                 0x0F0F0F0Fu;
            const h2 off = {(_Float16)1032, (_Float16)1032};   // 1024 + 8
            v[2 * i] = as_u32(pair02(nib) - off);
            v[2 * i + 1] = as_u32(pair13(nib) - off);
        } else {
            const uint32_t u = w.q[j][2 * kappa + i] ^ 0x80808080u;   // q + 128 per byte
            const h2 off = {(_Float16)1152, (_Float16)1152};          // 1024 + 128
            v[2 * i] = as_u32(pair02(u) - off);
            v[2 * i + 1] = as_u32(pair13(u) - off);
        }
    }
    (void)sc2;
    (void)nsc2;
    (void)h;
    return __builtin_bit_cast(h8, (u32x4){v[0], v[1], v[2], v[3]});
}

// Weight loads of one stage (the layout of formats.h, as load_weights in
// blockdot.h reads it), as raw buffer loads over the tile. FULLK (every
// group of the row a full 256-column group): always exactly kWeightLoads of
// them; the wait before each barrier leaves that many in flight and counts
// on them being the last vector memory instructions, so that it covers every
// copy issued before them. Rows with a short last Q8_0/Q4_0 group issue
// another count for that group and wait for all loads before each barrier.
template <unsigned T, bool FULLK>
constexpr int kWeightLoads = !FULLK ? 0 : T == Q8_0 ? 9 : 5;

template <unsigned T, bool FULLK>
__device__ __forceinline__ void load_stage(WStage<T> &w, __amdgpu_buffer_rsrc_t rs, const Lane &L, int g)
{
    auto ld = [&](int off) { return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0)); };
    const int R = L.R, r = L.r, h = L.h;
    if constexpr (T == Q4_K) {
        const int b = 144 * R * g;
#pragma unroll
        for (int p = 0; p < 4; ++p) w.q[p] = ld(b + 32 * R * p + 16 * R * h + 16 * r);
        w.sl = ld(b + 128 * R + 16 * r);
    } else {
        constexpr int quant = T == Q8_0 ? 32 : 16;
        const int b = (quant + 2) * 8 * R * g;
        auto full = [&]() {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (T == Q4_0 && j >= 4) w.q[j] = (u32x4){};
                else w.q[j] = ld(b + 32 * R * j + 16 * R * h + 16 * r);
            }
            const u32x4 d = ld(b + 8 * quant * R + 16 * r);
#pragma unroll
            for (int k = 0; k < 8; ++k) w.d[k] = k < 4 ? d[k] : 0u;
        };
        if constexpr (FULLK) {
            full();
        } else {
            const int nb = group_blocks(L, g);
            if (nb == 8) {
                full();
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int jj = j < nb ? j : nb - 1;
                    w.q[j] = ld(b + quant * R * jj + (T == Q8_0 ? 16 * R * h : 0) + 16 * r);
                    w.d[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, b + quant * R * nb + 2 * R * jj + 2 * r, 0, 0);
                }
            }
        }
    }
}

// Step g of prefill_f16: copy group g + 1 into the other buffer (its readers
// passed the last barrier), compute group g from `cur` (loaded two steps
// earlier), refill `cur` with group g + 2, wait for this wavefront's copies,
// barrier. Each B operand made from the weights serves the TW token tiles
// (two MFMAs each, one per activation piece). Copies and loads are
// unconditional (clamped to the last group): a branch would leave a path
// with another count of loads in flight. The two buffers come in as restrict
// pointers, which lets the compiler see that this step's LDS reads do not
// depend on the copies it issues.
template <unsigned T, int RT, int TW, bool FULLK>
__device__ __forceinline__ void group_step(WStage<T> &cur, f32x16 (&acc)[TW], lds_u8 *__restrict__ buf,
    lds_u8 *__restrict__ nbuf, const Pieces &p, const Lane &L, __amdgpu_buffer_rsrc_t rs, int a_off, int cols, int m0,
    int g, int groups)
{
    constexpr bool sums = T == Q4_K;
    // s_waitcnt immediate: vmcnt = kLoads (bits 3:0 and 15:14), expcnt and
    // lgkmcnt at their maxima (no wait).
    constexpr int kLoads = kWeightLoads<T, FULLK>;
    constexpr int kWaitCopies = (kLoads & 15) | ((kLoads >> 4) << 14) | (7 << 4) | (15 << 8);
    static_assert(kLoads < 64, "vmcnt field");
    const int lane = threadIdx.x & 63;
    copy_group<RT, TW>(nbuf, p, cols, m0, g + 1 < groups ? g + 1 : g, sums);
    // The weight loads below stay after the copies, in the compiler's view of
    // memory (the fence; the weights are not a restrict pointer) and in the
    // schedule.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const lds_u8 *xh = buf + a_off;
    if constexpr (T == Q4_K) {
        f32x16 C[TW];
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) C[tt] = (f32x16){};
        // Two token tiles: the A operands of block j + 1 are read while block
        // j's MFMAs run (xa[j % 2]: [token tile][K slice kappa][piece]). One
        // token tile (128 registers at eight wavefronts) reads each block's
        // operands in the block: the second set would spill.
        constexpr int kAhead = TW == 2 ? 1 : 0;
        h8 xa[2][TW][2][2];
        auto read_a = [&](int j, h8 (&dst)[TW][2][2]) {
#pragma unroll
            for (int tt = 0; tt < TW; ++tt)
#pragma unroll
                for (int kappa = 0; kappa < 2; ++kappa)
#pragma unroll
                    for (int pc = 0; pc < 2; ++pc)
                        dst[tt][kappa][pc] =
                            *(const h8 *)(xh + kTileBytes * tt + 128 * j + 32 * kappa + kPieceBytes * pc);
        };
        if constexpr (kAhead) {
            read_a(0, xa[0]);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (!kAhead) read_a(j, xa[j & 1]);
            else if (j < 7) read_a(j + 1, xa[(j + 1) & 1]);
            const uint32_t own = cur.sl[j >> 1];
            const float scf = (float)((own >> (12 * (j & 1))) & 63u);
            const h2 sc2 = {(_Float16)scf, (_Float16)scf};
            const h2 nsc2 = {(_Float16)(-1024.f * scf), (_Float16)(-1024.f * scf)};
#pragma unroll
            for (int kappa = 0; kappa < 2; ++kappa) {
                const h8 b = b_operand<T>(cur, j, kappa, L.h, sc2, nsc2);
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) {
                    C[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[j & 1][tt][kappa][0], b, C[tt], 0, 0, 0);
                    C[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[j & 1][tt][kappa][1], b, C[tt], 0, 0, 0);
                }
            }
            // Two token tiles: each MFMA followed by four VALU instructions
            // (the next operands) and one LDS read of the next block
            // (Q4_K 14336 x 4096 x 512: 172.6 -> 164.9 us; the compiler's own
            // order reads two operands, waits for them, then issues one
            // MFMA). One token tile keeps the compiler's order (this one
            // measured 36 % slower on 4096 x 4096 x 512).
            if constexpr (TW == 2) {
#pragma unroll
                for (int q = 0; q < 4 * TW; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                    if (j < 7) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
                }
            }
        }
        float d, dmin;
        group_scales<T>(cur, d, dmin);
        // Minimums: M = sum_j m_j * 2^-5 (sum of x s over block j) on one
        // fp16 MFMA per token tile, exact products: lane l supplies A = piece
        // l/32 (hi, lo) of the eight scaled block sums of token l % 32, and
        // B = m_j for row l % 32, j = 0..7 in both K halves. Then
        // acc += d C - 32 dmin M.
        h8 bm;
#pragma unroll
        for (int j = 0; j < 8; ++j) bm[j] = (_Float16)(int)((cur.sl[j >> 1] >> (12 * (j & 1) + 6)) & 63u);
        const float ndmin = -32.f * dmin;
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
            const h8 ys = *(const h8 *)(buf + kTileBytes * tt + 2 * kPieceBytes + 16 * lane);
            const f32x16 M = __builtin_amdgcn_mfma_f32_32x32x16_f16(ys, bm, (f32x16){}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[tt][r] = __builtin_fmaf(d, C[tt][r], __builtin_fmaf(ndmin, M[r], acc[tt][r]));
        }
    } else {
        // Per-block scales; a short last group has its own layout (formats.h).
        auto blocks = [&](auto full) {
            constexpr bool FULL = decltype(full)::value;
            const int nb = group_blocks(L, g);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (j >= nb) break;
                f32x16 C[TW];
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) C[tt] = (f32x16){};
#pragma unroll
                for (int kappa = 0; kappa < 2; ++kappa) {
                    const h8 b = b_operand<T, FULL>(cur, j, kappa, L.h, (h2){}, (h2){});
                    const int off = 128 * j + 32 * kappa;
#pragma unroll
                    for (int tt = 0; tt < TW; ++tt) {
                        const lds_u8 *x = xh + kTileBytes * tt + off;
                        C[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const h8 *)x, b, C[tt], 0, 0, 0);
                        C[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const h8 *)(x + kPieceBytes), b, C[tt], 0, 0, 0);
                    }
                }
                const float dj = f16_to_f32(block_d<FULL>(cur, j));
#pragma unroll
                for (int tt = 0; tt < TW; ++tt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[tt][r] += dj * C[tt][r];
            }
        };
        if (FULLK || group_blocks(L, g) == 8) blocks(std::true_type{});
        else blocks(std::false_type{});
    }
    load_stage<T, FULLK>(cur, rs, L, g + 2 < groups ? g + 2 : groups - 1);
    // This wavefront's copies are complete; then every wavefront's are,
    // past the barrier. (The fence keeps the loads above before the wait.)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitCopies);
    barrier();
}

// RT wavefronts (32-row tiles) per workgroup, TW token tiles of 32 per
// wavefront. TW = 1: 8 wavefronts (two workgroups per CU, four wavefronts
// per SIMD, at most 128 VGPRs) for Q4_K when the grid fills the chip, else 4
// (twice the workgroups). TW = 2: the 64 tokens' double buffer takes 139 KB
// of LDS, one workgroup per CU, 8 wavefronts of up to 256 VGPRs.
// The weights are deliberately not a restrict pointer: the compiler may
// then not move their loads across the memory fences of group_step.
template <unsigned T, int RT, int TW, bool FULLK>
__global__ __launch_bounds__(64 * RT) __attribute__((amdgpu_waves_per_eu(TW == 1 ? RT / 2 : RT / 4, TW == 1 ? RT / 2 : RT / 4))) void prefill_f16(
    const uint8_t *w, Pieces p, float *__restrict__ y, int rows, int cols, int batch, int token_blocks)
{
    __shared__ __align__(16) uint8_t smem0[kBufBytes<TW>], smem1[kBufBytes<TW>];
    lds_u8 *const B0 = (lds_u8 *)smem0, *const B1 = (lds_u8 *)smem1;
    constexpr bool sums = T == Q4_K;
    // The wavefront index is uniform: keeping it scalar keeps the tile base
    // and the copy addresses in SGPRs.
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const int by = blockIdx.x % token_blocks, bx = blockIdx.x / token_blocks;
    const int tile_raw = RT * bx + wave;
    const int tile = tile_raw < tiles ? tile_raw : tiles - 1;
    const int m0 = kTokens * TW * by, n = batch - m0;   // tokens left (> 0)
    const int R = rows - kTileRows * tile < kTileRows ? rows - kTileRows * tile : kTileRows;
    Lane L;
    L.tile = w + (size_t)kTileRows * tile * tiled_row_bytes<T>(cols);
    L.R = R;
    L.r = (lane & 31) < R ? (lane & 31) : R - 1;
    L.h = lane >> 5;
    L.slot = lane & 31;
    L.groups = (cols + kGroupCols - 1) / kGroupCols;
    L.blocks = cols / 32;
    const int groups = L.groups;
    // The tile's bytes (below 2^31: the library declines larger matrices).
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(L.tile), (short)0, (int)((size_t)R * tiled_row_bytes<T>(cols)), 0x00020000);

    WStage<T> st[2];
    // Both stages and the first copies complete before the loop, so the
    // first step reads only complete registers (after LDS copies are issued,
    // the compiler waits for all vector memory, those copies included, before
    // the first use of a register still loading; later steps read stages
    // completed by an earlier step's wait).
    copy_group<RT, TW>(B0, p, cols, m0, 0, sums);
    asm volatile("" ::: "memory");
    load_stage<T, FULLK>(st[0], rs, L, 0);
    load_stage<T, FULLK>(st[1], rs, L, groups > 1 ? 1 : 0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);
    barrier();

    // A operand of token r = lane % 32: columns 32j + 16h + 8kappa of the
    // group sit at pair r / 2, byte 32 (4j + 2h + kappa) + 16 (r & 1).
    const int a_off = kPairPitch * ((lane & 31) >> 1) + 16 * (lane & 1) + 64 * L.h;
    f32x16 acc[TW];
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) acc[tt] = (f32x16){};
    // Both steps of a pass unconditionally, an odd last group after the
    // loop: with the second step under a condition, the loop header would
    // merge a path on which stage 0's loads are still in flight, and the
    // compiler would wait for every load (the next group's copies included)
    // before each first step.
    int g = 0;
    for (; g + 1 < groups; g += 2) {
        group_step<T, RT, TW, FULLK>(st[0], acc, B0, B1, p, L, rs, a_off, cols, m0, g, groups);
        group_step<T, RT, TW, FULLK>(st[1], acc, B1, B0, p, L, rs, a_off, cols, m0, g + 1, groups);
    }
    if (g < groups) group_step<T, RT, TW, FULLK>(st[0], acc, B0, B1, p, L, rs, a_off, cols, m0, g, groups);

    if (tile_raw >= tiles || (lane & 31) >= R) return;
    const int row = kTileRows * tile + (lane & 31);
    // D register r of lane l is token 8 (r / 4) + 4 (l / 32) + r % 4 of its
    // token tile.
#pragma unroll
    for (int tt = 0; tt < TW; ++tt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 32 * tt + 8 * (r >> 2) + 4 * L.h + (r & 3);
            if (t < n) y[(size_t)(m0 + t) * rows + row] = acc[tt][r] * p.inv[m0 + t];
        }
}

}  // namespace

bool prefill_f16_supported(unsigned type) { return type == Q4_K || type == Q8_0 || type == Q4_0; }

// The pieces of the batch rounded up to 64 tokens (whole token blocks of
// either kernel shape).
size_t prefill_f16_workspace(int cols, int batch)
{
    const size_t np = ((size_t)batch + 2 * kTokens - 1) / (2 * kTokens) * (2 * kTokens);
    return np * ((size_t)4 * cols + (size_t)(cols / 32) * 4 + 4);
}

hipError_t launch_prefill_f16(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    int batch, void *workspace, hipStream_t s)
{
    const int np = (batch + 2 * kTokens - 1) / (2 * kTokens) * (2 * kTokens);
    const Pieces p = pieces_of(workspace, cols, np);
    hipLaunchKernelGGL(split_x, dim3((unsigned)batch), dim3(256), 0, s, x, cols, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const bool fullk = cols % kGroupCols == 0;
    // Two token tiles per wavefront (each weight operand serves four MFMAs)
    // where one workgroup per CU of 256 rows x 64 tokens fills the chip.
    const int tb2 = (batch + 2 * kTokens - 1) / (2 * kTokens);
    const int tb = (batch + kTokens - 1) / kTokens;
    const bool pair = (tiles + 7) / 8 * tb2 >= 256;
    // One token tile: Q8_0/Q4_0 stages (16 loads) do not fit 128 VGPRs
    // without spilling: four-wavefront workgroups only.
    const bool wide = type == Q4_K && (tiles + 7) / 8 * tb >= 256;
    const dim3 grid2((unsigned)((tiles + 7) / 8 * tb2));
    const dim3 grid((unsigned)((tiles + (wide ? 7 : 3)) / (wide ? 8 : 4) * tb));
#define FY_PREFILL(TT, RTT, TWW, FK, G, TB) \
    hipLaunchKernelGGL((prefill_f16<TT, RTT, TWW, FK>), G, dim3(64 * RTT), 0, s, w, p, y, rows, cols, batch, TB)
    switch (type) {
    case Q4_K:
        if (pair) FY_PREFILL(Q4_K, 8, 2, true, grid2, tb2);
        else if (wide) FY_PREFILL(Q4_K, 8, 1, true, grid, tb);
        else FY_PREFILL(Q4_K, 4, 1, true, grid, tb);
        break;
    case Q8_0:
        if (pair && fullk) FY_PREFILL(Q8_0, 8, 2, true, grid2, tb2);
        else if (pair) FY_PREFILL(Q8_0, 8, 2, false, grid2, tb2);
        else if (fullk) FY_PREFILL(Q8_0, 4, 1, true, grid, tb);
        else FY_PREFILL(Q8_0, 4, 1, false, grid, tb);
        break;
    case Q4_0:
        if (pair && fullk) FY_PREFILL(Q4_0, 8, 2, true, grid2, tb2);
        else if (pair) FY_PREFILL(Q4_0, 8, 2, false, grid2, tb2);
        else if (fullk) FY_PREFILL(Q4_0, 4, 1, true, grid, tb);
        else FY_PREFILL(Q4_0, 4, 1, false, grid, tb);
        break;
    default: return hipErrorInvalidValue;
    }
#undef FY_PREFILL
    return hipGetLastError();
}

}  // namespace fy
