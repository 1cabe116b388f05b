// Batch-1 matvec y = W x (token decode) for Q4_K, Q4_0, Q8_0 and Q6_K weights
// in the tiled layout of formats.h, with the block dot products on gfx950
// int8 MFMA (and, further down, the batches of 2..8 on the same layout).
//
// Activations. Each 32-column block of x is written as X * 2^(e-21) with
// 2^(e-1) <= max |x| < 2^e over the block and X integer, |X| <= 2^21, split
// into signed bytes X = a0 + 2^8 a1 + 2^16 a2. The conversion is one fma per
// digit: x 2^(21-e) + 1.5 * 2^23 (+ 128) rounds to the integer X (X + 128) in
// the low mantissa bits, whose bytes are the digits. Block dot products
// sum q * a_d are exact in int32.
//
// One token leaves most of an MFMA's A-rows empty, so each block takes the
// cheapest MFMA that still reads its whole 1 KiB weight operand as loaded:
// v_mfma_i32_16x16x64_i8 (half the cycles of v_mfma_i32_32x32x32_i8). Its B
// lane l holds column n = l%16 with K-chunk c = l/16; the weight load gives
// lane l row l%32 and column half l/32 of a 32-column block, so chunk c
// carries row half c%2 and column half c/2. A-rows 8 bsel + 4 rh + d hold
// digit d of x in the chunks of row half rh only (zeros elsewhere), so D rows
// 8 bsel + 4 rh .. +2 are the digit sums of rows 16 rh + n; blocks 2m and
// 2m + 1 chain through accumulator m as bsel = 0, 1. D lane l, register i
// holds D row 4(l/16) + i, column l%16, i.e. row l%32 of the weight tile and
// block 2m + l/32: lane half h holds blocks 2m + h (m = 0..3) in registers
// 0..2 of accumulator m and every epilogue instruction serves two blocks.
// The A operand of block k is read from LDS at a per-lane address fixed for
// the whole kernel. Q6_K, whose lane halves carry different 16-column scales,
// gives the column half the A-row bit of bsel: one block per MFMA, A-rows
// 8 h + 4 rh + d, so D lane l holds the sums of its own row l%32 and its own
// column half l/32 (see aoff6_of).
//
// Weights, as the reference decodes them (backend/core/llm_quant.c:70-142).
// Q4_K and Q4_0 bytes hold element l of blocks 2p (low nibble) and 2p + 1
// (high nibble); the low nibble enters the MFMA as q & 15, the high one in
// place as the signed byte (q & 0xF0) ^ 0x80 = 16 (q - 8), one instruction
// per word. Each block's activation data carries the factor and the
// correction that turn those sums into the format's: Q4_K w = (d sc) q - dmin
// m (odd blocks: 1/16 and + 8 sum x), Q4_0 w = d (q - 8) (even blocks: - 8
// sum x; odd blocks: 1/16), Q8_0 w = d q (signed bytes as they are). A
// non-finite x makes its block's sum of x, and with it every output,
// non-finite.
//
// The lane halves hold disjoint blocks of the same rows; their sums and those
// of the wavefronts of a tile are added in LDS in a fixed order.
#include "blockdot.h"
#include "kernels.h"

namespace fy {
namespace {

constexpr int kChunkCols = 16384;   // columns per launch (bounds the LDS copy of x)
constexpr int kMetaBytes = 16;      // per 32-column block: {s, c, sum x, 0}

// A-operand byte offsets within a group's 1 KiB of digits (digit slot d of
// block k at 128 k + 32 d, column half at + 16, slot 3 zero), per lane and
// block k = 2m + bsel of the 16x16x64 chain: lane l supplies A-row
// l%16 = 8 b + 4 rh + d for K-chunk c = l/16; it is live for its own bsel,
// row half c%2 == rh and digit d < 3, and reads the zero slot otherwise.
// Computed in registers (a few instructions per lane, no memory access before
// the weight loads).
__device__ __forceinline__ int aoff_of(int l, int k)
{
    const int m = l & 15, c = l >> 4, b = m >> 3, rh = (m >> 2) & 1, d = m & 3;
    const bool live = b == (k & 1) && (c & 1) == rh && d < 3;
    return 128 * k + 16 * (c >> 1) + 32 * (live ? d : 3);
}

// Q6_K: lane half h of block j (unit p = j/2, nibble m = j%2) holds columns
// 16 p%2 .. +15 of x-block xb = 4 (j/4) + 2 m + h, which has its own
// 16-column scale. Lane l supplies A-row l%16 = 8 hh + 4 rh + d for K-chunk
// c = l/16 (row half c%2, lane half c/2): live for rh == c%2, hh == c/2 and
// d < 3, reading digit d of x-block xb(j, hh); else the zero slot.
__device__ __forceinline__ int aoff6_of(int l, int j)
{
    const int m = l & 15, c = l >> 4, hh = m >> 3, rh = (m >> 2) & 1, d = m & 3;
    const bool live = (c & 1) == rh && (c >> 1) == hh && d < 3;
    const int xb = 4 * (j >> 2) + 2 * (j & 1) + (c >> 1);
    return 128 * xb + 32 * (live ? d : 3) + 16 * ((j >> 1) & 1);
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 8 lanes of an aligned half-row (quad swaps, then the
// half-row mirror); every lane receives the result.
__device__ __forceinline__ float sum8(float v)
{
    v += dppf<0xB1>(v);
    v += dppf<0x4E>(v);
    return v + dppf<0x141>(v);
}

__device__ __forceinline__ uint32_t fbits(float v) { return __builtin_bit_cast(uint32_t, v); }

template <int CTRL>
__device__ __forceinline__ uint32_t dppu(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t max8u(uint32_t v)
{
    v = __builtin_elementwise_max(v, dppu<0xB1>(v));
    v = __builtin_elementwise_max(v, dppu<0x4E>(v));
    return __builtin_elementwise_max(v, dppu<0x141>(v));
}

// Bytes b of four words, packed into one word (word i -> byte i).
__device__ __forceinline__ uint32_t pack_byte(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, int b)
{
    const uint32_t sel = 0x0c0c0000u | (uint32_t)(4 + b) << 8 | (uint32_t)b;
    return __builtin_amdgcn_perm(w1, w0, sel) | __builtin_amdgcn_perm(w3, w2, sel) << 16;
}

// Workgroups are dispatched round-robin over the eight XCDs: block b runs on
// XCD b % 8. Renumbered so that each XCD's blocks take one contiguous eighth
// of the rows (measured 1-6 % faster on 14336 x 4096 N=8 and the 128256-row
// Q6_K matvec; results are unchanged).
__device__ __forceinline__ int xcd_block()
{
    const int nb = gridDim.x, b = blockIdx.x;
    return nb % 8 ? b : (b % 8) * (nb / 8) + b / 8;
}

// Workgroup barrier that waits for no memory access: the empty asm keeps the
// compiler from moving loads across it, so it orders the issue of the loads
// before it ahead of those after it.
__device__ __forceinline__ void issue_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One 256-column group gl of x (chunk-local) into LDS: lane l holds columns
// 4l .. 4l+3, lanes 8b .. 8b+7 block b. Digit slot d of block xg at
// dig + 128 xg + 32 d (slot 3 zero); meta[xg] = {f 2^(e-21), c sum x,
// sum x, 0} with this lane's block factor f and correction c (kept as a
// product with sum x, so a non-finite sum stays non-finite).
__device__ __forceinline__ void quantize_group(float4 v, int gl, int lane, float fmul, float fcorr,
    uint8_t *__restrict__ dig, float4 *__restrict__ meta)
{
    // Largest magnitude of the block (integer order of |x| bit patterns).
    const uint32_t ma = fbits(v.x) & 0x7FFFFFFFu, mb = fbits(v.y) & 0x7FFFFFFFu;
    const uint32_t mc = fbits(v.z) & 0x7FFFFFFFu, md = fbits(v.w) & 0x7FFFFFFFu;
    const uint32_t mx = max8u(__builtin_elementwise_max(__builtin_elementwise_max(ma, mb), __builtin_elementwise_max(mc, md)));
    // x 2^sh with sh = 21 - e (capped where 2^sh would not be a float: such
    // blocks keep fewer digits of values below 2^-106).
    const int e = __builtin_amdgcn_frexp_expf(__builtin_bit_cast(float, mx));
    const int sh = 21 - e < 127 ? 21 - e : 127;
    const float scale = __builtin_bit_cast(float, (uint32_t)(sh + 127) << 23);
    // |x 2^sh| <= 2^21: x 2^sh + 1.5 * 2^23 stays in [2^23, 2^24), where the
    // float spacing is 1, so one fma rounds to the integer X and leaves the
    // bit pattern 0x4B400000 + X. Byte 0 of it is byte 0 of X; byte 1 of the
    // pattern with 128 more is byte 1 of X + 128; byte 2 of the pattern minus
    // 0x400000 - 32896 is byte 2 of X + 32896: the signed digits.
    constexpr float M0 = 12582912.f, M1 = 12583040.f;
    constexpr uint32_t K2 = 32896u - 0x400000u;
    const uint32_t a0 = fbits(__builtin_fmaf(v.x, scale, M0)), a1 = fbits(__builtin_fmaf(v.y, scale, M0));
    const uint32_t a2 = fbits(__builtin_fmaf(v.z, scale, M0)), a3 = fbits(__builtin_fmaf(v.w, scale, M0));
    const uint32_t w0 = pack_byte(a0, a1, a2, a3, 0);
    const uint32_t w1 = pack_byte(fbits(__builtin_fmaf(v.x, scale, M1)), fbits(__builtin_fmaf(v.y, scale, M1)),
                                  fbits(__builtin_fmaf(v.z, scale, M1)), fbits(__builtin_fmaf(v.w, scale, M1)), 1);
    const uint32_t w2 = pack_byte(a0 + K2, a1 + K2, a2 + K2, a3 + K2, 2);
    const float sx = sum8((v.x + v.y) + (v.z + v.w));
    const int xg = 8 * gl + (lane >> 3);
    uint8_t *dst = dig + 128 * xg + 4 * (lane & 7);
    *(uint32_t *)dst = w0;
    *(uint32_t *)(dst + 32) = w1;
    *(uint32_t *)(dst + 64) = w2;
    *(uint32_t *)(dst + 96) = 0u;
    if ((lane & 7) == 0)
        meta[xg] = make_float4(__builtin_amdgcn_ldexpf(fmul, -sh), fcorr * sx, sx, 0.f);
}

// One 256-column group of one 32-row tile, per format: the quant loads (16
// bytes each, lane half h holding columns 16h .. 16h+15 of a block) and the
// 16-byte scale word of the row.
template <unsigned T> struct MvStage;
template <> struct MvStage<Q4_K> { u32x4 q[4]; u32x4 sl; };   // sl: 6-bit sc/m, d, dmin
template <> struct MvStage<Q4_0> { u32x4 q[4]; u32x4 d; };    // d: eight fp16 block scales
template <> struct MvStage<Q8_0> { u32x4 q[8]; u32x4 d; };
template <> struct MvStage<Q6_K> { u32x4 ql[4], qh[4]; u32x4 sc; uint32_t d; };   // sc: int8 16-column scales
template <unsigned T> constexpr int kQuantLoads = T == Q8_0 ? 8 : 4;
template <unsigned T> constexpr int kGroupRowBytes = T == Q8_0 ? 272 : 144;   // per row, per group
template <unsigned T> constexpr int kScaleOffset = T == Q8_0 ? 256 : 128;    // per row, in the group

// Per-block activation factor and correction for lane l's block b = (l/8)%8
// of a group (see the header).
template <unsigned T> __device__ __forceinline__ float block_factor(int lane)
{
    if constexpr (T == Q6_K) return 0.25f;   // the weights enter as 4 (q6 - 32)
    return T != Q8_0 && ((lane >> 3) & 1) ? 0.0625f : 1.f;
}
template <unsigned T> __device__ __forceinline__ float block_correction(int lane)
{
    const bool odd = (lane >> 3) & 1;
    return T == Q4_K ? (odd ? 8.f : 0.f) : T == Q4_0 ? (odd ? 0.f : -8.f) : 0.f;
}

// B operand of block k of a stage.
template <unsigned T>
__device__ __forceinline__ i32x4 block_b(const MvStage<T> &w, int k)
{
    if constexpr (T == Q8_0) {
        return as_i32x4(w.q[k]);
    } else {
        const u32x4 q = w.q[k >> 1];
        return as_i32x4((k & 1) ? (q & 0xF0F0F0F0u) ^ 0x80808080u : q & 0x0F0F0F0Fu);
    }
}

// Q6_K B operand of MFMA block j for lane half h: 4 (q6 - 32) =
// (q6 << 2) ^ 0x80, from the nibble m = j%2 of unit p = j/2 (lane half h
// loaded ql half h, elements q = 2m + h) and bits 2q, 2q+1 of qh.
__device__ __forceinline__ i32x4 block_b6(const MvStage<Q6_K> &w, int j, int h)
{
    const int p = j >> 1, m = j & 1, q = 2 * m + h;
    u32x4 u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = m ? w.ql[p][k] >> 2 : w.ql[p][k] << 2;   // nibble to bits 2..5
        const uint32_t hi = w.qh[p][k] << (6 - 2 * q);                // two bits to 6..7
        u[k] = (lo & 0x3C3C3C3Cu) | ((hi & 0xC0C0C0C0u) ^ 0x80808080u);
    }
    return as_i32x4(u);
}

// One 256-column group of VT 32-row tiles: for each tile the eight block dots
// chained through one accumulator, then the scales. a points at this lane's
// A operand of block 0 of the group, mt at its activation data of block h;
// part[v] receives this lane half's share of the group's sum for row l%32 of
// tile v.
template <unsigned T, int VT>
__device__ __forceinline__ void group_dots(float (&part)[VT], const MvStage<T> (&w)[VT],
    const uint8_t *__restrict__ a, const int (&aoff)[8], const float4 *__restrict__ mt, int h)
{
    if constexpr (T == Q6_K) {
        // One MFMA per block (see aoff6_of); lane half h's block j reads
        // x-block 4 (j/4) + 2 (j%2) + h and the scale in byte q = 2 (j%2) + h
        // of scale word 2 (j/4) + (j/2)%2.
#pragma unroll
        for (int v = 0; v < VT; ++v) {
            i32x4 D[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                D[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const i32x4 *)(a + aoff[j]), block_b6(w[v], j, h),
                                                             (i32x4){0, 0, 0, 0}, 0, 0, 0);
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = j >> 2, jp = j & 3;
                const float4 md = mt[4 * c + 2 * (jp & 1)];
                // Sums reach 2^34: the top digit joins in float.
                const float G = __builtin_fmaf((float)D[j][2], 65536.f, (float)(D[j][1] * 256 + D[j][0]));
                const float t = __builtin_fmaf(G, md.x, md.y);
                const int q = 2 * (jp & 1) + h;
                // The builtin's result type is unsigned: convert it as the
                // signed value it holds.
                const float sc = (float)(int)__builtin_amdgcn_sbfe((int)w[v].sc[2 * c + (jp >> 1)], 8 * q, 8);
                sum = __builtin_fmaf(sc, t, sum);
            }
            part[v] = f16_to_f32(w[v].d & 0xFFFFu) * sum;
            // Tiles in load order (not interleaved by the scheduler): each
            // tile's work waits only for its own loads.
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        // One tile at a time: its four two-block chains, then its epilogue.
#pragma unroll
        for (int v = 0; v < VT; ++v) {
            i32x4 D[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                D[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const i32x4 *)(a + aoff[2 * m]), block_b<T>(w[v], 2 * m),
                                                             (i32x4){0, 0, 0, 0}, 0, 0, 0);
                D[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const i32x4 *)(a + aoff[2 * m + 1]),
                                                             block_b<T>(w[v], 2 * m + 1), D[m], 0, 0, 0);
            }
            // Lane half h: blocks 2m + h.
            float sum_s = 0.f, sum_m = 0.f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float4 md = mt[2 * m];
                // Sums reach 2^34: the top digit joins in float.
                const float G = __builtin_fmaf((float)D[m][2], 65536.f, (float)(D[m][1] * 256 + D[m][0]));
                const float t = __builtin_fmaf(G, md.x, md.y);
                if constexpr (T == Q4_K) {
                    // Slice word m packs sc and m of blocks 2m (bits 0..11) and
                    // 2m + 1 (bits 12..23).
                    const float sc = (float)__builtin_amdgcn_ubfe(w[v].sl[m], 12 * h, 6);
                    const float mn = (float)__builtin_amdgcn_ubfe(w[v].sl[m], 12 * h + 6, 6);
                    sum_s = __builtin_fmaf(sc, t, sum_s);
                    sum_m = __builtin_fmaf(mn, md.z, sum_m);
                } else {
                    // Scale word m holds the fp16 d of blocks 2m and 2m + 1.
                    sum_s = __builtin_fmaf(f16_to_f32(w[v].d[m] >> (16 * h)), t, sum_s);
                }
            }
            if constexpr (T == Q4_K) {
                const u32x4 sl = w[v].sl;   // byte 3 of the four words: d, dmin
                const uint32_t dd = (sl.x >> 24) | ((sl.y >> 24) << 8) | ((sl.z >> 24) << 16) | ((sl.w >> 24) << 24);
                part[v] = f16_to_f32(dd & 0xFFFFu) * sum_s - f16_to_f32(dd >> 16) * sum_m;
            } else {
                part[v] = sum_s;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Buffer resource over `bytes` bytes at p (raw loads, out-of-range reads
// return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes at voff + soff; NT: non-temporal (weights are streamed once).
template <bool NT>
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, int voff, int soff)
{
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, NT ? 2 : 0));
}

// Weights of group g of the tile (buffer r over the tile): q[p] at
// 32R p + 16R h + 16 r, slices at 128R + 16 r. The group offset joins the
// vector offset, which the buffer range check covers: groups past the tile
// (the ring's last stages) read zeros.
__device__ __forceinline__ void load_q4k(MvStage<Q4_K> &w, __amdgpu_buffer_rsrc_t tile, int R, int g, int vq, int vs)
{
    const int base = 144 * R * g;
#pragma unroll
    for (int p = 0; p < 4; ++p) w.q[p] = bload16<true>(tile, vq + base, 32 * R * p);
    w.sl = bload16<true>(tile, vs + base, 128 * R);
}

// The residual add and RMS normalization of the decoder folded into the
// x prologue (lane l holding elements 4 (64 q + l) .. + 3 of 256-column
// group q, as thread 64 q + l of the norm step):
// h = x + r (r may be null), xn = h * scale * g with
// scale = 1 / sqrt(sum h^2 / cols + eps), the sum of squares in double in
// the norm step's order; workgroup 0 writes h to hout.
struct NormIn {
    const float *r, *g;
    float *hout;
    float eps;
    // Rotary step of the q|k|v rows (positions null: none): q rows [0, qd)
    // rotated in y, k rows [qd, qd + kvd) rotated into keys and v rows into
    // values at the position's slot, as rope_qkv does.
    const int *positions;
    const float *freq;
    float *keys, *values;
    int qd, kvd, width, capacity;
    // Scaled products (x already h * g): the producing product's sums of
    // squares, kNormParts of them (see ResidOut).
    const double *parts;
    // The q|k|v row of the matrix's first row (even): a matrix may hold one
    // part of the rows (q|k of one weight type, v of another).
    int row0;
};

// Sums of squares handed from a product with the residual epilogue to the
// next product: one double per workgroup of the producer, zeros up to
// kNormParts.
constexpr int kNormParts = 256;

// The residual epilogue of one token's product (RESID): y is the residual,
// h = y + W x is written back in place (the addition the norm step makes),
// hn = h * g, and parts[j] = the double sum of h^2 over workgroup j's rows
// (parts[gridDim.x .. kNormParts) = 0).
struct ResidOut {
    const float *g;
    float *hn;
    double *parts;
    int block;   // this workgroup's index (set in the kernel)
};

// Element e of pair (e & ~1, e | 1) turned by `angle` as rope_qkv turns it:
// mine is the element's value, other its partner's.
__device__ __forceinline__ float rotate_element(float mine, float other, bool odd, float angle)
{
#pragma clang fp contract(off)
    const float c = cosf(angle), s = sinf(angle);
    return odd ? other * s + mine * c : mine * c - other * s;
}

__device__ __forceinline__ double sq4(float4 h)
{
#pragma clang fp contract(off)
    return (double)h.x * h.x + (double)h.y * h.y + (double)h.z * h.z + (double)h.w * h.w;
}
__device__ __forceinline__ float4 add4(float4 a, float4 b)
{
#pragma clang fp contract(off)
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 scale4(float4 h, float scale, float4 g)
{
#pragma clang fp contract(off)
    return make_float4(h.x * scale * g.x, h.y * scale * g.y, h.z * scale * g.z, h.w * scale * g.w);
}

// A wavefront's sum of one double per lane in the norm step's order
// (wave_sum; every lane ends with the same value).
__device__ __forceinline__ double wave_sum_pairs(double s)
{
    return wave_sum(s);
}

// The norm step's scale from its 16 wavefronts' sums of squares, in order.
__device__ __forceinline__ float norm_scale(const double *part, int cols, float eps)
{
    double total = part[0];
#pragma unroll
    for (int q = 1; q < 16; ++q) total += part[q];
    return (float)(1.0 / sqrt(total / (double)cols + (double)eps));
}

// One wavefront's share of the norm (its group in v, r and g loaded, zeros
// for a wavefront without one): v becomes xn; `writer` (workgroup 0) stores
// h. Every wavefront of the workgroup calls it once (one barrier).
__device__ __forceinline__ void norm_group(float4 &v, float4 r, float4 g, const NormIn &nm, int cols, int lane,
    int wave, bool writer, bool has_group)
{
    __shared__ double part[16];
    const float4 h = nm.r ? add4(v, r) : v;
    if (writer && has_group && nm.r && nm.hout) ((float4 *)nm.hout)[64 * wave + lane] = h;
    const double s = wave_sum_pairs(sq4(h));
    if (lane == 0) part[wave] = s;
    __syncthreads();
    v = scale4(h, norm_scale(part, cols, nm.eps), g);
}

// One workgroup per 32-row tile, KS wavefronts splitting its groups
// [g0c, g0c + ngc) (one column chunk); wavefront w takes chunk groups
// w, w + KS, ... through a RING-stage register ring.
// The engine's gated SiLU of one element, silu(g) u = g / (1 + e^-g) u
// (backend/core/llm_cpu.c:336-341), with the resident step's operations and
// none of them contracted (the step's file contracts nothing): uncontracted,
// the product cannot fuse into the block sums that use it either, so the
// vector is the step's bit for bit.
__device__ __forceinline__ float gated_silu(float g, float u)
{
#pragma clang fp contract(off)
    return g / (1.0f + expf(-g)) * u;
}
__device__ __forceinline__ float4 gated_silu(float4 g, float4 u)
{
    return make_float4(gated_silu(g.x, u.x), gated_silu(g.y, u.y), gated_silu(g.z, u.z), gated_silu(g.w, u.w));
}
// Gemma's gate, GELU with the tanh approximation (backend/core/llm_cpu.c:
// 329-341), in the resident step's operation order, uncontracted.
__device__ __forceinline__ float gated_gelu(float g, float u)
{
#pragma clang fp contract(off)
    return 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g))) * u;
}

// The gated activations of the interleaved gate|up products.
enum : int { kGateNone = 0, kGateSilu = 1, kGateGelu = 2 };

// GATE (SiLU or GELU): the rows come in 16-row blocks of gate rows and up
// rows (tile t holds gate rows 16t .. 16t + 15 as its rows 0..15, their up
// rows as 16..31) and y receives act(gate) * up, 16 values per tile at 16 t.
// SCALED: x is h * g of the decoder's residual h and norm weight g, and the
// row sums are multiplied by the norm's scale 1 / sqrt(sum h^2 / cols + eps)
// (W xn = scale W (h g)), the sum of squares from the kNormParts partial
// sums in nm.parts that the producing product's residual epilogue wrote.
// No workgroup waits for a reduction over the row before its products: the
// partial sums are added while the weights load and the scale joins at the
// final barrier. (Normalizing x in every workgroup instead, with the norm
// step's reduction before the quantization, measured 16.0 us at
// 28672 x 4096 against 15.3 us for the norm step followed by the product.)
template <int KS, int RING, int GATE = kGateNone, bool SCALED = false>
__global__ __launch_bounds__(64 * KS) __attribute__((amdgpu_waves_per_eu(2))) void matvec_q4k(
    const uint8_t *__restrict__ w, const float *__restrict__ x, float *__restrict__ y, int rows, int cols, int g0c,
    int ngc, int accumulate, NormIn nm)
{
    static_assert(!SCALED || 64 * KS >= kNormParts, "scaled: one partial sum per lane of the first wavefronts");
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[KS][64];
    const int ccols = (g0c + ngc) * kGroupCols < cols ? ngc * kGroupCols : cols - g0c * kGroupCols;
    const int xgroups = ccols / 32;
    uint8_t *sdig = lds;                                        // [xgroup][4 slots][32 B]
    float4 *smeta = (float4 *)(lds + (size_t)128 * xgroups);    // [xgroup]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = blockIdx.x, R = rows - kTileRows * t < kTileRows ? rows - kTileRows * t : kTileRows;
    const int h = lane >> 5, r = (lane & 31) < R ? (lane & 31) : R - 1;
    const size_t row_bytes = tiled_row_bytes<Q4_K>(cols);
    const __amdgpu_buffer_rsrc_t tile = buffer_of(w + (size_t)kTileRows * t * row_bytes, (uint32_t)(R * row_bytes));
    const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)ccols * 4u);
    const int vq = 16 * R * h + 16 * r, vs = 16 * r, vx = 16 * lane;
    // This wave's chunk groups: wave + KS k for k < ns.
    const int ns = wave < ngc ? (ngc - wave + KS - 1) / KS : 0;
    // The group goes into the vector offset, which the buffer range check
    // covers (the scalar offset is added after the check).
    auto xload = [&](int gl) { return __builtin_bit_cast(float4, bload16<false>(xb, vx + 1024 * gl, 0)); };

    // 1. x of the first RING groups, then the weights (loads complete in
    //    order: what the quantization needs comes first).
    float4 px[RING];
    // Unconditional: past the chunk the buffer range check returns zeros.
#pragma unroll
    for (int k = 0; k < RING; ++k) px[k] = xload(wave + KS * k);
    double pv = 0.0;
    if constexpr (SCALED) pv = nm.parts[(64 * wave + lane) & (kNormParts - 1)];
    asm volatile("" ::: "memory");
    MvStage<Q4_K> st[RING];
#pragma unroll
    for (int k = 0; k < RING; ++k) load_q4k(st[k], tile, R, g0c + wave + KS * k, vq, vs);
    // The partial sums, in the same order in every workgroup: wavefront
    // w < kNormParts / 64 adds 64 w .. 64 w + 63 (lanes l and l ^ o paired),
    // wave 0 the wavefronts' sums in turn after the final barrier.
    __shared__ double part[SCALED ? kNormParts / 64 : 1];
    if constexpr (SCALED) {
        if (wave < kNormParts / 64) {
            pv = wave_sum_pairs(pv);
            if (lane == 0) part[wave] = pv;
        }
    }

    // 2. Digits of this wave's groups into LDS.
    const float fmul = block_factor<Q4_K>(lane), fcorr = block_correction<Q4_K>(lane);
#pragma unroll
    for (int k = 0; k < RING; ++k) {
        asm volatile("" : "+v"(px[k].x), "+v"(px[k].y), "+v"(px[k].z), "+v"(px[k].w) :: "memory");
        if (k < ns) quantize_group(px[k], wave + KS * k, lane, fmul, fcorr, sdig, smeta);
    }
    for (int k = RING; k < ns; ++k)
        quantize_group(xload(wave + KS * k), wave + KS * k, lane, fmul, fcorr, sdig, smeta);
    // Each wave reads back only the groups it wrote.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 3. A-operand offsets (per lane, fixed for the kernel; loaded with x).
    int aoff[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) aoff[k] = aoff_of(lane, k);
    const uint8_t *abase = sdig + 1024 * wave;
    const float4 *mbase = smeta + 8 * wave + h;

    // 4. The ring: stage k holds group i + k; after computing it, it loads
    //    group i + k + RING. Loads are unconditional (static wait counts):
    //    past the matrix the buffer range check returns zeros.
    float acc = 0.f;
    auto pass = [&](int i) {
#pragma unroll
        for (int k = 0; k < RING; ++k) {
            if (i + k < ns) {
                const int gl = KS * (i + k);
                float part[1];
                group_dots<Q4_K, 1>(part, *(const MvStage<Q4_K>(*)[1])&st[k], abase + 1024 * gl, aoff, mbase + 8 * gl, h);
                acc += part[0];
            }
            load_q4k(st[k], tile, R, g0c + wave + KS * (i + k + RING), vq, vs);
        }
    };
    pass(0);
    for (int i = RING; i < ns; i += RING) pass(i);

    // 5. Lane halves and wavefronts, in a fixed order.
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0 || lane >= R) return;
    float v = red[0][lane] + red[0][lane + 32];
#pragma unroll
    for (int q = 1; q < KS; ++q) v += red[q][lane] + red[q][lane + 32];
    if constexpr (SCALED) {
        double total = part[0];
#pragma unroll
        for (int q = 1; q < kNormParts / 64; ++q) total += part[q];
        v *= (float)(1.0 / sqrt(total / (double)cols + (double)nm.eps));
    }
    if constexpr (GATE != kGateNone) {
        // Every tile is whole (R = 32): lane l < 16 takes its up row from l + 16.
        const float up = __shfl_down(v, 16, 32);
        if (lane < 16) y[16 * t + lane] = GATE == kGateGelu ? gated_gelu(v, up) : gated_silu(v, up);
        return;
    }
    float *dst = y + kTileRows * t + lane;
    *dst = accumulate ? *dst + v : v;
}

// Weights of group g for the lanes of one 32-row virtual tile in the whole
// matrix's buffer wb. A lane's row sits in packed tile tb (byte offset of its
// 32-row tile), at r with R rows in that tile: quant load p at
// tb + R(GB g + 32 p + 16 h) + 16 r, the scale word at tb + R(GB g + S) + 16 r
// (GB, S: the format's group bytes and scale offset per row). FULL (R = 32
// for every lane of the workgroup): the group and field parts are scalar
// offsets.
//
// A stage is loaded field by field: field 0 is the scale word (Q6_K: the
// 16-column scales and d), field 1 + p quant word p (Q6_K: ql and qh of unit
// p), in the order the dots use them. Issue order is fixed (the empty asm
// statements keep the compiler from reordering the loads) and a wavefront's
// loads return in order, so each block's dots wait only for the loads before
// its own, and the work left after the last load of a stage is one block's
// (left to the compiler, the scale word went last and every scale multiply
// waited for the whole stage).
template <unsigned T> constexpr int kFields = 1 + (T == Q6_K ? 4 : kQuantLoads<T>);

template <unsigned T, bool FULL>
__device__ __forceinline__ void load_field(MvStage<T> &w, __amdgpu_buffer_rsrc_t wb, int vq, int vs, int R, int g,
    int vd, int G, int f)
{
    if constexpr (T == Q6_K) {
        // Per group 208 R bytes: units p at 48 R p (ql half h at + 16 R h,
        // qh at + 32 R), scales at 192 R; the d of all G groups after them
        // (2 bytes per row at vd = tile + 2 r, group g at 208 R G + 2 R g).
        if (f == 0) {
            if constexpr (FULL) {
                w.sc = bload16<true>(wb, vs, kTileRows * (208 * g + 192));
                w.d = __builtin_amdgcn_raw_buffer_load_b16(wb, vd, kTileRows * (208 * G + 2 * g), 2);
            } else {
                w.sc = bload16<true>(wb, vs + R * (208 * g + 192), 0);
                w.d = __builtin_amdgcn_raw_buffer_load_b16(wb, vd + R * (208 * G + 2 * g), 0, 2);
            }
        } else {
            const int p = f - 1;
            if constexpr (FULL) {
                w.ql[p] = bload16<true>(wb, vq, kTileRows * (208 * g + 48 * p));
                w.qh[p] = bload16<true>(wb, vs, kTileRows * (208 * g + 48 * p + 32));
            } else {
                w.ql[p] = bload16<true>(wb, vq + R * (208 * g + 48 * p), 0);
                w.qh[p] = bload16<true>(wb, vs + R * (208 * g + 48 * p + 32), 0);
            }
        }
    } else {
        constexpr int GB = kGroupRowBytes<T>, S = kScaleOffset<T>;
        if (f == 0) {
            u32x4 sw;
            if constexpr (FULL) sw = bload16<true>(wb, vs, kTileRows * (GB * g + S));
            else sw = bload16<true>(wb, vs + R * (GB * g + S), 0);
            if constexpr (T == Q4_K) w.sl = sw;
            else w.d = sw;
        } else {
            const int p = f - 1;
            if constexpr (FULL) w.q[p] = bload16<true>(wb, vq, kTileRows * GB * g + 1024 * p);
            else w.q[p] = bload16<true>(wb, vq + R * (GB * g + 32 * p), 0);
        }
    }
}

template <unsigned T, bool FULL>
__device__ __forceinline__ void load_rows(MvStage<T> &w, __amdgpu_buffer_rsrc_t wb, int vq, int vs, int R, int g,
    int vd = 0, int G = 0)
{
#pragma unroll
    for (int f = 0; f < kFields<T>; ++f) {
        load_field<T, FULL>(w, wb, vq, vs, R, g, vd, G, f);
        asm volatile("" ::: "memory");
    }
    // Nothing after the loads is scheduled among them (an activation
    // instruction placed there waited for the x loads and held back the rest
    // of the stage).
    __builtin_amdgcn_sched_barrier(0);
}

// The same for VT virtual tiles at once, field by field (field f of every
// tile before field f + 1): for dots that take block b of every tile
// together.
template <unsigned T, bool FULL, int VT>
__device__ __forceinline__ void load_rows_fields(MvStage<T> (&w)[VT], __amdgpu_buffer_rsrc_t wb, const int (&vq)[VT],
    const int (&vs)[VT], const int (&R)[VT], int g, const int (&vd)[VT], int G)
{
#pragma unroll
    for (int f = 0; f < kFields<T>; ++f) {
#pragma unroll
        for (int v = 0; v < VT; ++v) load_field<T, FULL>(w[v], wb, vq[v], vs[v], R[v], g, vd[v], G, f);
        asm volatile("" ::: "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Row-balanced batch-1 matvec. One workgroup of sixteen wavefronts per CU
// takes a contiguous range of rw rows (rw = ceil(rows / workgroups)) as VT
// virtual 32-row tiles: lane l of virtual tile v owns row base + 32 v + l%32,
// wherever that row sits in the packed 32-row tiles, so every CU streams the
// same bytes whatever the row count. Wavefront w takes chunk groups
// w, w + 16, ... of all VT tiles: it reads and quantizes only those groups of
// x (no barrier before the dots), and each A operand it reads from LDS serves
// the VT tiles' interleaved MFMA chains. MULTI: some wavefront has more
// stages than its ring holds (rows wider than KS P RING groups); without it
// the ring is never refilled and that code is left out (it costs registers).
//
// P = 2 (up to 16 rows per workgroup, VT = 1): a stage holds two of
// the wavefront's groups, j = 2k and 2k + 1, for the same 16 rows. Lane l
// takes row l%16 of group j = 2k + (l/16)%2, so every 1 KiB load carries
// distinct bytes (with 32-row lanes, 16 of them would repeat the last row)
// and a wavefront needs half the memory round trips. The MFMA sees the same
// lane layout as at P = 1, with the second group where the second row half
// was: B chunk c = l/16 and the A-row half rh select group 2k + c%2 (the
// A operand of lanes with c odd is read from that group's digits), and D
// lane l holds row l%16 of group 2k + (l/16)%2. A stage whose second group
// is past the wavefront's last one repeats its first group in those lanes,
// and their sums are dropped.

// GATED: the vector multiplied is silu(x) * up elementwise (x and up of the
// same chunk layout), formed as each group is loaded. NORM: the residual add
// and norm of NormIn in the x prologue, one group per wavefront.

template <unsigned T, int VT, int RING, int KS, int P, bool FULL, bool MULTI, bool GATED, bool NORM = false,
    bool ROPE = false, bool RESID = false, bool SCALED = false>
__device__ __forceinline__ void matvec_rows_body(const uint8_t *__restrict__ w, const float *__restrict__ x,
    const float *__restrict__ up, float *__restrict__ y, int rows, int cols, int base, int live, int g0c, int ngc,
    int accumulate, uint8_t *sdig, float4 *smeta, float (*red)[VT][64], const NormIn &nm = NormIn{},
    const ResidOut &ro = ResidOut{})
{
    static_assert(!ROPE || ((NORM || SCALED) && VT == 1), "rotary: the normed one-tile product");
    static_assert(!SCALED || (!NORM && !GATED && KS * 64 >= kNormParts), "scaled: x is already h * g");
    static_assert(!RESID || (VT * kTileRows / P <= 64 && !NORM && !GATED), "residual: wave 0 holds every row");
    // The residual epilogue's inputs, loaded first (lane l: row slot l,
    // clamped into the workgroup's rows; used after the reduction).
    float res_in = 0.f, g_in = 0.f;
    if constexpr (RESID) {
        const int slot = (int)(threadIdx.x & 63), last = (VT * kTileRows / P < live ? VT * kTileRows / P : live) - 1;
        const int row = base + (slot < last ? slot : last);
        res_in = y[row];
        g_in = ro.g[row];
    }
    // The rotary inputs, loaded first (used after the reduction).
    int rope_position = 0;
    float rope_freq = 0.f;
    if constexpr (ROPE) {
        rope_position = nm.positions[0];
        const int row = nm.row0 + base + (int)(threadIdx.x & 63);
        const int e = row < nm.qd ? row : row - nm.qd;
        rope_freq = row < nm.qd + nm.kvd ? nm.freq[(e % nm.width) >> 1] : 0.f;
    }
    static_assert(!NORM || (P == 1 && RING == 1 && KS == 16 && !MULTI && !GATED), "norm: one group per wavefront");
    static_assert(P == 1 || (P == 2 && VT == 1), "two groups per stage: one 16-row virtual tile");
    constexpr int RT = kTileRows / P;   // rows per virtual tile
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, s = P == 2 ? (lane >> 4) & 1 : 0;
    const size_t row_bytes = tiled_row_bytes<T>(cols);
    const int tiles = (rows + kTileRows - 1) / kTileRows, rlast = rows - kTileRows * (tiles - 1);
    const __amdgpu_buffer_rsrc_t wb = buffer_of(w, (uint32_t)((size_t)rows * row_bytes));
    const uint32_t xbytes = (uint32_t)((g0c + ngc) * kGroupCols <= cols ? ngc : 0) * 1024u;
    const __amdgpu_buffer_rsrc_t xb = buffer_of(x, xbytes);
    const __amdgpu_buffer_rsrc_t ub = buffer_of(GATED ? up : x, GATED ? xbytes : 0u);
    // Lane offsets per virtual tile; rows past this workgroup's repeat its
    // last row (same addresses: no extra traffic).
    int vq[VT], vs[VT], vd[VT], R[VT];
#pragma unroll
    for (int v = 0; v < VT; ++v) {
        const int rl = RT * v + (lane & (RT - 1));
        const int row = base + (rl < live ? rl : live - 1);
        const int t = row / kTileRows, r = row - kTileRows * t;
        R[v] = t == tiles - 1 ? rlast : kTileRows;
        const int tb = (int)((size_t)kTileRows * t * row_bytes);
        vq[v] = tb + 16 * R[v] * h + 16 * r;
        vs[v] = tb + 16 * r;
        vd[v] = tb + 2 * r;
    }
    const int G = cols / kGroupCols;
    // This wave's chunk groups: wave + KS j for j < ns, in nst stages of P.
    const int ns = wave < ngc ? (ngc - wave + KS - 1) / KS : 0;
    const int nst = (ns + P - 1) / P;
    // Stage k of lane half s: its own group P k + s while there is one, else
    // the stage's first (and stages past the wave's last repeat that one).
    auto full_of = [&](int k) { return P == 1 || P * k + 1 < ns; };
    auto j_of = [&](int k) { const int kk = k < nst ? k : nst - 1; return P * kk + (full_of(kk) ? s : 0); };
    // Lane half s = 1 of a full stage: one group (KS groups of the chunk) on,
    // in the quant and scale fields (sq) and in Q6_K's d array (sd).
    constexpr int GB = T == Q6_K ? 208 : kGroupRowBytes<T>;
    int sq[VT], sd[VT];
#pragma unroll
    for (int v = 0; v < VT; ++v) {
        sq[v] = P == 2 && s ? KS * R[v] * GB : 0;
        sd[v] = P == 2 && s ? KS * R[v] * 2 : 0;
    }
    auto stage_load = [&](MvStage<T>(&st)[VT], int k) {
        const int kk = k < nst ? k : nst - 1, add = full_of(kk);
#pragma unroll
        for (int v = 0; v < VT; ++v)
            load_rows<T, FULL>(st[v], wb, vq[v] + (add ? sq[v] : 0), vs[v] + (add ? sq[v] : 0), R[v],
                               g0c + wave + KS * P * kk, vd[v] + (add ? sd[v] : 0), G);
    };
    float acc[VT];
#pragma unroll
    for (int v = 0; v < VT; ++v) acc[v] = 0.f;
    // 1. x of the first RING stages, then the weights (a wave's loads
    //    complete in order: what the quantization needs comes first). No
    //    workgroup barrier between the two: each wave issues its weights as
    //    soon as it runs (a barrier there, which put every wave's x ahead of
    //    all weights, held the first weights until the last of the 16 waves
    //    had started: 0.1 us per launch at 14336 x 4096, 0.27 us at Q8_0
    //    4096 x 4096). Groups past the wave's last repeat it. The x loads are unconditional, with the group in the
    //    range-checked vector offset (a wave without groups reads zeros):
    //    loaded under a condition, their registers would be merged after it,
    //    and the merge waits for the loads, holding back every weight load
    //    behind a full memory round trip.
    auto xgroup = [&](int j) { return wave + KS * (j < ns ? j : ns - 1); };
    float4 px[P * RING], pu[P * RING];
#pragma unroll
    for (int j = 0; j < P * RING; ++j) {
        px[j] = __builtin_bit_cast(float4, bload16<false>(xb, 16 * lane + 1024 * (ns > 0 ? xgroup(j) : wave), 0));
        if constexpr (GATED)
            pu[j] = __builtin_bit_cast(float4, bload16<false>(ub, 16 * lane + 1024 * (ns > 0 ? xgroup(j) : wave), 0));
    }
    float4 pr = {}, pg = {};
    if constexpr (NORM) {
        const __amdgpu_buffer_rsrc_t rb = buffer_of(nm.r ? nm.r : x, nm.r ? xbytes : 0u), gb = buffer_of(nm.g, xbytes);
        pr = __builtin_bit_cast(float4, bload16<false>(rb, 16 * lane + 1024 * wave, 0));
        pg = __builtin_bit_cast(float4, bload16<false>(gb, 16 * lane + 1024 * wave, 0));
    }
    // SCALED: the producer's partial sums of squares, added while the
    // weights load (as in matvec_q4k: wavefront w < kNormParts / 64 adds
    // 64 w .. 64 w + 63, wave 0 the wavefronts' sums after the barrier).
    __shared__ double spart[SCALED ? kNormParts / 64 : 1];
    double pv = 0.0;
    if constexpr (SCALED) pv = nm.parts[(64 * wave + lane) & (kNormParts - 1)];
    asm volatile("" ::: "memory");
    auto scaled_parts = [&]() {
        if (wave < kNormParts / 64) {
            pv = wave_sum_pairs(pv);
            if (lane == 0) spart[wave] = pv;
        }
    };
    if (ns > 0) {
        MvStage<T> st[RING][VT];
#pragma unroll
        for (int k = 0; k < RING; ++k) stage_load(st[k], k);

        if constexpr (NORM) norm_group(px[0], pr, pg, nm, cols, lane, wave, base == 0, xbytes > 0);
        if constexpr (SCALED) scaled_parts();   // after this wave's weights are requested
        // 2. Digits of this wave's groups into LDS.
        const float fmul = block_factor<T>(lane), fcorr = block_correction<T>(lane);
#pragma unroll
        for (int j = 0; j < P * RING; ++j) {
            asm volatile("" : "+v"(px[j].x), "+v"(px[j].y), "+v"(px[j].z), "+v"(px[j].w) :: "memory");
            if constexpr (GATED) {
                asm volatile("" : "+v"(pu[j].x), "+v"(pu[j].y), "+v"(pu[j].z), "+v"(pu[j].w) :: "memory");
                px[j] = gated_silu(px[j], pu[j]);
            }
            if (j < ns) quantize_group(px[j], xgroup(j), lane, fmul, fcorr, sdig, smeta);
        }
        if constexpr (MULTI)
            for (int j = P * RING; j < ns; ++j) {
                float4 v = __builtin_bit_cast(float4, bload16<false>(xb, 16 * lane, 1024 * xgroup(j)));
                if constexpr (GATED) v = gated_silu(v, __builtin_bit_cast(float4, bload16<false>(ub, 16 * lane, 1024 * xgroup(j))));
                quantize_group(v, xgroup(j), lane, fmul, fcorr, sdig, smeta);
            }
        // Each wave reads back only the groups it wrote.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // 3. The ring: stage k holds stage i + k of every virtual tile; after
        //    computing it, it loads stage i + k + RING (while there is one).
        int aoff[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) aoff[k] = T == Q6_K ? aoff6_of(lane, k) : aoff_of(lane, k);
        const uint8_t *abase = sdig + 1024 * wave;
        const float4 *mbase = smeta + 8 * wave + h;
        auto pass = [&](int i) {
#pragma unroll
            for (int k = 0; k < RING; ++k) {
                if (i + k < nst) {
                    const int gl = KS * j_of(i + k);
                    float part[VT];
                    group_dots<T, VT>(part, st[k], abase + 1024 * gl, aoff, mbase + 8 * gl, h);
                    const bool keep = full_of(i + k) || s == 0;
#pragma unroll
                    for (int v = 0; v < VT; ++v) acc[v] += keep ? part[v] : 0.f;
                    if (MULTI && i + k + RING < nst) stage_load(st[k], i + k + RING);
                }
            }
        };
        pass(0);
        if constexpr (MULTI)
            for (int i = RING; i < nst; i += RING) pass(i);
    } else if constexpr (NORM) {
        // A wavefront without a group still meets the others at the norm's
        // barrier (its sum is zero).
        norm_group(px[0], pr, pg, nm, cols, lane, wave, false, false);
    } else if constexpr (SCALED) {
        scaled_parts();
    }

    // 4. Lane halves and wavefronts, in a fixed order. Wave w sums slots
    //    64 w + l = RT v + r: row r of virtual tile v. All 2 KS partials are
    //    read before the first add, so the reads cost one LDS round trip
    //    (read, wait, add in turn measured 0.1 us slower at the end of every
    //    launch). At P = 2 the two groups of a stage are added first (lanes
    //    l and l ^ 16).
    if constexpr (P == 2) acc[0] += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, acc[0]), 0x401F));
#pragma unroll
    for (int v = 0; v < VT; ++v) red[wave][v][lane] = acc[v];
    __syncthreads();
    // VT RT result rows: wave 0 sums the first 64, wave 1 the next (VT = 3).
    if (64 * wave >= VT * RT) return;
    const int v = (64 * wave + lane) / RT, r = lane & (RT - 1);
    auto row_sum = [&]() {
        float p[2 * KS];
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            p[2 * q] = red[q][v][r];
            p[2 * q + 1] = red[q][v][r + 32];
        }
        asm volatile("" ::: "memory");
        float sum = p[0] + p[1];
#pragma unroll
        for (int q = 1; q < KS; ++q) sum += p[2 * q] + p[2 * q + 1];
        return sum;
    };
    if constexpr (RESID) {
        // Every lane of wave 0 joins the sum of squares (rows past the
        // workgroup's add zero), summed as the norm step pairs lanes.
        double sq = 0.0;
        if (v < VT && RT * v + r < live) {
            const float h = res_in + row_sum();
            y[base + RT * v + r] = h;
            ro.hn[base + RT * v + r] = h * g_in;
            sq = (double)h * h;
        }
        sq = wave_sum_pairs(sq);
        if (lane == 0) ro.parts[ro.block] = sq;
        if (ro.block == 0)
            for (int i = (int)gridDim.x + lane; i < kNormParts; i += 64) ro.parts[i] = 0.0;
        return;
    }
    if (v >= VT || RT * v + r >= live) return;
    float sum = row_sum();
    if constexpr (SCALED) {
        double total = spart[0];
#pragma unroll
        for (int q = 1; q < kNormParts / 64; ++q) total += spart[q];
        sum *= (float)(1.0 / sqrt(total / (double)cols + (double)nm.eps));
    }
    float *dst = y + base + RT * v + r;
    if constexpr (ROPE) {
        // Rows come in pairs within the workgroup (base and live even).
        const float other = __shfl_xor(sum, 1, 64);
        const int row = nm.row0 + base + r, position = rope_position;
        if (position >= 0 && position < nm.capacity) {
            const bool is_q = row < nm.qd, is_k = !is_q && row < nm.qd + nm.kvd;
            const int e = is_q ? row : row - nm.qd;
            if (is_q || is_k) {
                const float out = rotate_element(sum, other, e & 1, (float)position * rope_freq);
                if (is_q) {
                    *dst = out;
                    return;
                }
                nm.keys[(size_t)position * nm.kvd + e] = out;
            } else {
                nm.values[(size_t)position * nm.kvd + (row - nm.qd - nm.kvd)] = sum;
            }
        }
        *dst = sum;
        return;
    }
    *dst = accumulate ? *dst + sum : sum;
}

template <unsigned T, int VT, int RING, int KS, int P, bool MULTI, bool GATED = false>
__global__ __launch_bounds__(64 * KS) void matvec_rows(const uint8_t *__restrict__ w, const float *__restrict__ x,
    const float *__restrict__ up, float *__restrict__ y, int rows, int cols, int rw, int g0c, int ngc, int accumulate)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[KS][VT][64];
    const int ccols = (g0c + ngc) * kGroupCols < cols ? ngc * kGroupCols : cols - g0c * kGroupCols;
    uint8_t *sdig = lds;                                              // [xgroup][4 slots][32 B]
    float4 *smeta = (float4 *)(lds + (size_t)128 * (ccols / 32));     // [xgroup]
    const int base = xcd_block() * rw, live = rows - base < rw ? rows - base : rw;
    // Every lane of the workgroup in a 32-row tile (only the last tile of the
    // matrix may be shorter): group and field offsets are scalar.
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    if (rows % kTileRows == 0 || base + live <= kTileRows * (tiles - 1))
        matvec_rows_body<T, VT, RING, KS, P, true, MULTI, GATED>(w, x, up, y, rows, cols, base, live, g0c, ngc,
                                                                accumulate, sdig, smeta, red);
    else
        matvec_rows_body<T, VT, RING, KS, P, false, MULTI, GATED>(w, x, up, y, rows, cols, base, live, g0c, ngc,
                                                                 accumulate, sdig, smeta, red);
}

// matvec_rows of one column chunk with the residual epilogue (y: the
// residual, updated in place).
template <unsigned T, int VT, int RING, int KS, int P, bool MULTI>
__global__ __launch_bounds__(64 * KS) void matvec_rows_resid(const uint8_t *__restrict__ w,
    const float *__restrict__ x, float *__restrict__ y, int rows, int cols, int rw, ResidOut ro)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[KS][VT][64];
    uint8_t *sdig = lds;
    float4 *smeta = (float4 *)(lds + (size_t)128 * (cols / 32));
    ro.block = xcd_block();
    const int base = ro.block * rw, live = rows - base < rw ? rows - base : rw;
    const int tiles = (rows + kTileRows - 1) / kTileRows, ngc = cols / kGroupCols;
    if (rows % kTileRows == 0 || base + live <= kTileRows * (tiles - 1))
        matvec_rows_body<T, VT, RING, KS, P, true, MULTI, false, false, false, true>(
            w, x, nullptr, y, rows, cols, base, live, 0, ngc, 0, sdig, smeta, red, NormIn{}, ro);
    else
        matvec_rows_body<T, VT, RING, KS, P, false, MULTI, false, false, false, true>(
            w, x, nullptr, y, rows, cols, base, live, 0, ngc, 0, sdig, smeta, red, NormIn{}, ro);
}

// One token's product of the normalized residual: matvec_rows with one
// 256-column group per wavefront (cols <= 4096) and the norm in the x
// prologue.
// SCALED: x is h * g with the norm's scale from nm.parts instead (see
// matvec_q4k), the rotary step after the scale.
template <unsigned T, bool ROPE = false, bool SCALED = false>
__global__ __launch_bounds__(1024) void matvec_rows_norm(const uint8_t *__restrict__ w, const float *__restrict__ x,
    float *__restrict__ y, int rows, int cols, int rw, NormIn nm)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[16][1][64];
    uint8_t *sdig = lds;
    float4 *smeta = (float4 *)(lds + (size_t)128 * (cols / 32));
    const int base = xcd_block() * rw, live = rows - base < rw ? rows - base : rw;
    const int tiles = (rows + kTileRows - 1) / kTileRows, ngc = cols / kGroupCols;
    if (rows % kTileRows == 0 || base + live <= kTileRows * (tiles - 1))
        matvec_rows_body<T, 1, 1, 16, 1, true, false, false, !SCALED, ROPE, false, SCALED>(
            w, x, nullptr, y, rows, cols, base, live, 0, ngc, 0, sdig, smeta, red, nm);
    else
        matvec_rows_body<T, 1, 1, 16, 1, false, false, false, !SCALED, ROPE, false, SCALED>(
            w, x, nullptr, y, rows, cols, base, live, 0, ngc, 0, sdig, smeta, red, nm);
}

// The rotary product over q|k|v rows stored as two matrices of types T0
// (rows [0, rows0)) and T1 (the rest) in one launch: workgroups [0, wgs0)
// (in xcd_block order) take rw0 rows each of the first, the others rw1 rows
// of the second, each with matvec_rows_norm's body; only the first part
// writes the updated residual (nm1.hout null).
template <unsigned T0, unsigned T1, bool SCALED>
__global__ __launch_bounds__(1024) void matvec_rows_norm_pair(const uint8_t *__restrict__ w0,
    const uint8_t *__restrict__ w1, const float *__restrict__ x, float *__restrict__ y, int rows0, int rows1,
    int cols, int rw0, int rw1, int wgs0, NormIn nm0, NormIn nm1)
{
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[16][1][64];
    uint8_t *sdig = lds;
    float4 *smeta = (float4 *)(lds + (size_t)128 * (cols / 32));
    const int b = xcd_block(), ngc = cols / kGroupCols;
    if (b < wgs0) {
        const int base = b * rw0, live = rows0 - base < rw0 ? rows0 - base : rw0;
        const int tiles = (rows0 + kTileRows - 1) / kTileRows;
        if (rows0 % kTileRows == 0 || base + live <= kTileRows * (tiles - 1))
            matvec_rows_body<T0, 1, 1, 16, 1, true, false, false, !SCALED, true, false, SCALED>(
                w0, x, nullptr, y, rows0, cols, base, live, 0, ngc, 0, sdig, smeta, red, nm0);
        else
            matvec_rows_body<T0, 1, 1, 16, 1, false, false, false, !SCALED, true, false, SCALED>(
                w0, x, nullptr, y, rows0, cols, base, live, 0, ngc, 0, sdig, smeta, red, nm0);
    } else {
        const int base = (b - wgs0) * rw1, live = rows1 - base < rw1 ? rows1 - base : rw1;
        const int tiles = (rows1 + kTileRows - 1) / kTileRows;
        if (rows1 % kTileRows == 0 || base + live <= kTileRows * (tiles - 1))
            matvec_rows_body<T1, 1, 1, 16, 1, true, false, false, !SCALED, true, false, SCALED>(
                w1, x, nullptr, y + rows0, rows1, cols, base, live, 0, ngc, 0, sdig, smeta, red, nm1);
        else
            matvec_rows_body<T1, 1, 1, 16, 1, false, false, false, !SCALED, true, false, SCALED>(
                w1, x, nullptr, y + rows0, rows1, cols, base, live, 0, ngc, 0, sdig, smeta, red, nm1);
    }
}

size_t matvec_lds(int ccols)
{
    return (size_t)ccols / 32 * (128 + kMetaBytes);
}

// Workgroups of the row-balanced kernel: one per CU.
int cu_count() { return device_cu_count(); }

}  // namespace

int device_cu_count()
{
    static int counts[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!counts[dev]) {
        int n = 0;
        counts[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
            ? n : 256;
    }
    return counts[dev];
}

namespace {

// Row-balanced layout: rows per workgroup (one workgroup per CU).
int rows_per_workgroup(int rows)
{
    const int cus = cu_count();
    return (rows + cus - 1) / cus;
}

// One launch of matvec_rows over chunk groups [g0, g0 + ng).
// ro: the residual epilogue (one chunk, at most 64 rows per workgroup).
template <unsigned T, int VT, int RING, int KS, int P = 1, bool GATED = false>
void launch_rows_kernel(int wgs, size_t lds, hipStream_t s, const uint8_t *w, const float *xc, const float *uc,
    float *y, int rows, int cols, int rw, int g0, int ng, const ResidOut *ro = nullptr)
{
    if constexpr (!GATED && VT * kTileRows / P <= 64) {
        if (ro) {
            if (((ng + KS - 1) / KS + P - 1) / P > RING)
                hipLaunchKernelGGL((matvec_rows_resid<T, VT, RING, KS, P, true>), dim3(wgs), dim3(64 * KS), lds, s, w,
                                   xc, y, rows, cols, rw, *ro);
            else
                hipLaunchKernelGGL((matvec_rows_resid<T, VT, RING, KS, P, false>), dim3(wgs), dim3(64 * KS), lds, s,
                                   w, xc, y, rows, cols, rw, *ro);
            return;
        }
    }
    // A chunk has at most kChunkCols / kGroupCols groups: past KS P RING of
    // them no wavefront needs the refill code.
    if constexpr (KS * P * RING < kChunkCols / kGroupCols) {
        if (((ng + KS - 1) / KS + P - 1) / P > RING) {
            hipLaunchKernelGGL((matvec_rows<T, VT, RING, KS, P, true, GATED>), dim3(wgs), dim3(64 * KS), lds, s, w, xc,
                               uc, y, rows, cols, rw, g0, ng, g0 > 0);
            return;
        }
    }
    hipLaunchKernelGGL((matvec_rows<T, VT, RING, KS, P, false, GATED>), dim3(wgs), dim3(64 * KS), lds, s, w, xc, uc, y,
                       rows, cols, rw, g0, ng, g0 > 0);
}

template <unsigned T, bool GATED = false>
hipError_t launch_rows(const uint8_t *w, const float *x, float *y, int rows, int cols, hipStream_t s,
    const float *up = nullptr, const ResidOut *ro = nullptr)
{
    // Past two tiles per CU (Q6_K only): one workgroup per 32-row tile.
    // Q4_K at 65..80 rows per CU stays row-balanced, three tiles per
    // workgroup (x 4096 columns against matvec_q4k: 16640 rows 9.13 -> 8.65
    // us, 20480 rows 9.60 -> 9.13 us; at 96 rows 10.27 -> 10.34 us, and four
    // tiles spill).
    const int rpw = rows_per_workgroup(rows);
    const int rw = T == Q4_K && !GATED && 2 * rpw <= 5 * kTileRows ? rpw : rpw > 2 * kTileRows ? kTileRows : rpw;
    const int groups = cols / kGroupCols, wgs = (rows + rw - 1) / rw;
    for (int g0 = 0; g0 < groups; g0 += kChunkCols / kGroupCols) {
        const int ng = groups - g0 < kChunkCols / kGroupCols ? groups - g0 : kChunkCols / kGroupCols;
        const float *xc = x + (size_t)g0 * kGroupCols, *uc = GATED ? up + (size_t)g0 * kGroupCols : nullptr;
        const size_t lds = matvec_lds(ng * kGroupCols);
        // Up to 16 rows per CU: two groups per stage (P = 2, 4096 x 11008
        // Q4_0: 7.53 -> 7.07 us), and a second stage where a wavefront has
        // three or more groups (4096 x 14336: Q4_K 8.84 -> 7.92 us, Q6_K
        // 11.19 -> 10.75 us; with one or two it only adds loads). Eight
        // wavefronts with three or four stages measured 5-12 % slower.
        const bool deep = (ng + 15) / 16 >= 3;
        // Q6_K (37-register stages) from 17 rows per CU: one stage per
        // wavefront (two or three stages at eight wavefronts measured
        // 13-17 % slower on 4096 x 14336); two tiles per CU take eight
        // wavefronts of up to 256 registers.
        if constexpr (T == Q6_K) {
            if (rw <= kTileRows / 2 && deep)
                launch_rows_kernel<T, 1, 2, 16, 2, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if (rw <= kTileRows / 2)
                launch_rows_kernel<T, 1, 1, 16, 2, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if (rw <= kTileRows && rpw > 2 * kTileRows)   // one tile per workgroup (128256 x 4096: 84.7 -> 72.5 us)
                launch_rows_kernel<T, 1, 1, 8, 1, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if (rw <= kTileRows)
                launch_rows_kernel<T, 1, 1, 16, 1, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else
                launch_rows_kernel<T, 2, 1, 8, 1, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
        } else {
            // One stage per wavefront from 17 rows per CU on, also where it
            // has several groups (two stages measured 2-10 % slower).
            if (rw <= kTileRows / 2 && deep)
                launch_rows_kernel<T, 1, 2, 16, 2, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if (rw <= kTileRows / 2)
                launch_rows_kernel<T, 1, 1, 16, 2, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if (rw <= kTileRows)
                launch_rows_kernel<T, 1, 1, 16, 1, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if (rw <= 2 * kTileRows)
                launch_rows_kernel<T, 2, 1, 16, 1, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
            else if constexpr (T == Q4_K && !GATED)
                launch_rows_kernel<T, 3, 1, 16, 1, GATED>(wgs, lds, s, w, xc, uc, y, rows, cols, rw, g0, ng, ro);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---- batches of 2..8 ------------------------------------------------------
//
// Same row balance and weight loads as matvec_rows; the A rows of the MFMA
// carry the tokens: A-row 4t + d holds digit d of token t (d = 3 reads a
// zero slot), so D lane l, register 4j + d holds digit d of token 2j + l/32
// for weight row l%32, and each block needs its own epilogue. To keep that
// epilogue short the exponent is shared by a token's 256-column group:
// X = x 2^(21-e) with 2^(e-1) <= max |x| < 2^e over the group (|X| <= 2^21,
// error <= 2^-22 of the group's largest magnitude). Q4_K block scales are
// then small integers that multiply the three digit sums in int32
// (v_mad_i32_i24: |sc sum q a| < 2^22, eight blocks < 2^25), and the float
// work per (row, token) is once per group: d s G - dmin sum_b m_b (sum x)_b
// (the block sums of the quantized x, so the result is the exact dot with
// the quantized x).
// Q4_0 (as 16 (q - 8)) and Q8_0 keep one fma per block with its fp16 scale.
//
// Every wavefront takes 256-column groups w, w + 16, ... and quantizes each
// for 2, 4 or 8 token slots into its own LDS slot; slots past the batch read
// zeros (buffer range check), and A rows past the slots read a zero slot.

// One wavefront's LDS slot for NP token slots: digits [block][token][3
// digits][32 B] (a 96-byte token pitch puts the tokens of one digit word on
// distinct banks), one 32-byte zero slot that the A rows of digit 3 and of
// tokens past NP read for every block, the block sums of the quantized x
// sx[token][block] (Q4_K) and the token scales s[4 (t & 1) + t / 2] (lane
// half h reads tokens h, 2 + h, 4 + h, 6 + h at once).
constexpr int kTokPitch = 96;
constexpr int kRowsWaves = 16;
template <int NP> struct RowsSlot {
    static constexpr int kBlockPitch = NP * kTokPitch;
    static constexpr int kZero = 8 * kBlockPitch;
    static constexpr int kSx = kZero + 32;
    static constexpr int kScale = kSx + NP * 8 * 4;
    static constexpr int kBytes = kScale + 8 * 4;
    static_assert(kBytes % 16 == 0, "16-byte LDS accesses");
};

// Token t of NP is quantized by the L = 64 / NP lanes t L .. t L + L - 1;
// lane j of them takes columns 4 (j % 8) .. +3 of blocks k (L / 8) + j / 8
// (v[k], k < NP): one load reads 16 L consecutive bytes of the token. SUMS:
// also the block sums of the quantized values (Q4_K minimums).
struct NoHook {
    __device__ void operator()(int) const {}
};

// hook(k) runs after block step k (the caller's weight loads, issued
// between the steps).
template <bool SUMS, int NP, typename Hook = NoHook>
__device__ __forceinline__ void quantize_tokens(const float4 (&v)[NP], int lane, uint8_t *__restrict__ slot,
    const Hook &hook = Hook{})
{
    typedef RowsSlot<NP> S;
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    constexpr int L = 64 / NP;
    const int t = lane / L, j = lane % L, p = j >> 3, jj = j & 7;
    // Largest magnitude; the IEEE maximum keeps a NaN, so an inf or NaN
    // anywhere in the group gives a bit pattern of at least 0x7F800000.
    float mf = 0.f;
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        mf = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mf, __builtin_fabsf(v[k].x)), __builtin_fabsf(v[k].y));
        mf = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mf, __builtin_fabsf(v[k].z)), __builtin_fabsf(v[k].w));
    }
    // The token's group maximum: eight lanes, then the mirrored half-row
    // (16), then the other row of the pair (32).
    uint32_t m = max8u(fbits(mf) & 0x7FFFFFFFu);
    if constexpr (L >= 16) m = __builtin_elementwise_max(m, dppu<0x140>(m));
    if constexpr (L >= 32) m = __builtin_elementwise_max(m, (uint32_t)__shfl_xor((int)m, 16, 64));
    const int e = __builtin_amdgcn_frexp_expf(__builtin_bit_cast(float, m));
    const int sh = 21 - e < 127 ? 21 - e : 127;
    const float scale = __builtin_bit_cast(float, (uint32_t)(sh + 127) << 23);
    // As in quantize_group, one fma leaves a = 0x4B400000 + X. Its low half
    // is X mod 2^16: two of them side by side take + 128 in one packed
    // 16-bit add, whose odd bytes are then digit 1 (byte 1 of X + 128); the
    // even bytes before the add are digit 0. Digit 2 is byte 2 of a + K2.
    constexpr float M0 = 12582912.f;
    constexpr uint32_t K2 = 32896u - 0x400000u;
    uint8_t *rec = slot + kTokPitch * t + 4 * jj;
    int part[NP];   // per block: the sum of this lane's four X
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const float4 x = v[k];
        const uint32_t a0 = fbits(__builtin_fmaf(x.x, scale, M0)), a1 = fbits(__builtin_fmaf(x.y, scale, M0));
        const uint32_t a2 = fbits(__builtin_fmaf(x.z, scale, M0)), a3 = fbits(__builtin_fmaf(x.w, scale, M0));
        const uint32_t p01 = __builtin_amdgcn_perm(a1, a0, 0x05040100u), p23 = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
        const uint32_t q01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, p01) + (u16x2){128, 128});
        const uint32_t q23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, p23) + (u16x2){128, 128});
        uint32_t *w = (uint32_t *)(rec + S::kBlockPitch * (k * (L / 8) + p));
        w[0] = __builtin_amdgcn_perm(p23, p01, 0x06040200u);
        w[8] = __builtin_amdgcn_perm(q23, q01, 0x07050301u);
        w[16] = pack_byte(a0 + K2, a1 + K2, a2 + K2, a3 + K2, 2);
        // The four offsets 0x4B400000 wrap away.
        if constexpr (SUMS) part[k] = (int)((a0 + a1) + (a2 + a3) - 4u * 0x4B400000u);
        hook(k);
    }
    if (lane < 2) *(u32x4 *)(slot + S::kZero + 16 * lane) = (u32x4){0u, 0u, 0u, 0u};
    if constexpr (SUMS) {
        // Block sums over the eight lanes of a block (jj = 0..7), reduced
        // and scattered: partners jj and 7 - jj (half-row mirror), then
        // jj ^ 2 and jj ^ 1 (quad swaps); each step keeps half of the
        // blocks while more than one is left, then sums in full. Lane jj
        // ends with part index kf, written by the lanes that own it.
        // |sum| <= 2^26.
        const bool up4 = jj & 4, up2 = jj & 2, up1 = jj & 1;
        int sum, kf;
        bool writer;
        if constexpr (NP == 8) {
            int h4[4], h2[2];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                h4[k] = (up4 ? part[k + 4] : part[k]) +
                        __builtin_amdgcn_update_dpp(0, up4 ? part[k] : part[k + 4], 0x141, 0xF, 0xF, false);
#pragma unroll
            for (int k = 0; k < 2; ++k)
                h2[k] = (up2 ? h4[k + 2] : h4[k]) +
                        __builtin_amdgcn_update_dpp(0, up2 ? h4[k] : h4[k + 2], 0x4E, 0xF, 0xF, false);
            sum = (up1 ? h2[1] : h2[0]) + __builtin_amdgcn_update_dpp(0, up1 ? h2[0] : h2[1], 0xB1, 0xF, 0xF, false);
            kf = jj;
            writer = true;
        } else if constexpr (NP == 4) {
            int h2[2];
#pragma unroll
            for (int k = 0; k < 2; ++k)
                h2[k] = (up4 ? part[k + 2] : part[k]) +
                        __builtin_amdgcn_update_dpp(0, up4 ? part[k] : part[k + 2], 0x141, 0xF, 0xF, false);
            sum = (up2 ? h2[1] : h2[0]) + __builtin_amdgcn_update_dpp(0, up2 ? h2[0] : h2[1], 0x4E, 0xF, 0xF, false);
            sum += __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, false);
            kf = 2 * up4 + up2;
            writer = !up1;
        } else {
            sum = (up4 ? part[1] : part[0]) + __builtin_amdgcn_update_dpp(0, up4 ? part[0] : part[1], 0x141, 0xF, 0xF, false);
            sum += __builtin_amdgcn_update_dpp(0, sum, 0x4E, 0xF, 0xF, false);
            sum += __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, false);
            kf = up4;
            writer = !up2 && !up1;
        }
        if (writer) ((float *)(slot + S::kSx))[8 * t + kf * (L / 8) + p] = __builtin_amdgcn_ldexpf((float)sum, -sh);
    }
    // s = 2^(e-21); NaN when the group holds an inf or NaN (then every
    // output of the token is NaN).
    if (j == 0)
        ((float *)(slot + S::kScale))[4 * (t & 1) + (t >> 1)] =
            m < 0x7F800000u ? __builtin_amdgcn_ldexpf(1.f, -sh) : __builtin_nanf("");
}

// B operand of block k: Q4_K nibbles as they are (0..15), Q4_0 as
// 16 (q - 8), Q8_0 bytes as they are.
template <unsigned T>
__device__ __forceinline__ i32x4 block_b_tokens(const MvStage<T> &w, int k)
{
    if constexpr (T == Q8_0) {
        return as_i32x4(w.q[k]);
    } else if constexpr (T == Q4_K) {
        const u32x4 q = w.q[k >> 1];
        return as_i32x4((k & 1) ? (q >> 4) & 0x0F0F0F0Fu : q & 0x0F0F0F0Fu);
    } else {
        const u32x4 q = w.q[k >> 1];
        return as_i32x4(((k & 1) ? q & 0xF0F0F0F0u : (q << 4) & 0xF0F0F0F0u) ^ 0x80808080u);
    }
}

// Accumulators per lane and virtual tile: tokens 2j + h, or for Q6_K (each
// lane half owns its own 16-column scale groups) every token.
template <unsigned T, int NP> constexpr int kTokAcc = T == Q6_K ? NP : NP / 2;

// The group's dots for VT virtual tiles and NP token slots: y[v][j] += this
// group's share of token 2j + h (j < NP / 2; Q6_K: token j), row l%32 of
// tile v. This lane's A operand of block b sits at aoff + b astride in the
// slot (Q6_K: see below).
template <unsigned T, int VT, int NP>
__device__ __forceinline__ void group_dots_tokens(float (&y)[VT][(kTokAcc<T, NP>)], const MvStage<T> (&w)[VT],
    const uint8_t *__restrict__ slot, int aoff, int astride, int h)
{
    typedef RowsSlot<NP> S;
    constexpr int J = NP / 2;
    const float4 sv = *(const float4 *)(slot + S::kScale + 16 * h);
    const float s4[4] = {sv.x, sv.y, sv.z, sv.w};
    if constexpr (T == Q6_K) {
        // MFMA block j = 4c + jp: lane half h holds columns 16 (jp / 2) .. +15
        // of x-block 4c + 2 (jp % 2) + h with scale sc[8c + 2q + jp / 2],
        // q = 2 (jp % 2) + h. A-row 8t' + 4h' + d: digit d of token t' + 4th
        // in K-half h' only, so D lane half h holds its own half's sums of
        // four tokens per MFMA (registers 4t' .. 4t'+2). aoff: this lane's
        // A row in x-block h of the group for token half 0; bit th of
        // astride: the row is live for token half th (else the zero slot).
        constexpr int TH = NP > 4 ? 2 : 1, TT = NP < 4 ? NP : 4;
        const float4 s0 = *(const float4 *)(slot + S::kScale), s1 = *(const float4 *)(slot + S::kScale + 16);
        const float sraw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};   // token t at 4 (t & 1) + t / 2
        int acc[VT][TH][TT][3];
#pragma unroll
        for (int v = 0; v < VT; ++v)
#pragma unroll
            for (int th = 0; th < TH; ++th)
#pragma unroll
                for (int t = 0; t < TT; ++t) acc[v][th][t][0] = acc[v][th][t][1] = acc[v][th][t][2] = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = j >> 2, jp = j & 3, q = 2 * (jp & 1) + h;
            const int uoff = S::kBlockPitch * (4 * c + 2 * (jp & 1)) + 16 * (jp >> 1);
#pragma unroll
            for (int th = 0; th < TH; ++th) {
                const int off = (astride >> th) & 1 ? aoff + 4 * kTokPitch * th + uoff : S::kZero;
                const i32x4 a = *(const i32x4 *)(slot + off);
#pragma unroll
                for (int v = 0; v < VT; ++v) {
                    const i32x16 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, block_b6(w[v], j, h), (i32x16){}, 0, 0, 0);
                    const int sc = (int)__builtin_amdgcn_sbfe((int)w[v].sc[2 * c + (jp >> 1)], 8 * q, 8);
                    // |D| < 2^18, |sc| <= 128: 24-bit multiply-adds, eight
                    // blocks below 2^28.
#pragma unroll
                    for (int t = 0; t < TT; ++t)
#pragma unroll
                        for (int d = 0; d < 3; ++d) {
                            acc[v][th][t][d] += ((D[4 * t + d] << 8) >> 8) * sc;
                            asm("" : "+v"(acc[v][th][t][d]));
                        }
                }
                // One MFMA result live at a time (register budget).
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int v = 0; v < VT; ++v) {
            const float d4 = 0.25f * f16_to_f32(w[v].d & 0xFFFFu);   // the weights entered as 4 (q6 - 32)
#pragma unroll
            for (int th = 0; th < TH; ++th)
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const int tok = 4 * th + t;
                    const float G = __builtin_fmaf((float)acc[v][th][t][2], 65536.f,
                                                   __builtin_fmaf((float)acc[v][th][t][1], 256.f, (float)acc[v][th][t][0]));
                    y[v][tok] = __builtin_fmaf(sraw[4 * (tok & 1) + (tok >> 1)] * d4, G, y[v][tok]);
                }
        }
    } else if constexpr (T == Q4_K) {
        // The minimum term sum_b m_b (sum x)_b first: it needs only the scale
        // words (each tile's first load) and the block sums in LDS, so it runs
        // while the quants stream in.
        float mterm[VT][J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float4 xa = *(const float4 *)(slot + S::kSx + 32 * (2 * j + h));
            const float4 xb = *(const float4 *)(slot + S::kSx + 32 * (2 * j + h) + 16);
            const float sx[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int v = 0; v < VT; ++v) {
                float m = 0.f;
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    m = __builtin_fmaf((float)__builtin_amdgcn_ubfe(w[v].sl[b >> 1], 12 * (b & 1) + 6, 6), sx[b], m);
                mterm[v][j] = m;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // Then block by block, each block's two MFMAs (one per tile) and their
        // scale multiply-adds interleaved: the loads come field by field, so
        // block pair p waits only for quant word p of each tile.
        int acc[VT][J][3];
#pragma unroll
        for (int v = 0; v < VT; ++v)
#pragma unroll
            for (int j = 0; j < J; ++j) acc[v][j][0] = acc[v][j][1] = acc[v][j][2] = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const i32x4 a = *(const i32x4 *)(slot + aoff + astride * b);
#pragma unroll
            for (int v = 0; v < VT; ++v) {
                const i32x16 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, block_b_tokens<T>(w[v], b), (i32x16){}, 0, 0, 0);
                const int sc = (int)__builtin_amdgcn_ubfe(w[v].sl[b >> 1], 12 * (b & 1), 6);
                // |D| < 2^16: the 24-bit multiply-add takes it whole. The
                // empty asm keeps each sum a chain of multiply-adds (not
                // products summed in threes); it names only the
                // accumulators, never an MFMA result.
#pragma unroll
                for (int j = 0; j < J; ++j)
#pragma unroll
                    for (int d = 0; d < 3; ++d) {
                        acc[v][j][d] += ((D[4 * j + d] << 8) >> 8) * sc;
                        asm("" : "+v"(acc[v][j][d]));
                    }
            }
        }
#pragma unroll
        for (int v = 0; v < VT; ++v) {
            const u32x4 sl = w[v].sl;   // byte 3 of the four words: d, dmin
            const uint32_t dd = (sl.x >> 24) | ((sl.y >> 24) << 8) | ((sl.z >> 24) << 16) | ((sl.w >> 24) << 24);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const float G = __builtin_fmaf((float)acc[v][j][2], 65536.f,
                                               __builtin_fmaf((float)acc[v][j][1], 256.f, (float)acc[v][j][0]));
                y[v][j] = __builtin_fmaf(-f16_to_f32(dd >> 16), mterm[v][j],
                                         __builtin_fmaf(s4[j] * f16_to_f32(dd & 0xFFFFu), G, y[v][j]));
            }
        }
    } else {
        // Block by block over the tiles, as for Q4_K.
        float acc[VT][J];
#pragma unroll
        for (int v = 0; v < VT; ++v)
#pragma unroll
            for (int j = 0; j < J; ++j) acc[v][j] = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const i32x4 a = *(const i32x4 *)(slot + aoff + astride * b);
#pragma unroll
            for (int v = 0; v < VT; ++v) {
                const i32x16 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, block_b_tokens<T>(w[v], b), (i32x16){}, 0, 0, 0);
                const float db = f16_to_f32((w[v].d[b >> 1] >> (16 * (b & 1))) & 0xFFFFu);
                // Sums reach 2^34: the top digit joins in float.
#pragma unroll
                for (int j = 0; j < J; ++j)
                    acc[v][j] = __builtin_fmaf(__builtin_fmaf((float)D[4 * j + 2], 65536.f,
                                                              (float)(D[4 * j + 1] * 256 + D[4 * j])), db, acc[v][j]);
            }
        }
        constexpr float kWeightFactor = T == Q4_0 ? 0.0625f : 1.f;
#pragma unroll
        for (int v = 0; v < VT; ++v)
#pragma unroll
            for (int j = 0; j < J; ++j) y[v][j] = __builtin_fmaf(s4[j] * kWeightFactor, acc[v][j], y[v][j]);
    }
}

template <unsigned T, int VT, int NP, bool LOOP, int KS, bool FULL>
__device__ __forceinline__ void smalln_rows_body(const uint8_t *__restrict__ w, const float *__restrict__ x,
    float *__restrict__ y, int rows, int cols, int n, int base, int live, uint8_t *lds)
{
    typedef RowsSlot<NP> S;
    constexpr int J = kTokAcc<T, NP>, L = 64 / NP;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    const int groups = cols / kGroupCols;
    const size_t row_bytes = tiled_row_bytes<T>(cols);
    const int tiles = (rows + kTileRows - 1) / kTileRows, rlast = rows - kTileRows * (tiles - 1);
    const __amdgpu_buffer_rsrc_t wb = buffer_of(w, (uint32_t)((size_t)rows * row_bytes));
    const __amdgpu_buffer_rsrc_t xb = buffer_of(x, (uint32_t)n * (uint32_t)cols * 4u);
    float acc[VT][J];
#pragma unroll
    for (int v = 0; v < VT; ++v)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[v][j] = 0.f;
    // x first, then the weights of every virtual tile (rows past this
    // workgroup's repeat its last row). A wavefront's loads complete in
    // order, so its quantization never waits for its own weights; for Q4_K
    // and Q8_0 a barrier also puts every wavefront's x ahead of all weights
    // (see below). Tokens past n read zeros (buffer range check).
    // This wave's groups: wave + 16 k for k < ns (one slot, reused).
    const int ns = wave < groups ? (groups - wave + KS - 1) / KS : 0;
    const int vx = 4 * (lane / L) * cols + 16 * (lane % L);
    float4 px[NP];
    auto load_x = [&](int g) {
#pragma unroll
        for (int k = 0; k < NP; ++k) px[k] = __builtin_bit_cast(float4, bload16<false>(xb, vx, 1024 * g + 16 * L * k));
    };
    if (ns > 0) load_x(wave);
    // Q4_K and Q8_0: the barrier puts every wavefront's x ahead of all
    // weights (Q8_0 4096 x 4096 N=8 6.9 -> 6.4 us with it); Q6_K and Q4_0
    // issue their weights at once (Q6_K 4096 x 14336 24.4 -> 23.95 us,
    // 4096 x 4096 9.0 -> 8.45 us; Q4_0 11008 x 4096 9.37 -> 9.0 us without it).
    if constexpr (T == Q4_K || T == Q8_0) issue_barrier();
    else asm volatile("" ::: "memory");
    if (ns > 0) {
        uint8_t *slot = lds + S::kBytes * wave;
        // A-row 4t + d: digit d < 3 of token t < NP, or the zero slot.
        int aoff, astride;
        if constexpr (T == Q6_K) {
            // A-row 8t' + 4h' + d: live in K-half h' = h for digit d < 3 of
            // tokens t' (bit 0) and t' + 4 (bit 1) below NP.
            const int tq = (lane & 31) >> 3, hq = ((lane & 31) >> 2) & 1, ad = lane & 3;
            const bool row = hq == h && ad < 3;
            aoff = S::kBlockPitch * h + kTokPitch * tq + 32 * ad;
            astride = (row && tq < NP ? 1 : 0) | (row && tq + 4 < NP ? 2 : 0);
        } else {
            // A-row 4t + d: digit d < 3 of token t < NP, or the zero slot.
            const int at = (lane & 31) >> 2, ad = lane & 3;
            const bool digit = at < NP && ad < 3;
            aoff = (digit ? kTokPitch * at + 32 * ad : S::kZero) + 16 * h;
            astride = digit ? S::kBlockPitch : 0;
        }
        MvStage<T> st[VT];
        if constexpr (!LOOP) {
            // One group per wavefront (cols <= 4096); the dots take block b
            // of every tile together, so the tiles load field by field.
            int vq[VT], vs[VT], vd[VT], R[VT];
#pragma unroll
            for (int v = 0; v < VT; ++v) {
                const int row = base + (kTileRows * v + (lane & 31) < live ? kTileRows * v + (lane & 31) : live - 1);
                const int t = row / kTileRows, r = row - kTileRows * t;
                R[v] = t == tiles - 1 ? rlast : kTileRows;
                const int tb = (int)((size_t)kTileRows * t * row_bytes);
                vq[v] = tb + 16 * R[v] * h + 16 * r;
                vs[v] = tb + 16 * r;
                vd[v] = tb + 2 * r;
            }
            if constexpr (T == Q4_K && NP == 8 && VT == 2) {
                // The scale words, then quant word k/2 of tile k%2 after block
                // step k of the quantization: a wave's loads wait in the CU's
                // queue (its sixteen waves request 160 KiB of weights), and a
                // wave stalled on a load's issue cannot quantize behind it;
                // interleaved, it quantizes while its later loads wait
                // (14336 x 4096 N=8 10.0-10.5 -> 9.8-9.9 us).
#pragma unroll
                for (int v = 0; v < VT; ++v) load_field<T, FULL>(st[v], wb, vq[v], vs[v], R[v], wave, vd[v], groups, 0);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                auto hook = [&](int k) {
                    __builtin_amdgcn_sched_barrier(0);
                    load_field<T, FULL>(st[k & 1], wb, vq[k & 1], vs[k & 1], R[k & 1], wave, vd[k & 1], groups,
                                        (k >> 1) + 1);
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                };
                quantize_tokens<true, NP>(px, lane, slot, hook);
            } else {
                load_rows_fields<T, FULL, VT>(st, wb, vq, vs, R, wave, vd, groups);
                quantize_tokens<T == Q4_K, NP>(px, lane, slot);
            }
            // Each wave reads back only its own slot.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            group_dots_tokens<T, VT, NP>(acc, st, slot, aoff, astride, h);
        } else {
            static_assert(VT == 1, "one virtual tile when looping over groups");
            // Several groups per wavefront (one virtual tile): after each
            // group's dots the next group's x, then its weights (no prefetch
            // across the dots: x and a stage together would not fit the 128
            // registers of sixteen wavefronts).
            const int row = base + ((lane & 31) < live ? (lane & 31) : live - 1);
            const int t = row / kTileRows, r = row - kTileRows * t;
            const int R = t == tiles - 1 ? rlast : kTileRows;
            const int tb = (int)((size_t)kTileRows * t * row_bytes);
            const int vq = tb + 16 * R * h + 16 * r, vs = tb + 16 * r, vd = tb + 2 * r;
            load_rows<T, FULL>(st[0], wb, vq, vs, R, wave, vd, groups);
            for (int k = 0; k < ns; ++k) {
                if (k > 0) {
                    load_x(wave + KS * k);
                    load_rows<T, FULL>(st[0], wb, vq, vs, R, wave + KS * k, vd, groups);
                }
                quantize_tokens<T == Q4_K, NP>(px, lane, slot);
                // Each wave reads back only its own slot (and rewrites it
                // only after this group's dots: a wave's LDS accesses
                // complete in order).
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                group_dots_tokens<T, VT, NP>(acc, st, slot, aoff, astride, h);
                // Keeps the next group's loads after these dots (their
                // registers and those of the dots would not fit together).
                asm volatile("" ::: "memory");
            }
        }
    }

    // Wavefronts' shares, in a fixed order (the slots are reused).
    __syncthreads();
    float *red = (float *)lds;   // [wave][VT][J][64]
#pragma unroll
    for (int v = 0; v < VT; ++v)
#pragma unroll
        for (int j = 0; j < J; ++j) red[((wave * VT + v) * J + j) * 64 + lane] = acc[v][j];
    __syncthreads();
    const int i = threadIdx.x;
    if (i >= VT * 256) return;
    const int v = i >> 8, t = (i >> 5) & 7, r = i & 31;
    if (t >= n || kTileRows * v + r >= live) return;
    // Every wavefront wrote its share (zero for a wavefront without groups).
    // All KS partials are read before the first add: one LDS round trip, not
    // one per partial.
    float s = 0.f;
    if constexpr (T == Q6_K) {
        // Every lane holds every token: its lane half's columns.
        float p[2 * KS];
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            p[2 * q] = red[((q * VT + v) * J + t) * 64 + r];
            p[2 * q + 1] = red[((q * VT + v) * J + t) * 64 + r + 32];
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int q = 0; q < KS; ++q) s += p[2 * q] + p[2 * q + 1];
    } else {
        const int ln = r + 32 * (t & 1);
        float p[KS];
#pragma unroll
        for (int q = 0; q < KS; ++q) p[q] = red[((q * VT + v) * J + (t >> 1)) * 64 + ln];
        asm volatile("" ::: "memory");
#pragma unroll
        for (int q = 0; q < KS; ++q) s += p[q];
    }
    y[(size_t)t * rows + base + kTileRows * v + r] = s;
}

template <unsigned T, int VT, int NP, bool LOOP, int KS = kRowsWaves>
__global__ __launch_bounds__(64 * KS) void smalln_rows(const uint8_t *__restrict__ w,
    const float *__restrict__ x, float *__restrict__ y, int rows, int cols, int n, int rw)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int base = xcd_block() * rw, live = rows - base < rw ? rows - base : rw;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    if (rows % kTileRows == 0 || base + live <= kTileRows * (tiles - 1))
        smalln_rows_body<T, VT, NP, LOOP, KS, true>(w, x, y, rows, cols, n, base, live, lds);
    else
        smalln_rows_body<T, VT, NP, LOOP, KS, false>(w, x, y, rows, cols, n, base, live, lds);
}

// LDS of one smalln_rows workgroup: the wavefront slots, or the reduction
// array [wave][VT][NP or NP / 2][64] floats that reuses them, whichever is
// larger.
template <int VT, int NP, int KS = kRowsWaves>
constexpr size_t rows_lds()
{
    const size_t slots = (size_t)RowsSlot<NP>::kBytes * KS;
    const size_t red = (size_t)KS * VT * NP * 64 * 4;
    return slots > red ? slots : red;
}

template <unsigned T, int NP>
hipError_t launch_tokens_np(const uint8_t *w, const float *x, float *y, int rows, int cols, int n, hipStream_t s)
{
    // Past two tiles per CU (Q6_K: past one), one workgroup per 32-row tile
    // (each quantizes x again; Q6_K 128256 x 4096 N=2 98 -> 83 us, Q4_K
    // 57344 x 4096 N=2 33 -> 24 us against the tile kernel).
    const int rpw = rows_per_workgroup(rows);
    const int rw = (T == Q6_K && rpw > kTileRows) || rpw > 2 * kTileRows ? kTileRows : rpw, wgs = (rows + rw - 1) / rw;
    if constexpr (T == Q6_K && NP == 8) {
        if (cols > kRowsWaves * kGroupCols) {
            // Wide Q6_K rows at eight slots: eight wavefronts of up to 256
            // registers (sixteen of 128 would spill).
            hipLaunchKernelGGL((smalln_rows<T, 1, NP, true, 8>), dim3(wgs), dim3(512), (rows_lds<1, NP, 8>()), s, w, x,
                               y, rows, cols, n, rw);
            return hipGetLastError();
        }
    }
    if (cols > kRowsWaves * kGroupCols)   // several groups per wavefront (one tile per CU)
        hipLaunchKernelGGL((smalln_rows<T, 1, NP, !(T == Q6_K && NP == 8)>), dim3(wgs), dim3(64 * kRowsWaves), (rows_lds<1, NP>()), s, w,
                           x, y, rows, cols, n, rw);
    else if (T == Q6_K || rw <= kTileRows)
        hipLaunchKernelGGL((smalln_rows<T, 1, NP, false>), dim3(wgs), dim3(64 * kRowsWaves), (rows_lds<1, NP>()), s, w,
                           x, y, rows, cols, n, rw);
    else if constexpr (T != Q6_K)
        hipLaunchKernelGGL((smalln_rows<T, 2, NP, false>), dim3(wgs), dim3(64 * kRowsWaves), (rows_lds<2, NP>()), s, w,
                           x, y, rows, cols, n, rw);
    return hipGetLastError();
}

// Token slots: 2, 4 or 8 (a token's quantization takes 64 / slots lanes).
template <unsigned T>
hipError_t launch_tokens(const uint8_t *w, const float *x, float *y, int rows, int cols, int n, hipStream_t s)
{
    if (n <= 2) return launch_tokens_np<T, 2>(w, x, y, rows, cols, n, s);
    if (n <= 4) return launch_tokens_np<T, 4>(w, x, y, rows, cols, n, s);
    return launch_tokens_np<T, 8>(w, x, y, rows, cols, n, s);
}

}  // namespace

// Batches of 2..8 on the row-balanced kernel: Q4_K, Q4_0, Q8_0 and Q6_K rows
// in whole 256-column groups. Rows of up to 4096 columns take any row count
// (past two tiles per CU, one for Q6_K: one workgroup per tile); wider rows,
// where a wavefront has several groups, up to one tile per CU.
bool smalln_rows_supported(unsigned type, int rows, int cols, int batch)
{
    if (type != Q4_K && type != Q4_0 && type != Q8_0 && type != Q6_K) return false;
    if (batch < 2 || batch > 8 || cols % kGroupCols) return false;
    // Rows of several 256-column groups per wavefront loop over the groups
    // with one virtual tile per workgroup (two would spill); past 32 rows per
    // CU such matrices run faster on the tile kernel.
    const bool wide = cols > kRowsWaves * kGroupCols;
    return !wide || rows_per_workgroup(rows) <= kTileRows;
}

hipError_t launch_smalln_rows(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    int batch, hipStream_t s)
{
    if (!smalln_rows_supported(type, rows, cols, batch)) return hipErrorInvalidValue;
    if (type == Q4_K) return launch_tokens<Q4_K>(w, x, y, rows, cols, batch, s);
    if (type == Q4_0) return launch_tokens<Q4_0>(w, x, y, rows, cols, batch, s);
    if (type == Q6_K) return launch_tokens<Q6_K>(w, x, y, rows, cols, batch, s);
    return launch_tokens<Q8_0>(w, x, y, rows, cols, batch, s);
}

// The row-balanced kernel takes up to two 32-row tiles per CU (Q4_K: up to
// 80 rows) and whole 256-column groups (Q8_0/Q4_0: rows of complete groups);
// beyond that, Q4_K and Q6_K run one workgroup per tile (matvec_q4k, or the
// row kernel over single tiles).
bool matvec_supported(unsigned type, int rows, int cols)
{
    if (type != Q4_K && type != Q4_0 && type != Q8_0 && type != Q6_K) return false;
    if (cols % kGroupCols) return false;
    if (type == Q4_K || type == Q6_K) return true;
    return rows_per_workgroup(rows) <= 2 * kTileRows;
}

const char *matvec_kernel(unsigned type, int rows, int cols)
{
    if (!matvec_supported(type, rows, cols)) return nullptr;
    if (type == Q4_K && 2 * rows_per_workgroup(rows) > 5 * kTileRows) return "matvec_q4k";
    return "matvec_rows";
}

hipError_t launch_matvec(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols,
    hipStream_t s)
{
    if (!matvec_supported(type, rows, cols)) return hipErrorInvalidValue;
    if (type == Q4_0) return launch_rows<Q4_0>(w, x, y, rows, cols, s);
    if (type == Q8_0) return launch_rows<Q8_0>(w, x, y, rows, cols, s);
    if (type == Q6_K) return launch_rows<Q6_K>(w, x, y, rows, cols, s);
    if (2 * rows_per_workgroup(rows) <= 5 * kTileRows) return launch_rows<Q4_K>(w, x, y, rows, cols, s);
    // More than 80 rows per CU: one workgroup per 32-row tile, eight
    // wavefronts, two groups each in flight.
    const int groups = cols / kGroupCols;
    const unsigned tiles = (unsigned)((rows + kTileRows - 1) / kTileRows);
    for (int g0 = 0; g0 < groups; g0 += kChunkCols / kGroupCols) {
        const int ng = groups - g0 < kChunkCols / kGroupCols ? groups - g0 : kChunkCols / kGroupCols;
        hipLaunchKernelGGL((matvec_q4k<8, 2>), dim3(tiles), dim3(512), matvec_lds(ng * kGroupCols), s, w,
                           x + (size_t)g0 * kGroupCols, y, rows, cols, g0, ng, g0 > 0, NormIn{});
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

bool matvec_gated_supported(unsigned type, int rows, int cols)
{
    return matvec_supported(type, rows, cols) && (type != Q4_K || rows_per_workgroup(rows) <= 2 * kTileRows);
}

bool matvec_normed_supported(unsigned type, int rows, int cols)
{
    return matvec_supported(type, rows, cols) && cols <= 16 * kGroupCols && rows_per_workgroup(rows) <= kTileRows;
}

bool matvec_normed_rope_supported(unsigned type, int rows, int cols)
{
    return matvec_normed_supported(type, rows, cols) && rows % 2 == 0 && rows_per_workgroup(rows) % 2 == 0;
}

hipError_t launch_matvec_normed_rope(unsigned type, const uint8_t *w, const float *x, const float *r, const float *g,
    float *hout, float eps, float *y, int rows, int cols, int row0, const int *positions, const float *freq,
    float *keys, float *values, int qd, int kvd, int width, int capacity, hipStream_t s)
{
    if (!matvec_normed_rope_supported(type, rows, cols) || row0 % 2) return hipErrorInvalidValue;
    const int rw = rows_per_workgroup(rows), wgs = (rows + rw - 1) / rw;
    NormIn nm{r, g, hout, eps, positions, freq, keys, values, qd, kvd, width, capacity};
    nm.row0 = row0;
    const size_t lds = matvec_lds(cols);
#define FY_NORMED(TT) \
    hipLaunchKernelGGL((matvec_rows_norm<TT, true>), dim3(wgs), dim3(1024), lds, s, w, x, y, rows, cols, rw, nm)
    switch (type) {
    case Q4_K: FY_NORMED(Q4_K); break;
    case Q6_K: FY_NORMED(Q6_K); break;
    case Q8_0: FY_NORMED(Q8_0); break;
    case Q4_0: FY_NORMED(Q4_0); break;
    default: return hipErrorInvalidValue;
    }
#undef FY_NORMED
    return hipGetLastError();
}

// The workgroup split of a two-part rotary product: the CUs shared by the
// parts' bytes, rows per workgroup even and at most one tile.
struct RopePair {
    int rw0, rw1, wgs0, wgs1;
};

bool rope_pair_split(unsigned type0, int rows0, unsigned type1, int rows1, int cols, RopePair *out)
{
    if (type0 != Q4_K || type1 != Q6_K || rows0 <= 0 || rows1 <= 0 || rows0 % 2 || rows1 % 2 ||
        cols % kGroupCols || cols > 16 * kGroupCols)
        return false;
    const int cus = cu_count();
    const double b0 = (double)rows0 * tiled_row_bytes<Q4_K>(cols), b1 = (double)rows1 * tiled_row_bytes<Q6_K>(cols);
    int wgs1 = (int)(cus * b1 / (b0 + b1) + 0.5);
    wgs1 = wgs1 < 1 ? 1 : wgs1 > cus - 1 ? cus - 1 : wgs1;
    RopePair p;
    p.rw1 = (rows1 + wgs1 - 1) / wgs1;
    p.rw1 += p.rw1 % 2;
    p.wgs1 = (rows1 + p.rw1 - 1) / p.rw1;
    const int wgs0 = cus - p.wgs1;
    if (wgs0 < 1) return false;
    p.rw0 = (rows0 + wgs0 - 1) / wgs0;
    p.rw0 += p.rw0 % 2;
    p.wgs0 = (rows0 + p.rw0 - 1) / p.rw0;
    if (p.rw0 > kTileRows || p.rw1 > kTileRows) return false;
    *out = p;
    return true;
}

bool matvec_rope_pair_supported(unsigned type0, int rows0, unsigned type1, int rows1, int cols)
{
    RopePair p;
    return rope_pair_split(type0, rows0, type1, rows1, cols, &p);
}

hipError_t launch_matvec_rope_pair(unsigned type0, const uint8_t *w0, int rows0, unsigned type1, const uint8_t *w1,
    int rows1, int cols, const float *x, const float *r, const float *g, float *hout, const double *parts, float eps,
    float *y, const int *positions, const float *freq, float *keys, float *values, int qd, int kvd, int width,
    int capacity, hipStream_t s)
{
    RopePair p;
    if (!rope_pair_split(type0, rows0, type1, rows1, cols, &p)) return hipErrorInvalidValue;
    NormIn nm0{r, g, hout, eps, positions, freq, keys, values, qd, kvd, width, capacity};
    nm0.parts = parts;
    NormIn nm1 = nm0;
    nm1.hout = nullptr;
    nm1.row0 = rows0;
    const dim3 grid((unsigned)(p.wgs0 + p.wgs1));
    if (parts)
        hipLaunchKernelGGL((matvec_rows_norm_pair<Q4_K, Q6_K, true>), grid, dim3(1024), matvec_lds(cols), s, w0, w1,
                           x, y, rows0, rows1, cols, p.rw0, p.rw1, p.wgs0, nm0, nm1);
    else
        hipLaunchKernelGGL((matvec_rows_norm_pair<Q4_K, Q6_K, false>), grid, dim3(1024), matvec_lds(cols), s, w0, w1,
                           x, y, rows0, rows1, cols, p.rw0, p.rw1, p.wgs0, nm0, nm1);
    return hipGetLastError();
}

hipError_t launch_matvec_scaled_rope(unsigned type, const uint8_t *w, const float *hn, const double *parts, float eps,
    float *y, int rows, int cols, int row0, const int *positions, const float *freq, float *keys, float *values,
    int qd, int kvd, int width, int capacity, hipStream_t s)
{
    if (!matvec_normed_rope_supported(type, rows, cols) || row0 % 2) return hipErrorInvalidValue;
    const int rw = rows_per_workgroup(rows), wgs = (rows + rw - 1) / rw;
    NormIn nm{nullptr, nullptr, nullptr, eps, positions, freq, keys, values, qd, kvd, width, capacity};
    nm.parts = parts;
    nm.row0 = row0;
    const size_t lds = matvec_lds(cols);
#define FY_SCALED(TT) \
    hipLaunchKernelGGL((matvec_rows_norm<TT, true, true>), dim3(wgs), dim3(1024), lds, s, w, hn, y, rows, cols, rw, nm)
    switch (type) {
    case Q4_K: FY_SCALED(Q4_K); break;
    case Q6_K: FY_SCALED(Q6_K); break;
    case Q8_0: FY_SCALED(Q8_0); break;
    case Q4_0: FY_SCALED(Q4_0); break;
    default: return hipErrorInvalidValue;
    }
#undef FY_SCALED
    return hipGetLastError();
}

hipError_t launch_matvec_normed(unsigned type, const uint8_t *w, const float *x, const float *r, const float *g,
    float *hout, float eps, float *y, int rows, int cols, hipStream_t s)
{
    if (!matvec_normed_supported(type, rows, cols)) return hipErrorInvalidValue;
    const int rw = rows_per_workgroup(rows), wgs = (rows + rw - 1) / rw;
    const NormIn nm{r, g, hout, eps, nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0};
    const size_t lds = matvec_lds(cols);
#define FY_NORMED(TT) hipLaunchKernelGGL(matvec_rows_norm<TT>, dim3(wgs), dim3(1024), lds, s, w, x, y, rows, cols, rw, nm)
    switch (type) {
    case Q4_K: FY_NORMED(Q4_K); break;
    case Q6_K: FY_NORMED(Q6_K); break;
    case Q8_0: FY_NORMED(Q8_0); break;
    case Q4_0: FY_NORMED(Q4_0); break;
    default: return hipErrorInvalidValue;
    }
#undef FY_NORMED
    return hipGetLastError();
}

bool matvec_swiglu_supported(unsigned type, int rows, int cols)
{
    return type == Q4_K && rows % (2 * 16) == 0 && cols % kGroupCols == 0 && cols <= kChunkCols &&
           rows_per_workgroup(rows) > kTileRows;
}

hipError_t launch_matvec_swiglu(unsigned type, const uint8_t *w, const float *x, float *hidden, int rows, int cols,
    hipStream_t s)
{
    if (!matvec_swiglu_supported(type, rows, cols)) return hipErrorInvalidValue;
    const int groups = cols / kGroupCols;
    hipLaunchKernelGGL((matvec_q4k<8, 2, kGateSilu>), dim3((unsigned)(rows / kTileRows)), dim3(512),
                       matvec_lds(groups * kGroupCols), s, w, x, hidden, rows, cols, 0, groups, 0, NormIn{});
    return hipGetLastError();
}

hipError_t launch_matvec_geglu(unsigned type, const uint8_t *w, const float *x, float *hidden, int rows, int cols,
    hipStream_t s)
{
    if (!matvec_swiglu_supported(type, rows, cols)) return hipErrorInvalidValue;
    const int groups = cols / kGroupCols;
    hipLaunchKernelGGL((matvec_q4k<8, 2, kGateGelu>), dim3((unsigned)(rows / kTileRows)), dim3(512),
                       matvec_lds(groups * kGroupCols), s, w, x, hidden, rows, cols, 0, groups, 0, NormIn{});
    return hipGetLastError();
}

bool matvec_swiglu_scaled_supported(unsigned type, int rows, int cols)
{
    return matvec_swiglu_supported(type, rows, cols);
}

hipError_t launch_matvec_swiglu_scaled(unsigned type, const uint8_t *w, const float *hn, const double *parts,
    float eps, float *hidden, int rows, int cols, hipStream_t s)
{
    if (!matvec_swiglu_scaled_supported(type, rows, cols)) return hipErrorInvalidValue;
    NormIn nm{};
    nm.eps = eps;
    nm.parts = parts;
    const int groups = cols / kGroupCols;
    hipLaunchKernelGGL((matvec_q4k<8, 2, kGateSilu, true>), dim3((unsigned)(rows / kTileRows)), dim3(512),
                       matvec_lds(groups * kGroupCols), s, w, hn, hidden, rows, cols, 0, groups, 0, nm);
    return hipGetLastError();
}

// The residual epilogue: the row-balanced kernel at up to 64 rows per
// workgroup (wave 0 holds every row), one column chunk, at most kNormParts
// workgroups.
bool matvec_residual_supported(unsigned type, int rows, int cols)
{
    return matvec_supported(type, rows, cols) && cols <= kChunkCols && rows_per_workgroup(rows) <= 2 * kTileRows &&
           cu_count() <= kNormParts;
}

hipError_t launch_matvec_residual(unsigned type, const uint8_t *w, const float *x, float *res, const float *g,
    float *hn, double *parts, int rows, int cols, hipStream_t s)
{
    if (!matvec_residual_supported(type, rows, cols)) return hipErrorInvalidValue;
    const ResidOut ro{g, hn, parts, 0};
    switch (type) {
    case Q4_K: return launch_rows<Q4_K>(w, x, res, rows, cols, s, nullptr, &ro);
    case Q6_K: return launch_rows<Q6_K>(w, x, res, rows, cols, s, nullptr, &ro);
    case Q8_0: return launch_rows<Q8_0>(w, x, res, rows, cols, s, nullptr, &ro);
    case Q4_0: return launch_rows<Q4_0>(w, x, res, rows, cols, s, nullptr, &ro);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec_gated(unsigned type, const uint8_t *w, const float *gate, const float *up, float *y,
    int rows, int cols, hipStream_t s)
{
    if (!matvec_gated_supported(type, rows, cols)) return hipErrorInvalidValue;
    if (type == Q4_0) return launch_rows<Q4_0, true>(w, gate, y, rows, cols, s, up);
    if (type == Q8_0) return launch_rows<Q8_0, true>(w, gate, y, rows, cols, s, up);
    if (type == Q6_K) return launch_rows<Q6_K, true>(w, gate, y, rows, cols, s, up);
    return launch_rows<Q4_K, true>(w, gate, y, rows, cols, s, up);
}

}  // namespace fy
