// Prefill GEMM: Y[m][n] = sum_k X[m][k] * W[n][k] for batches above the
// small-N kernels' 8 columns (prompt tiles), on gfx950 MFMA.
//
// Numerics. Weights are dequantized to fp32 exactly as the reference decodes
// them (backend/core/llm_quant.c:70-142: Q4_K (d*sc)*q - dmin*m, Q6_K
// (d*sc)*q6, Q8_0 d*q, Q4_0 d*(q-8), no contraction). Every fp32 value v is
// then written as three bf16 pieces v = v0 + v1 + v2 with v0 = bf16(v),
// v1 = bf16(v - v0), v2 = bf16(v - v0 - v1); the split is exact for normal
// fp32 values (8 + 8 + 8 significand bits). The MFMA unit accumulates the six
// piece products x_i * w_j with i + j <= 2 in fp32; the dropped terms are below
// 2^-26 of |x*w|, so results carry fp32 accumulation error only, as the
// reference's fp32 tiles do (CUDA/gemm.cu:1-3, :13-15). Products of bf16
// pieces are exact in fp32.
//
// Work split. gemm_split_x writes the activation pieces once into the
// caller's workspace ([3][M][K] bf16). gemm_tile computes a 128 x 128 tile of
// Y per 256-thread workgroup: four wavefronts of 64 x 64, each a 2 x 2 grid of
// v_mfma_f32_32x32x16_bf16. K advances 32 columns per step (one Q8_0/Q4_0
// block, one nibble half of a Q4_K unit, two scale groups of a Q6_K unit).
// LDS holds two steps of activation and weight pieces (double buffer,
// 120 KiB, one barrier per step): while the MFMAs consume step s, the
// wavefronts decode and split step s+1 into the other buffer and fetch step
// s+2 from global memory into registers. Rows are padded to 40 bf16 so the
// 16-byte fragment reads of eight consecutive lanes cover all 32 banks.
#include "device.h"
#include "formats.h"
#include "kernels.h"

namespace fy {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// Native vector type for 16-byte staging: HIP's uint4 is a union whose
// copies become memcpy calls that keep a register array in scratch.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32, PITCH = BK + 8, PIECES = 3;
constexpr int kThreads = 256;
constexpr int kXChunks = PIECES * BM * (BK / 8) / kThreads;   // 16-byte activation chunks per thread

__device__ __forceinline__ uint32_t bf16_bits(float v)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v);
}

__device__ __forceinline__ float bf16_value(uint32_t bits)
{
    return __builtin_bit_cast(float, bits << 16);
}

// The three bf16 pieces of v0 and v1, packed in pairs: p[i] = piece i of
// v0 | piece i of v1 << 16.
__device__ __forceinline__ void split_pair(float v0, float v1, uint32_t (&p)[PIECES])
{
    const uint32_t a0 = bf16_bits(v0), a1 = bf16_bits(v1);
    const float r0 = v0 - bf16_value(a0), r1 = v1 - bf16_value(a1);
    const uint32_t b0 = bf16_bits(r0), b1 = bf16_bits(r1);
    const float s0 = r0 - bf16_value(b0), s1 = r1 - bf16_value(b1);
    p[0] = a0 | (a1 << 16);
    p[1] = b0 | (b1 << 16);
    p[2] = bf16_bits(s0) | (bf16_bits(s1) << 16);
}

__global__ __launch_bounds__(256) void gemm_split_x(const float4 *__restrict__ x, uint2 *__restrict__ out,
    size_t count4)
{
    for (size_t i = blockIdx.x * 256u + threadIdx.x; i < count4; i += (size_t)gridDim.x * 256u) {
        const float4 v = x[i];
        uint32_t a[PIECES], b[PIECES];
        split_pair(v.x, v.y, a);
        split_pair(v.z, v.w, b);
#pragma unroll
        for (int p = 0; p < PIECES; ++p) out[count4 * p + i] = make_uint2(a[p], b[p]);
    }
}

// Raw bytes behind 16 of the 32 columns of one K step of one weight row
// (`half` selects which 16): loaded two steps ahead, decoded one step ahead.
struct WRaw { u32x4 q, c; uint32_t e, f; };

// K step s covers 32 columns. Q8_0/Q4_0: block s. Q4_K: unit s/2, nibble
// s%2 (the low nibble sub-block then the high one), natural column order.
// Q6_K: unit u = s/2 = 4t + 2h + l16, whose scale groups q = 2(s%2) and
// 2(s%2)+1 cover columns 256t + 128h + 32q + 16*l16 + i (i < 16), taken in
// (q, i) order. x_column maps a step-local column k to X's column.
template <unsigned T>
__device__ __forceinline__ int x_column(int step, int k)
{
    if constexpr (T == Q6_K) {
        const int u = step >> 1, q = 2 * (step & 1) + (k >> 4);
        return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * q + 16 * (u & 1) + (k & 15);
    } else {
        return BK * step + k;
    }
}

template <unsigned T>
__device__ __forceinline__ void load_w(WRaw &r, const uint8_t *__restrict__ w, int rows, int cols, int row,
    int step, int half)
{
    // The tiled layout of formats.h: tile of 32 rows, 256-column groups.
    const int tile = row / kTileRows, rr = row % kTileRows;
    const int R = rows - kTileRows * tile < kTileRows ? rows - kTileRows * tile : kTileRows;
    const uint8_t *tb = w + (size_t)kTileRows * tile * tiled_row_bytes<T>(cols);
    if constexpr (T == Q4_K) {
        const int g = step >> 3, p = (step >> 1) & 3;
        const uint8_t *b = tb + (size_t)144 * R * g;
        r.q = *(const u32x4 *)(b + 32 * R * p + 16 * R * half + 16 * rr);   // qa (half 0) or qb (half 1)
        r.c = *(const u32x4 *)(b + 128 * R + 16 * rr);                      // the superblock's four slices
    } else if constexpr (T == Q6_K) {
        const int u = step >> 1, g = u >> 2, p = u & 3;
        const uint8_t *b = tb + (size_t)208 * R * g;
        r.q = *(const u32x4 *)(b + 48 * R * p + 16 * R * half + 16 * rr);   // ql of scale groups 0,2 (la) or 1,3 (lb)
        r.c = *(const u32x4 *)(b + 48 * R * p + 32 * R + 16 * rr);          // qh
        r.e = *(const uint32_t *)(b + 192 * R + 16 * rr + 4 * p);           // sc of scale groups 0..3
        r.f = *(const uint16_t *)(tb + (size_t)208 * R * ((cols + 255) / 256) + 2 * R * g + 2 * rr);   // d
    } else {
        constexpr int quant = T == Q8_0 ? 32 : 16;
        const int g = step >> 3, j = step & 7, left = cols / 32 - 8 * g, nb = left < 8 ? left : 8;
        const uint8_t *b = tb + (size_t)(quant + 2) * 8 * R * g;
        r.q = *(const u32x4 *)(b + quant * R * j + quant * rr + (T == Q8_0 ? 16 * half : 0));
        r.e = *(const uint16_t *)(b + quant * R * nb + 2 * R * j + 2 * rr);
    }
}

// Step-local columns 16*half .. 16*half+15 as fp32, in the reference's
// per-element arithmetic (backend/core/llm_quant.c:70-142).
template <unsigned T>
__device__ __forceinline__ void decode_w(float (&v)[16], const WRaw &r, int step, int half)
{
    if constexpr (T == Q4_K) {
        const int nib = step & 1;
        const uint32_t own = r.c[(step >> 1) & 3];
        const uint32_t dd = (r.c.x >> 24) | ((r.c.y >> 24) << 8) | ((r.c.z >> 24) << 16) | ((r.c.w >> 24) << 24);
        const float d = f16_to_f32(dd & 0xFFFFu), dmin = f16_to_f32(dd >> 16);
        const uint32_t sc = (own >> (12 * nib)) & 63u, mn = (own >> (12 * nib + 6)) & 63u;
        const float factor = __fmul_rn(d, (float)sc), bias = __fmul_rn(dmin, (float)mn);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t q = (r.q[j] >> (4 * nib)) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * j + b] = __fmul_rn(factor, ubyte_f32(q, b)) - bias;
        }
    } else if constexpr (T == Q6_K) {
        const int q = 2 * (step & 1) + half;
        const float d = f16_to_f32(r.f);
        const float factor = __fmul_rn(d, (float)(int8_t)((r.e >> (8 * q)) & 0xFFu));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = ((r.q[j] >> (4 * (step & 1))) & 0x0F0F0F0Fu) | (((r.c[j] >> (2 * q)) & 0x03030303u) << 4);
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * j + b] = __fmul_rn(factor, ubyte_f32(u, b) - 32.f);
        }
    } else if constexpr (T == Q8_0) {
        const float d = f16_to_f32(r.e);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * j + b] = d * (float)(int8_t)((r.q[j] >> (8 * b)) & 0xFFu);
    } else {
        const float d = f16_to_f32(r.e);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * j + b] = d * (float)((int)((r.q[j] >> (8 * b + 4 * half)) & 15u) - 8);
    }
}

// LDS for two steps: [buffer][piece][row][PITCH] of activations (m) and
// weights (n).
struct Tiles {
    uint16_t a[2][PIECES][BM][PITCH];
    uint16_t b[2][PIECES][BN][PITCH];
};

// Global loads of one K step: this thread's activation chunks (3 pieces x
// 128 rows x 4 chunks of 8 bf16 = 1536 chunks, 6 per thread; rows past the
// batch reload row 0, discarded) and its weight bytes (16 columns, half
// `whalf`, of row `wr`; rows past the matrix reload its last row).
template <unsigned T>
__device__ __forceinline__ void load_step(u32x4 (&a_reg)[kXChunks], WRaw &raw, const uint8_t *__restrict__ w,
    const uint16_t *__restrict__ xp, size_t plane, int rows, int cols, int batch, int m0, int wr, int step,
    int whalf)
{
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
        const int c = threadIdx.x + kThreads * i, piece = c / (BM * 4), r = (c >> 2) & (BM - 1), ch = c & 3;
        const int m = m0 + r < batch ? m0 + r : 0;
        a_reg[i] = *(const u32x4 *)(xp + plane * piece + (size_t)m * cols + x_column<T>(step, 8 * ch));
    }
    load_w<T>(raw, w, rows, cols, wr, step, whalf);
}

// LDS stores of one K step into buffer `buf`: activation chunks as loaded,
// weight columns decoded to fp32 and split into bf16 pieces.
template <unsigned T>
__device__ __forceinline__ void store_step(Tiles &t, int buf, const u32x4 (&a_reg)[kXChunks], const WRaw &raw,
    int wrow, int step, int whalf)
{
#pragma unroll
    for (int i = 0; i < kXChunks; ++i) {
        const int c = threadIdx.x + kThreads * i, piece = c / (BM * 4), r = (c >> 2) & (BM - 1), ch = c & 3;
        *(u32x4 *)&t.a[buf][piece][r][8 * ch] = a_reg[i];
    }
    float v[16];
    decode_w<T>(v, raw, step, whalf);
    u32x4 out[PIECES][2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t p[PIECES];
        split_pair(v[2 * i], v[2 * i + 1], p);
#pragma unroll
        for (int k = 0; k < PIECES; ++k) out[k][i >> 2][i & 3] = p[k];
    }
#pragma unroll
    for (int k = 0; k < PIECES; ++k) {
        *(u32x4 *)&t.b[buf][k][wrow][16 * whalf] = out[k][0];
        *(u32x4 *)&t.b[buf][k][wrow][16 * whalf + 8] = out[k][1];
    }
}

template <unsigned T>
__global__ __launch_bounds__(kThreads) void gemm_tile(const uint8_t *__restrict__ w, const uint16_t *__restrict__ xp,
    float *__restrict__ y, int rows, int cols, int batch, int batch_total)
{
    __shared__ __align__(16) Tiles t;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const size_t plane = (size_t)batch_total * cols;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int steps = cols / BK;
    // Weight staging: thread t decodes 16 columns (half t&1) of row t>>1.
    const int wrow = tid >> 1, whalf = tid & 1;
    const int wr = n0 + wrow < rows ? n0 + wrow : rows - 1;
    u32x4 a_reg[kXChunks];
    WRaw raw;
    load_step<T>(a_reg, raw, w, xp, plane, rows, cols, batch, m0, wr, 0, whalf);
    store_step<T>(t, 0, a_reg, raw, wrow, 0, whalf);
    load_step<T>(a_reg, raw, w, xp, plane, rows, cols, batch, m0, wr, steps > 1 ? 1 : 0, whalf);
    __syncthreads();
    for (int step = 0; step < steps; ++step) {
        const int cur = step & 1;
        // Step+1 into the other buffer (read by nobody since the last
        // barrier), then fetch step+2. Past the end both repeat the last
        // step: harmless, and it keeps the loop body branch-free.
        store_step<T>(t, cur ^ 1, a_reg, raw, wrow, step + 1 < steps ? step + 1 : steps - 1, whalf);
        load_step<T>(a_reg, raw, w, xp, plane, rows, cols, batch, m0, wr, step + 2 < steps ? step + 2 : steps - 1,
            whalf);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kc = 16 * ks + 8 * (lane >> 5);
            bf16x8 a[2][PIECES], b[2][PIECES];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int p = 0; p < PIECES; ++p) {
                    a[i][p] = *(const bf16x8 *)&t.a[cur][p][wm + 32 * i + (lane & 31)][kc];
                    b[i][p] = *(const bf16x8 *)&t.b[cur][p][wn + 32 * i + (lane & 31)][kc];
                }
            // Smallest terms first; the four tiles interleave so that no
            // MFMA waits on the one before it.
#pragma unroll
            for (int term = 0; term < 6; ++term) {
                constexpr int pa[6] = {2, 1, 0, 1, 0, 0}, pb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][pa[term]], b[j][pb[term]],
                            acc[i][j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    // D lane l, register r: row 8(r/4) + 4(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < batch && n < rows) y[(size_t)m * rows + n] = acc[i][j][r];
            }
        }
}

template <unsigned T>
hipError_t launch_tiles(const uint8_t *w, const uint16_t *xp, float *y, int rows, int cols, int batch, hipStream_t s)
{
    // Weight tiles along x; batch tiles along y, at most 65535 per launch.
    constexpr int kMaxY = 65535;
    for (int m = 0; m < batch; m += kMaxY * BM) {
        const int mb = batch - m < kMaxY * BM ? batch - m : kMaxY * BM;
        const dim3 grid((unsigned)((rows + BN - 1) / BN), (unsigned)((mb + BM - 1) / BM));
        hipLaunchKernelGGL(gemm_tile<T>, grid, dim3(kThreads), 0, s, w, xp + (size_t)m * cols, y + (size_t)m * rows,
            rows, cols, mb, batch);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

bool gemm_supported(unsigned type, int cols)
{
    return (type == Q4_K || type == Q6_K || type == Q8_0 || type == Q4_0) && cols % 64 == 0;
}

size_t gemm_workspace(int cols, int batch)
{
    return (size_t)2 * PIECES * cols * batch;   // three bf16 pieces of X
}

hipError_t launch_gemm(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, int batch,
    void *workspace, hipStream_t s)
{
    const size_t count4 = (size_t)cols * batch / 4;
    const size_t blocks = (count4 + 255) / 256;
    hipLaunchKernelGGL(gemm_split_x, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, s,
        (const float4 *)x, (uint2 *)workspace, count4);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint16_t *xp = (const uint16_t *)workspace;
    switch (type) {
    case Q4_K: return launch_tiles<Q4_K>(w, xp, y, rows, cols, batch, s);
    case Q6_K: return launch_tiles<Q6_K>(w, xp, y, rows, cols, batch, s);
    case Q8_0: return launch_tiles<Q8_0>(w, xp, y, rows, cols, batch, s);
    case Q4_0: return launch_tiles<Q4_0>(w, xp, y, rows, cols, batch, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace fy
