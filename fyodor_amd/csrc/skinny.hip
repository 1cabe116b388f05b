// Batch 1..8 quantized matrix products (decode matvec and the small-N path).
//
// Work split: a 256-thread workgroup is four wavefronts; each wavefront owns
// R consecutive output rows (per-wavefront row ownership) and its 64 lanes
// split the columns into units of 32 or 64 elements, so one lane reads one
// unit of each of its R rows with 16-byte loads, unpacks it in registers and
// multiplies it against the activations, which the workgroup stages once
// per column chunk in LDS together with their 16-element sums. Per-lane
// partial sums are reduced across the wavefront at the end.
//
// Arithmetic follows the block definitions of backend/core/llm_quant.c:
// 206-311 with the per-block scale factored out of the block sum:
//   Q8_0  d * (sum (q+128) x - 128 * sum x)
//   Q4_0  d * (sum q x - 8 * sum x)
//   Q4_K  d*sc * sum q x - dmin*m * sum x          (per 32-element group)
//   Q6_K  d*sc * (sum q6 x - 32 * sum x)            (per 16-element group)
// Products and sums are fp32; only the order of the reduction differs from
// the reference's sequential loop.
#include "device.h"
#include "formats.h"
#include "kernels.h"

namespace fy {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// Columns staged per chunk: 32 KiB of fp32 activations at any batch.
template <int N> constexpr int chunk_cols() { return N <= 1 ? 8192 : N == 2 ? 4096 : N <= 4 ? 2048 : 1024; }
// LDS index of chunk column k: 4 floats of padding after every 32 columns
// spread the lanes' unit bases over the banks.
__host__ __device__ constexpr int padded(int k) { return k + (k >> 5) * 4; }

template <unsigned T> struct unit_elems { static constexpr int value = 64; };
template <> struct unit_elems<Q8_0> { static constexpr int value = 32; };
template <> struct unit_elems<Q4_0> { static constexpr int value = 32; };

template <int N>
struct Stage {
    static constexpr int KC = chunk_cols<N>();
    static constexpr int XS = padded(KC);      // floats per staged column
    static constexpr int GS = KC / 16;         // 16-element sums per column
};

// ---- Q4_K: unit = (superblock s, nibble pair p): qs[32p .. 32p+32) ----
template <int N, int R>
__device__ __forceinline__ void unit_q4k(const uint8_t *__restrict__ w, int cols, int row0, int nrow,
    int unit, int local, const float *xs, const float *gs, float (&acc)[R][N])
{
    using S = Stage<N>;
    const size_t row_bytes = (size_t)(cols / 256) * 144;
    const int s = unit >> 2, p = unit & 3;
    uint4 hd[R], qa[R], qb[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r < nrow) {
            const uint8_t *b = w + (size_t)(row0 + r) * row_bytes + (size_t)s * 144;
            hd[r] = *(const uint4 *)b;
            qa[r] = *(const uint4 *)(b + 16 + 32 * p);
            qb[r] = *(const uint4 *)(b + 32 + 32 * p);
        }
    }
    // Sub-blocks 2p and 2p+1 (backend/core/llm_quant.c:249-250).
    float f0[R], f1[R], c0[R], c1[R];
    const int shift = 16 * (p & 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r >= nrow) continue;
        const float d = f16_to_f32(hd[r].x & 0xFFFFu), dmin = f16_to_f32(hd[r].x >> 16);
        const uint32_t a = hd[r].y >> shift, bm = hd[r].z >> shift, hw = hd[r].w >> shift;
        uint32_t sc0, sc1, m0, m1;
        if (p < 2) {
            sc0 = a & 63u; m0 = bm & 63u; sc1 = (a >> 8) & 63u; m1 = (bm >> 8) & 63u;
        } else {
            sc0 = (hw & 15u) | (((a >> 6) & 3u) << 4);
            m0 = ((hw >> 4) & 15u) | (((bm >> 6) & 3u) << 4);
            sc1 = ((hw >> 8) & 15u) | (((a >> 14) & 3u) << 4);
            m1 = ((hw >> 12) & 15u) | (((bm >> 14) & 3u) << 4);
        }
        f0[r] = d * (float)sc0; f1[r] = d * (float)sc1;
        c0[r] = dmin * (float)m0; c1[r] = dmin * (float)m1;
    }
    const int base = local * 64;
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float *xn = xs + n * S::XS;
        float A[R], B[R];
#pragma unroll
        for (int r = 0; r < R; ++r) { A[r] = 0.f; B[r] = 0.f; }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 xl = *(const float4 *)(xn + padded(base + 4 * j));
            const float4 xh = *(const float4 *)(xn + padded(base + 32 + 4 * j));
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t dw = j < 4 ? word_of(qa[r], j) : word_of(qb[r], j - 4);
                const uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
                A[r] += ubyte_f32(lo, 0) * xl.x + ubyte_f32(lo, 1) * xl.y + ubyte_f32(lo, 2) * xl.z + ubyte_f32(lo, 3) * xl.w;
                B[r] += ubyte_f32(hi, 0) * xh.x + ubyte_f32(hi, 1) * xh.y + ubyte_f32(hi, 2) * xh.z + ubyte_f32(hi, 3) * xh.w;
            }
        }
        const float *g = gs + n * S::GS + base / 16;
        const float s0 = g[0] + g[1], s1 = g[2] + g[3];
#pragma unroll
        for (int r = 0; r < R; ++r)
            acc[r][n] += f0[r] * A[r] + f1[r] * B[r] - (c0[r] * s0 + c1[r] * s1);
    }
}

// ---- Q6_K: unit = (superblock s, half h, lane half l16): 16 lanes l of
// all four quarters q, i.e. elements 128h + 32q + 16*l16 + i ----
template <int N, int R>
__device__ __forceinline__ void unit_q6k(const uint8_t *__restrict__ w, int rows, int cols, int row0, int nrow,
    int unit, int local, const float *xs, const float *gs, float (&acc)[R][N])
{
    using S = Stage<N>;
    const size_t ns = (size_t)(cols / 256);
    const uint8_t *qp = w, *sp = w + (size_t)rows * ns * 192, *dp = w + (size_t)rows * ns * 208;
    const int s = unit >> 2, h = (unit >> 1) & 1, l16 = unit & 1;
    uint4 la[R], lb[R], qh[R];
    uint2 sc[R];
    uint32_t dh[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r < nrow) {
            const size_t block = (size_t)(row0 + r) * ns + s;
            const uint8_t *q = qp + block * 192;
            la[r] = *(const uint4 *)(q + 64 * h + 16 * l16);
            lb[r] = *(const uint4 *)(q + 64 * h + 32 + 16 * l16);
            qh[r] = *(const uint4 *)(q + 128 + 32 * h + 16 * l16);
            sc[r] = *(const uint2 *)(sp + block * 16 + 8 * h);
            dh[r] = *(const uint16_t *)(dp + block * 2);
        }
    }
    // Scale of quarter q is sc[8h + 2q + l16] (backend/core/llm_quant.c:256-262).
    float f[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r >= nrow) continue;
        const float d = f16_to_f32(dh[r]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int byte = l16 + 2 * q;
            const uint32_t word = byte < 4 ? sc[r].x : sc[r].y;
            const int8_t v = (int8_t)((word >> (8 * (byte & 3))) & 0xFFu);
            f[r][q] = d * (float)v;
        }
    }
    const int base = (local >> 2) * 256 + 128 * h + 16 * l16;
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float *xn = xs + n * S::XS;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float A[R];
#pragma unroll
            for (int r = 0; r < R; ++r) A[r] = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 x4 = *(const float4 *)(xn + padded(base + 32 * q + 4 * j));
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t ql = word_of((q & 1) ? lb[r] : la[r], j);
                    const uint32_t v = ((ql >> (4 * (q >> 1))) & 0x0F0F0F0Fu) |
                        (((word_of(qh[r], j) >> (2 * q)) & 0x03030303u) << 4);
                    A[r] += ubyte_f32(v, 0) * x4.x + ubyte_f32(v, 1) * x4.y + ubyte_f32(v, 2) * x4.z + ubyte_f32(v, 3) * x4.w;
                }
            }
            const float s16 = gs[n * S::GS + (base + 32 * q) / 16];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][n] += f[r][q] * (A[r] - 32.f * s16);
        }
    }
}

// ---- Q8_0: unit = one 32-element block ----
template <int N, int R>
__device__ __forceinline__ void unit_q80(const uint8_t *__restrict__ w, int rows, int cols, int row0, int nrow,
    int unit, int local, const float *xs, const float *gs, float (&acc)[R][N])
{
    using S = Stage<N>;
    const size_t nb = (size_t)(cols / 32);
    const uint8_t *dp = w + (size_t)rows * nb * 32;
    uint4 qa[R], qb[R];
    uint32_t dh[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r < nrow) {
            const size_t block = (size_t)(row0 + r) * nb + unit;
            qa[r] = *(const uint4 *)(w + block * 32);
            qb[r] = *(const uint4 *)(w + block * 32 + 16);
            dh[r] = *(const uint16_t *)(dp + block * 2);
        }
    }
    const int base = local * 32;
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float *xn = xs + n * S::XS;
        float A[R];
#pragma unroll
        for (int r = 0; r < R; ++r) A[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 x4 = *(const float4 *)(xn + padded(base + 4 * j));
#pragma unroll
            for (int r = 0; r < R; ++r) {
                // Flipping the sign bit maps int8 q to the byte q + 128.
                const uint32_t v = (j < 4 ? word_of(qa[r], j) : word_of(qb[r], j - 4)) ^ 0x80808080u;
                A[r] += ubyte_f32(v, 0) * x4.x + ubyte_f32(v, 1) * x4.y + ubyte_f32(v, 2) * x4.z + ubyte_f32(v, 3) * x4.w;
            }
        }
        const float *g = gs + n * S::GS + base / 16;
        const float s32 = g[0] + g[1];
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r < nrow) acc[r][n] += f16_to_f32(dh[r]) * (A[r] - 128.f * s32);
    }
}

// ---- Q4_0: unit = one 32-element block ----
template <int N, int R>
__device__ __forceinline__ void unit_q40(const uint8_t *__restrict__ w, int rows, int cols, int row0, int nrow,
    int unit, int local, const float *xs, const float *gs, float (&acc)[R][N])
{
    using S = Stage<N>;
    const size_t nb = (size_t)(cols / 32);
    const uint8_t *dp = w + (size_t)rows * nb * 16;
    uint4 qa[R];
    uint32_t dh[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r < nrow) {
            const size_t block = (size_t)(row0 + r) * nb + unit;
            qa[r] = *(const uint4 *)(w + block * 16);
            dh[r] = *(const uint16_t *)(dp + block * 2);
        }
    }
    const int base = local * 32;
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float *xn = xs + n * S::XS;
        float A[R];
#pragma unroll
        for (int r = 0; r < R; ++r) A[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 xl = *(const float4 *)(xn + padded(base + 4 * j));
            const float4 xh = *(const float4 *)(xn + padded(base + 16 + 4 * j));
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t dw = word_of(qa[r], j);
                const uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
                A[r] += ubyte_f32(lo, 0) * xl.x + ubyte_f32(lo, 1) * xl.y + ubyte_f32(lo, 2) * xl.z + ubyte_f32(lo, 3) * xl.w;
                A[r] += ubyte_f32(hi, 0) * xh.x + ubyte_f32(hi, 1) * xh.y + ubyte_f32(hi, 2) * xh.z + ubyte_f32(hi, 3) * xh.w;
            }
        }
        const float *g = gs + n * S::GS + base / 16;
        const float s32 = g[0] + g[1];
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r < nrow) acc[r][n] += f16_to_f32(dh[r]) * (A[r] - 8.f * s32);
    }
}

template <unsigned T, int N, int R>
__global__ __launch_bounds__(kThreads) void skinny_quant(const uint8_t *__restrict__ w,
    const float *__restrict__ x, float *__restrict__ y, int rows, int cols)
{
    using S = Stage<N>;
    constexpr int UE = unit_elems<T>::value;
    __shared__ float xs[N * S::XS];
    __shared__ float gs[N * S::GS];
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
    const int nrow = rows - row0 < R ? rows - row0 : R;
    float acc[R][N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < N; ++n) acc[r][n] = 0.f;
    for (int k0 = 0; k0 < cols; k0 += S::KC) {
        const int kc = cols - k0 < S::KC ? cols - k0 : S::KC;
        __syncthreads();
        for (int i = threadIdx.x; i < N * kc; i += kThreads) {
            const int n = i / kc, k = i - n * kc;
            xs[n * S::XS + padded(k)] = x[(size_t)n * cols + k0 + k];
        }
        __syncthreads();
        for (int i = threadIdx.x; i < N * (kc / 16); i += kThreads) {
            const int n = i / (kc / 16), g = i - n * (kc / 16);
            const float *v = xs + n * S::XS + padded(16 * g);
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) s += v[e];
            gs[n * S::GS + g] = s;
        }
        __syncthreads();
        if (nrow > 0) {
            const int units = kc / UE, first = k0 / UE;
            for (int u = lane; u < units; u += 64) {
                if constexpr (T == Q4_K) unit_q4k<N, R>(w, cols, row0, nrow, first + u, u, xs, gs, acc);
                else if constexpr (T == Q6_K) unit_q6k<N, R>(w, rows, cols, row0, nrow, first + u, u, xs, gs, acc);
                else if constexpr (T == Q8_0) unit_q80<N, R>(w, rows, cols, row0, nrow, first + u, u, xs, gs, acc);
                else unit_q40<N, R>(w, rows, cols, row0, nrow, first + u, u, xs, gs, acc);
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

// F32 / F16 / BF16: lanes stride over the columns of R rows.
template <unsigned T, int N, int R>
__global__ __launch_bounds__(kThreads) void skinny_dense(const uint8_t *__restrict__ w,
    const float *__restrict__ x, float *__restrict__ y, int rows, int cols)
{
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
    const int nrow = rows - row0 < R ? rows - row0 : R;
    if (nrow <= 0) return;
    float acc[R][N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < N; ++n) acc[r][n] = 0.f;
    for (int k = lane; k < cols; k += 64) {
        float xv[N];
#pragma unroll
        for (int n = 0; n < N; ++n) xv[n] = x[(size_t)n * cols + k];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r >= nrow) continue;
            const size_t at = (size_t)(row0 + r) * cols + k;
            float wv;
            if constexpr (T == F32) wv = ((const float *)w)[at];
            else if constexpr (T == F16) wv = f16_to_f32(((const uint16_t *)w)[at]);
            else wv = bf16_to_f32(((const uint16_t *)w)[at]);
#pragma unroll
            for (int n = 0; n < N; ++n) acc[r][n] += wv * xv[n];
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

template <int N> constexpr int rows_per_wave() { return N <= 2 ? 4 : 2; }

template <unsigned T, int N>
hipError_t launch_n(const uint8_t *w, const float *x, float *y, int rows, int cols, hipStream_t stream)
{
    constexpr int R = rows_per_wave<N>();
    const int rows_per_block = kWaves * R;
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
    if constexpr (T == F32 || T == F16 || T == BF16)
        hipLaunchKernelGGL((skinny_dense<T, N, R>), grid, dim3(kThreads), 0, stream, w, x, y, rows, cols);
    else
        hipLaunchKernelGGL((skinny_quant<T, N, R>), grid, dim3(kThreads), 0, stream, w, x, y, rows, cols);
    return hipGetLastError();
}

template <unsigned T>
hipError_t launch_type(const uint8_t *w, const float *x, float *y, int rows, int cols, int batch, hipStream_t s)
{
    switch (batch) {
    case 1: return launch_n<T, 1>(w, x, y, rows, cols, s);
    case 2: return launch_n<T, 2>(w, x, y, rows, cols, s);
    case 3: return launch_n<T, 3>(w, x, y, rows, cols, s);
    case 4: return launch_n<T, 4>(w, x, y, rows, cols, s);
    case 5: return launch_n<T, 5>(w, x, y, rows, cols, s);
    case 6: return launch_n<T, 6>(w, x, y, rows, cols, s);
    case 7: return launch_n<T, 7>(w, x, y, rows, cols, s);
    case 8: return launch_n<T, 8>(w, x, y, rows, cols, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_skinny(unsigned type, const uint8_t *w, const float *x, float *y,
    int rows, int cols, int batch, hipStream_t s)
{
    switch (type) {
    case F32: return launch_type<F32>(w, x, y, rows, cols, batch, s);
    case F16: return launch_type<F16>(w, x, y, rows, cols, batch, s);
    case BF16: return launch_type<BF16>(w, x, y, rows, cols, batch, s);
    case Q4_0: return launch_type<Q4_0>(w, x, y, rows, cols, batch, s);
    case Q8_0: return launch_type<Q8_0>(w, x, y, rows, cols, batch, s);
    case Q4_K: return launch_type<Q4_K>(w, x, y, rows, cols, batch, s);
    case Q6_K: return launch_type<Q6_K>(w, x, y, rows, cols, batch, s);
    default: return hipErrorInvalidValue;
    }
}

const char *skinny_name(unsigned type, int batch)
{
    (void)batch;
    return type == F32 || type == F16 || type == BF16 ? "skinny_dense" : "skinny_quant";
}

}  // namespace fy
