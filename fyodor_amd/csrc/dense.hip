// Batch 1..8 products of dense F32 / F16 / BF16 weights with fp32
// activations. Each wavefront owns R rows; its lanes stride over the columns
// (coalesced 4- or 2-byte loads) and the per-lane fp32 sums are reduced
// across the wavefront. These storage types have no block structure; the
// reference decodes them per element (backend/core/llm_quant.c:161-204).
#include "device.h"
#include "formats.h"
#include "kernels.h"
#include <stdint.h>

namespace fy {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

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
    hipLaunchKernelGGL((skinny_dense<T, N, R>), grid, dim3(kThreads), 0, stream, w, x, y, rows, cols);
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

hipError_t launch_dense(unsigned type, const uint8_t *w, const float *x, float *y,
    int rows, int cols, int batch, hipStream_t s)
{
    switch (type) {
    case F32: return launch_type<F32>(w, x, y, rows, cols, batch, s);
    case F16: return launch_type<F16>(w, x, y, rows, cols, batch, s);
    case BF16: return launch_type<BF16>(w, x, y, rows, cols, batch, s);
    default: return hipErrorInvalidValue;
    }
}

namespace {
__global__ __launch_bounds__(256) void copy16(uint4 *__restrict__ dst, const uint4 *__restrict__ src, size_t count)
{
    for (size_t i = blockIdx.x * 256u + threadIdx.x; i < count; i += (size_t)gridDim.x * 256u) dst[i] = src[i];
}
}  // namespace

hipError_t launch_copy(uint4 *dst, const uint4 *src, size_t count, hipStream_t stream)
{
    const size_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(copy16, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, stream, dst, src, count);
    return hipGetLastError();
}

namespace {
// Plain streaming read of `bytes` (a multiple of 16): one workgroup of four
// wavefronts per CU over a contiguous share; each wavefront issues 32
// non-temporal 16-byte loads per lane per pass (1 KiB per load, wavefronts
// interleaved per KiB), the fastest plain read of a 33 MB matrix measured
// among 2..16 wavefronts and 8..64 loads in flight. Loads past the share
// read zeros (buffer range check); they stay live through an xor that is
// stored only if it equals a constant.
constexpr int kReadWaves = 4, kReadDepth = 32;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(64 * kReadWaves) void read16(const uint8_t *__restrict__ src, size_t bytes, size_t share,
    unsigned *__restrict__ sink)
{
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t begin = (size_t)blockIdx.x * share;
    const size_t n = begin < bytes ? (bytes - begin < share ? bytes - begin : share) : 0;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src + begin), (short)0, (int)n, 0x00020000);
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (size_t pass = 0; pass < n; pass += (size_t)1024 * kReadWaves * kReadDepth) {
        u32x4 v[kReadDepth];
#pragma unroll
        for (int u = 0; u < kReadDepth; ++u)
            v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       r, (int)(pass + 1024 * (u * kReadWaves + wave)) + 16 * lane, 0, 2));
#pragma unroll
        for (int u = 0; u < kReadDepth; ++u) acc ^= v[u];
    }
    const unsigned x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}
}  // namespace

hipError_t launch_read(const uint4 *src, size_t count, unsigned *sink, hipStream_t stream)
{
    const int cus = device_cu_count();
    const unsigned blocks = (unsigned)(cus < kReadSinkWords ? cus : kReadSinkWords);
    const size_t bytes = count * 16;
    // Shares are whole KiB, and below 2 GiB for the 32-bit buffer range.
    const size_t share = (bytes + (size_t)1024 * blocks - 1) / ((size_t)1024 * blocks) * 1024;
    if (share > (size_t)INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(read16, dim3(blocks), dim3(64 * kReadWaves), 0, stream, (const uint8_t *)src, bytes, share,
                       sink);
    return hipGetLastError();
}

namespace {
// The same streaming read in other shapes, to find the fastest plain read of
// a given size: W wavefronts per workgroup, D 16-byte loads in flight per
// lane per pass, and the loads either into registers (MODE 0 non-temporal,
// MODE 1 the default cache policy) or straight into LDS (MODE 2,
// buffer_load_dwordx4 ... lds: wavefront w's D KiB at LDS offset w D KiB,
// waited for before the next pass reuses it). A workgroup reads one
// contiguous share; past it the buffer range check returns zeros.
template <int W, int D, int MODE>
__global__ __launch_bounds__(64 * W) void read_shaped(const uint8_t *__restrict__ src, size_t bytes, size_t share,
    unsigned *__restrict__ sink)
{
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t begin = (size_t)blockIdx.x * share;
    const size_t n = begin < bytes ? (bytes - begin < share ? bytes - begin : share) : 0;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src + begin), (short)0, (int)n, 0x00020000);
    u32x4 acc = {0u, 0u, 0u, 0u};
    if constexpr (MODE == 2) {
        extern __shared__ __align__(16) uint8_t lds[];
        for (size_t pass = 0; pass < n; pass += (size_t)1024 * W * D) {
#pragma unroll
            for (int u = 0; u < D; ++u)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    r, (__attribute__((address_space(3))) void *)(lds + 1024 * (wave * D + u)), 16, 16 * lane,
                    (int)(pass + 1024 * (u * W + wave)), 0, 0);
            // The copies land before the next pass overwrites the same LDS.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        acc = *(const u32x4 *)(lds + 1024 * wave * D + 16 * lane);
    } else {
        for (size_t pass = 0; pass < n; pass += (size_t)1024 * W * D) {
            u32x4 v[D];
#pragma unroll
            for (int u = 0; u < D; ++u)
                v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           r, (int)(pass + 1024 * (u * W + wave)) + 16 * lane, 0, MODE == 0 ? 2 : 0));
#pragma unroll
            for (int u = 0; u < D; ++u) acc ^= v[u];
        }
    }
    const unsigned x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9E3779B9u) sink[blockIdx.x % kReadSinkWords] = x;
}

template <int W, int D, int MODE>
hipError_t launch_shaped(const uint8_t *src, size_t bytes, size_t share, unsigned blocks, unsigned *sink,
    hipStream_t stream)
{
    const size_t lds = MODE == 2 ? (size_t)1024 * W * D : 0;
    hipLaunchKernelGGL((read_shaped<W, D, MODE>), dim3(blocks), dim3(64 * W), lds, stream, src, bytes, share, sink);
    return hipGetLastError();
}
}  // namespace

// (waves, depth) pairs: 4 x 32, 4 x 16, 8 x 16, 8 x 8, 16 x 8, 16 x 4, all
// at most 128 KiB in flight per workgroup (the LDS form holds them all).
hipError_t launch_read_shaped(const uint4 *src, size_t count, unsigned *sink, int waves, int depth, int per_cu,
    int mode, hipStream_t stream)
{
    if (mode < 0 || mode > 2 || per_cu < 1 || per_cu > 4) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)(device_cu_count() * per_cu);
    const size_t bytes = count * 16;
    const size_t share = (bytes + (size_t)1024 * blocks - 1) / ((size_t)1024 * blocks) * 1024;
    if (share > (size_t)INT32_MAX) return hipErrorInvalidValue;
    const uint8_t *s = (const uint8_t *)src;
#define FY_SHAPE(w, d)                                                                                            \
    if (waves == w && depth == d) {                                                                               \
        if (mode == 0) return launch_shaped<w, d, 0>(s, bytes, share, blocks, sink, stream);                     \
        if (mode == 1) return launch_shaped<w, d, 1>(s, bytes, share, blocks, sink, stream);                     \
        return launch_shaped<w, d, 2>(s, bytes, share, blocks, sink, stream);                                    \
    }
    FY_SHAPE(4, 32)
    FY_SHAPE(4, 16)
    FY_SHAPE(8, 16)
    FY_SHAPE(8, 8)
    FY_SHAPE(16, 8)
    FY_SHAPE(16, 4)
#undef FY_SHAPE
    return hipErrorInvalidValue;
}

}  // namespace fy
