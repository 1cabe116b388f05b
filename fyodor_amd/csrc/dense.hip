// Batch 1..8 products of dense F32 / F16 / BF16 weights with fp32
// activations. Each wavefront owns R rows; its lanes stride over the columns
// (coalesced 4- or 2-byte loads) and the per-lane fp32 sums are reduced
// across the wavefront. These storage types have no block structure; the
// reference decodes them per element (backend/core/llm_quant.c:161-204).
#include "device.h"
#include "formats.h"
#include "kernels.h"

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

}  // namespace fy
