// The vector operations of one decoder token kept on the device (the resident
// plan of the ROCm provider): the embedding row, RMS normalization, rotary
// position encoding, causal attention over the KV cache, the gated SiLU and
// the residual add. Each restates one step of the engine's CPU token forward
// (backend/core/llm_cpu.c:424-578, LLaMA branch) with the same operation
// order per element; arithmetic is not contracted into fused multiply-adds
// (the reference's C17 build does not contract either). The matrix products
// between them are the library's quantized kernels.
#include <math.h>

#include "kernels.h"

#pragma clang fp contract(off)

namespace fy {
namespace {

__device__ __forceinline__ float half_at(const uint8_t *p)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8)));
}

// Element i of a row stored in GGUF layout (backend/core/llm_quant.c:70-142;
// Q4_K and Q6_K with the reference's own float operation order).
__device__ float element(const uint8_t *row, unsigned type, int i)
{
    switch (type) {
    case 0: return __builtin_bit_cast(float, (uint32_t)row[4 * i] | (uint32_t)row[4 * i + 1] << 8 |
                                                 (uint32_t)row[4 * i + 2] << 16 | (uint32_t)row[4 * i + 3] << 24);
    case 1: return half_at(row + 2 * i);
    case 30: return __builtin_bit_cast(float, ((uint32_t)row[2 * i] | (uint32_t)row[2 * i + 1] << 8) << 16);
    case 8: {
        const uint8_t *b = row + i / 32 * 34;
        return half_at(b) * (float)(int8_t)b[2 + i % 32];
    }
    case 2: {
        const uint8_t *b = row + i / 32 * 18;
        const int at = i % 32, packed = b[2 + at % 16];
        return half_at(b) * (float)((at < 16 ? packed & 15 : packed >> 4) - 8);
    }
    case 12: {
        const uint8_t *b = row + i / 256 * 144, *s = b + 4;
        const int at = i % 256, g = at / 32;
        const unsigned sc = g < 4 ? s[g] & 63u : (s[g + 4] & 15u) | ((unsigned)(s[g - 4] >> 6) << 4);
        const unsigned mn = g < 4 ? s[g + 4] & 63u : (s[g + 4] >> 4) | ((unsigned)(s[g] >> 6) << 4);
        const unsigned q = (b[16 + g / 2 * 32 + at % 32] >> (g % 2 * 4)) & 15u;
        return half_at(b) * (float)sc * (float)q - half_at(b + 2) * (float)mn;
    }
    case 14: {
        const uint8_t *b = row + i / 256 * 210;
        const int at = i % 256, half = at / 128, quarter = at % 128 / 32, lane = at % 32;
        const unsigned lo = b[half * 64 + quarter % 2 * 32 + lane], hi = b[128 + half * 32 + lane];
        const int q = (int)(((lo >> (quarter / 2 * 4)) & 15u) | (((hi >> (quarter * 2)) & 3u) << 4)) - 32;
        const int8_t sc = (int8_t)b[192 + half * 8 + quarter * 2 + lane / 16];
        return half_at(b + 208) * (float)sc * (float)q;
    }
    default: return 0.f;
    }
}

__global__ __launch_bounds__(256) void dequant_row(const uint8_t *__restrict__ w, unsigned type, size_t row_bytes,
    size_t row, int cols, float *__restrict__ out)
{
    const uint8_t *r = w + row * row_bytes;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < cols; i += gridDim.x * 256) out[i] = element(r, type, i);
}

// One workgroup. x += r first when r is given (written back); then
// out = x * scale * w with scale = 1 / sqrt(sum x^2 / n + eps), the sum of
// squares in double (backend/core/llm_cpu.c:83-104).
__global__ __launch_bounds__(1024) void rms_norm(float *__restrict__ x, const float *__restrict__ r,
    const float *__restrict__ w, float *__restrict__ out, int n, float eps)
{
    __shared__ double part[16];
    const int t = threadIdx.x;
    double s = 0.0;
    for (int i = t; i < n; i += 1024) {
        float v = x[i];
        if (r) {
            v = v + r[i];
            x[i] = v;
        }
        s += (double)v * v;
    }
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    double total = 0.0;
    for (int k = 0; k < 16; ++k) total += part[k];
    const float scale = (float)(1.0 / sqrt(total / (double)n + (double)eps));
    for (int i = t; i < n; i += 1024) out[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

// Interleaved pairs of every head rotated by angle position * freq[j]
// (backend/core/llm_cpu.c:298-324, angles :429-432).
__global__ __launch_bounds__(256) void rope(float *__restrict__ v, int heads, int width,
    const float *__restrict__ freq, int position)
{
    const int pairs = width / 2;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < heads * pairs; i += gridDim.x * 256) {
        const int h = i / pairs, j = i % pairs;
        const float angle = (float)position * freq[j];
        const float c = cosf(angle), s = sinf(angle);
        float *p = v + h * width + 2 * j;
        const float a = p[0], b = p[1];
        p[0] = a * c - b * s;
        p[1] = a * s + b * c;
    }
}

__device__ __forceinline__ float block_reduce(float v, float *red, bool maximum)
{
    for (int o = 32; o >= 1; o >>= 1) {
        const float u = __shfl_xor(v, o, 64);
        v = maximum ? fmaxf(v, u) : v + u;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int k = 1; k < 4; ++k) r = maximum ? fmaxf(r, red[k]) : r + red[k];
    return r;
}

// One workgroup per query head: scores q.k_t * scale for t < length, a
// softmax over them, out = sum_t p_t v_t (backend/core/llm_cpu.c:491-511):
// each score and each output element sums in the reference's order; the
// maximum and the softmax denominator are reduced over the workgroup.
// keys / values: [position][kv_heads * width] of one layer.
__global__ __launch_bounds__(256) void attention(const float *__restrict__ q, const float *__restrict__ keys,
    const float *__restrict__ values, float *__restrict__ out, float *__restrict__ scores, int heads, int kv_heads,
    int width, int length, float scale)
{
    __shared__ float red[4];
    const int head = blockIdx.x, kvh = head / (heads / kv_heads), kvdim = kv_heads * width, t0 = threadIdx.x;
    const float *qh = q + (size_t)head * width;
    float *sc = scores + (size_t)head * length;
    float m = -INFINITY;
    for (int t = t0; t < length; t += 256) {
        const float *k = keys + (size_t)t * kvdim + kvh * width;
        float s = 0.f;
        for (int j = 0; j < width; ++j) s += qh[j] * k[j];
        s = s * scale;
        sc[t] = s;
        m = fmaxf(m, s);
    }
    m = block_reduce(m, red, true);
    float sum = 0.f;
    for (int t = t0; t < length; t += 256) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    __syncthreads();   // every score of this head written before any is read
    for (int t = t0; t < length; t += 256) sc[t] = sc[t] / sum;
    __syncthreads();
    for (int j = t0; j < width; j += 256) {
        float acc = 0.f;
        for (int t = 0; t < length; ++t) acc += sc[t] * values[(size_t)t * kvdim + kvh * width + j];
        out[(size_t)head * width + j] = acc;
    }
}

// gate = silu(gate) * up, silu(x) = x / (1 + e^-x) (backend/core/llm_cpu.c:336-341).
__global__ __launch_bounds__(256) void silu_mul(float *__restrict__ gate, const float *__restrict__ up, int n)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const float x = gate[i];
        gate[i] = x / (1.0f + expf(-x)) * up[i];
    }
}

__global__ __launch_bounds__(256) void add(float *__restrict__ x, const float *__restrict__ r, int n)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) x[i] = x[i] + r[i];
}

unsigned grid_of(long n) { return (unsigned)(n < 256 * 1024 ? (n + 255) / 256 : 1024); }

}  // namespace

hipError_t launch_dequant_row(const uint8_t *w, unsigned type, size_t row_bytes, size_t row, int cols, float *out,
    hipStream_t s)
{
    hipLaunchKernelGGL(dequant_row, dim3(grid_of(cols)), dim3(256), 0, s, w, type, row_bytes, row, cols, out);
    return hipGetLastError();
}

hipError_t launch_rms_norm(float *x, const float *r, const float *w, float *out, int n, float eps, hipStream_t s)
{
    hipLaunchKernelGGL(rms_norm, dim3(1), dim3(1024), 0, s, x, r, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope(float *v, int heads, int width, const float *freq, int position, hipStream_t s)
{
    hipLaunchKernelGGL(rope, dim3(grid_of((long)heads * (width / 2))), dim3(256), 0, s, v, heads, width, freq,
                       position);
    return hipGetLastError();
}

hipError_t launch_attention(const float *q, const float *keys, const float *values, float *out, float *scores,
    int heads, int kv_heads, int width, int length, float scale, hipStream_t s)
{
    hipLaunchKernelGGL(attention, dim3((unsigned)heads), dim3(256), 0, s, q, keys, values, out, scores, heads,
                       kv_heads, width, length, scale);
    return hipGetLastError();
}

hipError_t launch_silu_mul(float *gate, const float *up, int n, hipStream_t s)
{
    hipLaunchKernelGGL(silu_mul, dim3(grid_of(n)), dim3(256), 0, s, gate, up, n);
    return hipGetLastError();
}

hipError_t launch_add(float *x, const float *r, int n, hipStream_t s)
{
    hipLaunchKernelGGL(add, dim3(grid_of(n)), dim3(256), 0, s, x, r, n);
    return hipGetLastError();
}

}  // namespace fy
