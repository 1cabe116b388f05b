// The vector operations of one decoder token kept on the device (the resident
// plan of the ROCm provider): the embedding row, RMS normalization with the
// residual add folded in, rotary position encoding with the KV cache store,
// causal attention over the KV cache and the gated SiLU. Each restates one step of the engine's CPU token forward
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

// One workgroup of 1024 holding n <= 4096 K elements in registers (K float4
// per thread; x, r and w all loaded before the first use). x += r first when
// r is given (written back); then out = x * scale * w with
// scale = 1 / sqrt(sum x^2 / n + eps), the sum of squares in double
// (backend/core/llm_cpu.c:83-104; the order of the sum differs from the
// reference's sequential one, in double either way).
template <int K>
__global__ __launch_bounds__(1024) void rms_norm_regs(float4 *__restrict__ x, const float4 *__restrict__ r,
    const float4 *__restrict__ w, float4 *__restrict__ out, int n4, float eps)
{
    __shared__ double part[16];
    const int t = threadIdx.x;
    float4 v[K], u[K], g[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = t + 1024 * k;
        const bool in = i < n4;
        v[k] = in ? x[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        u[k] = in && r ? r[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        g[k] = in && w ? w[i] : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = t + 1024 * k;
        if (r) {
            v[k] = make_float4(v[k].x + u[k].x, v[k].y + u[k].y, v[k].z + u[k].z, v[k].w + u[k].w);
            if (i < n4) x[i] = v[k];
        }
        s += (double)v[k].x * v[k].x + (double)v[k].y * v[k].y + (double)v[k].z * v[k].z +
             (double)v[k].w * v[k].w;
    }
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    double total = part[0];
#pragma unroll
    for (int q = 1; q < 16; ++q) total += part[q];
    const float scale = (float)(1.0 / sqrt(total / (double)(4 * n4) + (double)eps));
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = t + 1024 * k;
        if (i < n4)
            out[i] = make_float4(v[k].x * scale * g[k].x, v[k].y * scale * g[k].y, v[k].z * scale * g[k].z,
                                 v[k].w * scale * g[k].w);
    }
}

// The same for any n and alignment: one workgroup of 256.
__global__ __launch_bounds__(256) void rms_norm(float *__restrict__ x, const float *__restrict__ r,
    const float *__restrict__ w, float *__restrict__ out, int n, float eps, bool vector4)
{
    __shared__ double part[4];
    const int t = threadIdx.x;
    double s = 0.0;
    if (vector4) {
        float4 *x4 = (float4 *)x;
        const float4 *r4 = (const float4 *)r;
        for (int i = t; i < n / 4; i += 256) {
            float4 v = x4[i];
            if (r) {
                const float4 u = r4[i];
                v = make_float4(v.x + u.x, v.y + u.y, v.z + u.z, v.w + u.w);
                x4[i] = v;
            }
            s += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
        }
    } else {
        for (int i = t; i < n; i += 256) {
            float v = x[i];
            if (r) {
                v = v + r[i];
                x[i] = v;
            }
            s += (double)v * v;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    const double total = part[0] + part[1] + part[2] + part[3];
    const float scale = (float)(1.0 / sqrt(total / (double)n + (double)eps));
    for (int i = t; i < n; i += 256) out[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

// The rotary step of one token on the fused q|k|v product (q: heads * width,
// then k and v: kv_heads * width each): every interleaved pair of q rotated
// in place and of k rotated into the key cache slot, by angle
// position * freq[j] (backend/core/llm_cpu.c:298-324, angles :429-432); v
// copied into the value cache slot.
__global__ __launch_bounds__(256) void rope_qkv(float *__restrict__ qkv, int heads, int kv_heads, int width,
    const float *__restrict__ freq, int position, float *__restrict__ key, float *__restrict__ value)
{
    const int pairs = width / 2, qn = heads * pairs, kn = kv_heads * pairs, vn = kv_heads * width;
    const float *v_in = qkv + (size_t)(heads + kv_heads) * width;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < qn + kn + vn; i += gridDim.x * 256) {
        if (i < qn + kn) {
            const bool is_q = i < qn;
            const int e = is_q ? i : i - qn, h = e / pairs, j = e % pairs;
            const float angle = (float)position * freq[j];
            const float c = cosf(angle), s = sinf(angle);
            const float *src = qkv + (is_q ? 0 : (size_t)heads * width) + (size_t)h * width + 2 * j;
            float *dst = (is_q ? qkv : key) + (size_t)h * width + 2 * j;
            const float a = src[0], b = src[1];
            dst[0] = a * c - b * s;
            dst[1] = a * s + b * c;
        } else {
            const int e = i - qn - kn;
            value[e] = v_in[e];
        }
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

constexpr int kLdsScores = 8192;   // scores kept in LDS up to this length
constexpr int kMaxWidth = 256;     // head width limit of the attention kernel

// One workgroup per query head, head width W (64, 128 or 256; q, keys and
// values 16-byte aligned): scores q.k_t * scale for t < length, a softmax
// over them, out = sum_t p_t v_t (backend/core/llm_cpu.c:491-511).
// Scores: 16 lanes per key row, lane l16 holding float4 columns
// l16 + 16 c of q and of the row; 64 rows in flight per workgroup (four per
// 16 lanes), reduced across the 16 lanes. p_t = e^(s_t - max) / sum as in
// the reference. Output: thread (g, c) sums float4 column c over
// t = g, g + G, ... (G = 1024 / W groups), then the groups add up in order.
// Scores in LDS up to kLdsScores positions, else in the [heads][length]
// global scratch.
template <int W, bool LDS>
__global__ __launch_bounds__(256) void attention_w(const float *__restrict__ q, const float *__restrict__ keys,
    const float *__restrict__ values, float *__restrict__ out, float *__restrict__ scores, int heads, int kv_heads,
    int length, float scale)
{
    constexpr int C = W / 64;            // float4 per lane per row
    constexpr int U = 4;                 // rows per 16 lanes in flight
    constexpr int G = 1024 / W;          // output groups of t (W / 4 float4 columns each)
    __shared__ float lds_scores[LDS ? kLdsScores : 1];
    __shared__ float4 part[256];
    __shared__ float red[4];
    const int tid = threadIdx.x, head = blockIdx.x, kvh = head / (heads / kv_heads);
    const int kv4 = kv_heads * (W / 4);  // float4 per cached position
    float *sc = LDS ? lds_scores : scores + (size_t)head * length;
    const int l16 = tid & 15, row = tid >> 4;
    const float4 *q4 = (const float4 *)q + (size_t)head * (W / 4);
    float4 qr[C];
#pragma unroll
    for (int c = 0; c < C; ++c) qr[c] = q4[l16 + 16 * c];
    const float4 *k4 = (const float4 *)keys + (size_t)kvh * (W / 4);
    float m = -INFINITY;
    for (int t0 = 0; t0 < length; t0 += 16 * U) {
        float4 kr[U][C];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + 16 * u + row;
            const int tt = t < length ? t : length - 1;
#pragma unroll
            for (int c = 0; c < C; ++c) kr[u][c] = k4[(size_t)tt * kv4 + l16 + 16 * c];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float s = 0.f;
#pragma unroll
            for (int c = 0; c < C; ++c)
                s += qr[c].x * kr[u][c].x + qr[c].y * kr[u][c].y + qr[c].z * kr[u][c].z + qr[c].w * kr[u][c].w;
            for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 16);
            const int t = t0 + 16 * u + row;
            if (t < length) {
                s = s * scale;
                if (l16 == 0) sc[t] = s;
                m = fmaxf(m, s);
            }
        }
    }
    m = block_reduce(m, red, true);
    __syncthreads();   // every score written before any thread reads one
    float sum = 0.f;
    for (int t = tid; t < length; t += 256) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    for (int t = tid; t < length; t += 256) sc[t] = sc[t] / sum;
    __syncthreads();
    const int c = tid % (W / 4), g = tid / (W / 4);
    const float4 *v4 = (const float4 *)values + (size_t)kvh * (W / 4) + c;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int t0 = g; t0 < length; t0 += 4 * G) {
        float4 vr[4];
        float p[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int t = t0 + G * u, tt = t < length ? t : length - 1;
            vr[u] = v4[(size_t)tt * kv4];
            p[u] = t < length ? sc[tt] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            acc.x += p[u] * vr[u].x;
            acc.y += p[u] * vr[u].y;
            acc.z += p[u] * vr[u].z;
            acc.w += p[u] * vr[u].w;
        }
    }
    part[tid] = acc;
    __syncthreads();
    if (tid < W / 4) {
        float4 o = part[tid];
#pragma unroll
        for (int k = 1; k < G; ++k) {
            const float4 b = part[k * (W / 4) + tid];
            o = make_float4(o.x + b.x, o.y + b.y, o.z + b.z, o.w + b.w);
        }
        ((float4 *)out)[(size_t)head * (W / 4) + tid] = o;
    }
}

// The same for any even width up to kMaxWidth and any 4-byte alignment:
// one workgroup per query head. Scores: 16 lanes per key row (a wave takes four rows at once, lanes
// striding the width), reduced across the 16; p_t = e^(s_t - max) / sum as in
// the reference. Output: 256 / width groups of threads each sum a strided
// share of t per element, then the groups add up. keys / values:
// [position][kv_heads * width] of one layer; scores in LDS, or in the
// [heads][length] global scratch beyond kLdsScores.
template <bool LDS>
__global__ __launch_bounds__(256) void attention(const float *__restrict__ q, const float *__restrict__ keys,
    const float *__restrict__ values, float *__restrict__ out, float *__restrict__ scores, int heads, int kv_heads,
    int width, int length, float scale)
{
    __shared__ float lds_scores[LDS ? kLdsScores : 1];
    __shared__ float qs[kMaxWidth];
    __shared__ float part[256];
    __shared__ float red[4];
    const int tid = threadIdx.x, head = blockIdx.x, kvh = head / (heads / kv_heads);
    const size_t kvdim = (size_t)kv_heads * width;
    float *sc = LDS ? lds_scores : scores + (size_t)head * length;
    for (int j = tid; j < width; j += 256) qs[j] = q[(size_t)head * width + j];
    __syncthreads();
    const int l16 = tid & 15, row = tid >> 4;   // 16 rows in flight per workgroup
    const float *kb = keys + (size_t)kvh * width;
    float m = -INFINITY;
    for (int t0 = 0; t0 < length; t0 += 16) {
        const int t = t0 + row;
        float s = 0.f;
        if (t < length) {
            const float *kr = kb + (size_t)t * kvdim;
            for (int j = l16; j < width; j += 16) s += qs[j] * kr[j];
        }
        for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 16);
        if (t < length) {
            s = s * scale;
            if (l16 == 0) sc[t] = s;
            m = fmaxf(m, s);
        }
    }
    m = block_reduce(m, red, true);
    float sum = 0.f;
    __syncthreads();   // every score written before any thread reads one
    for (int t = tid; t < length; t += 256) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        sum += e;
    }
    sum = block_reduce(sum, red, false);
    for (int t = tid; t < length; t += 256) sc[t] = sc[t] / sum;
    __syncthreads();
    const int groups = 256 / width, g = tid / width, j = tid % width;
    if (g < groups) {
        const float *vb = values + (size_t)kvh * width + j;
        float acc = 0.f;
        for (int t = g; t < length; t += groups) acc += sc[t] * vb[(size_t)t * kvdim];
        part[tid] = acc;
    }
    __syncthreads();
    if (tid < width) {
        float acc = part[tid];
        for (int k = 1; k < groups; ++k) acc += part[k * width + tid];
        out[(size_t)head * width + tid] = acc;
    }
}

// gate = silu(gate) * up, silu(x) = x / (1 + e^-x) (backend/core/llm_cpu.c:336-341):
// four elements per thread (16-byte aligned, n a multiple of 4), else one.
__device__ __forceinline__ float silu_times(float x, float u) { return x / (1.0f + expf(-x)) * u; }

__global__ __launch_bounds__(256) void silu_mul4(float4 *__restrict__ gate, const float4 *__restrict__ up, int n4)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n4; i += gridDim.x * 256) {
        const float4 g = gate[i], u = up[i];
        gate[i] = make_float4(silu_times(g.x, u.x), silu_times(g.y, u.y), silu_times(g.z, u.z), silu_times(g.w, u.w));
    }
}

__global__ __launch_bounds__(256) void silu_mul(float *__restrict__ gate, const float *__restrict__ up, int n)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        gate[i] = silu_times(gate[i], up[i]);
    }
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
    const bool vector4 = (n & 3) == 0 && (((uintptr_t)x | (uintptr_t)r) & 15u) == 0;
    const bool regs = vector4 && (((uintptr_t)w | (uintptr_t)out) & 15u) == 0 && n <= 4 * 4096;
    const int n4 = n / 4;
    if (regs && n4 <= 1024)
        hipLaunchKernelGGL(rms_norm_regs<1>, dim3(1), dim3(1024), 0, s, (float4 *)x, (const float4 *)r,
                           (const float4 *)w, (float4 *)out, n4, eps);
    else if (regs && n4 <= 2048)
        hipLaunchKernelGGL(rms_norm_regs<2>, dim3(1), dim3(1024), 0, s, (float4 *)x, (const float4 *)r,
                           (const float4 *)w, (float4 *)out, n4, eps);
    else if (regs)
        hipLaunchKernelGGL(rms_norm_regs<4>, dim3(1), dim3(1024), 0, s, (float4 *)x, (const float4 *)r,
                           (const float4 *)w, (float4 *)out, n4, eps);
    else
        hipLaunchKernelGGL(rms_norm, dim3(1), dim3(256), 0, s, x, r, w, out, n, eps, vector4);
    return hipGetLastError();
}

hipError_t launch_rope_qkv(float *qkv, int heads, int kv_heads, int width, const float *freq, int position, float *key,
    float *value, hipStream_t s)
{
    const long n = (long)(heads + kv_heads) * (width / 2) + (long)kv_heads * width;
    hipLaunchKernelGGL(rope_qkv, dim3(grid_of(n)), dim3(256), 0, s, qkv, heads, kv_heads, width, freq, position, key,
                       value);
    return hipGetLastError();
}

template <int W>
void launch_attention_w(const float *q, const float *keys, const float *values, float *out, float *scores, int heads,
    int kv_heads, int length, float scale, hipStream_t s)
{
    if (length <= kLdsScores)
        hipLaunchKernelGGL((attention_w<W, true>), dim3((unsigned)heads), dim3(256), 0, s, q, keys, values, out, scores,
                           heads, kv_heads, length, scale);
    else
        hipLaunchKernelGGL((attention_w<W, false>), dim3((unsigned)heads), dim3(256), 0, s, q, keys, values, out,
                           scores, heads, kv_heads, length, scale);
}

hipError_t launch_attention(const float *q, const float *keys, const float *values, float *out, float *scores,
    int heads, int kv_heads, int width, int length, float scale, hipStream_t s)
{
    if (width > kMaxWidth) return hipErrorInvalidValue;
    const bool aligned = (((uintptr_t)q | (uintptr_t)keys | (uintptr_t)values | (uintptr_t)out) & 15u) == 0;
    if (aligned && width == 128)
        launch_attention_w<128>(q, keys, values, out, scores, heads, kv_heads, length, scale, s);
    else if (aligned && width == 64)
        launch_attention_w<64>(q, keys, values, out, scores, heads, kv_heads, length, scale, s);
    else if (aligned && width == 256)
        launch_attention_w<256>(q, keys, values, out, scores, heads, kv_heads, length, scale, s);
    else if (length <= kLdsScores)
        hipLaunchKernelGGL(attention<true>, dim3((unsigned)heads), dim3(256), 0, s, q, keys, values, out, scores,
                           heads, kv_heads, width, length, scale);
    else
        hipLaunchKernelGGL(attention<false>, dim3((unsigned)heads), dim3(256), 0, s, q, keys, values, out, scores,
                           heads, kv_heads, width, length, scale);
    return hipGetLastError();
}

hipError_t launch_silu_mul(float *gate, const float *up, int n, hipStream_t s)
{
    if ((n & 3) == 0 && (((uintptr_t)gate | (uintptr_t)up) & 15u) == 0)
        hipLaunchKernelGGL(silu_mul4, dim3(grid_of(n / 4)), dim3(256), 0, s, (float4 *)gate, (const float4 *)up, n / 4);
    else
        hipLaunchKernelGGL(silu_mul, dim3(grid_of(n)), dim3(256), 0, s, gate, up, n);
    return hipGetLastError();
}

}  // namespace fy
