// The vector operations of the decoder kept on the device (the resident
// plan of the ROCm provider), each over `count` tokens at once (one token
// when decoding, a prompt chunk when prefilling): the embedding rows, RMS
// normalization with the residual add folded in (through the branch's post
// norm for Gemma), rotary position encoding with the KV cache store (after
// per-head norms for Gemma), causal attention over the KV cache (with a
// local window), the gated SiLU or GELU and the logit soft cap. Each
// restates one step of the engine's CPU token forward
// (backend/core/llm_cpu.c:424-578, LLaMA and Gemma branches) with the same operation
// order per element where the step is elementwise; arithmetic is not
// contracted into fused multiply-adds (the reference's C17 build does not
// contract either). The matrix products between them are the library's
// quantized kernels. Token ids and positions are device arrays, so one
// sequence of launches serves any token (and can be recorded once).
#include <math.h>

#include "device.h"
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

// out[i][c] = element c of row tokens[i] times scale (a token past the
// matrix gives a zero row; the host checks ids first).
__global__ __launch_bounds__(256) void embed(const uint8_t *__restrict__ w, unsigned type, size_t row_bytes,
    int rows, const uint32_t *__restrict__ tokens, int cols, float *__restrict__ out, float scale)
{
    const uint32_t token = tokens[blockIdx.y];
    float *o = out + (size_t)blockIdx.y * cols;
    const uint8_t *r = w + (size_t)token * row_bytes;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < cols; i += gridDim.x * 256)
        o[i] = token < (uint32_t)rows ? element(r, type, i) * scale : 0.f;
}

// One workgroup of 1024 per row (token), holding n <= 4096 K elements in
// registers (K float4 per thread; x, r and w all loaded before the first
// use). x += r first when r is given (written back); then
// out = x * scale * w with scale = 1 / sqrt(sum x^2 / n + eps), the sum of
// squares in double (backend/core/llm_cpu.c:83-104; the order of the sum
// differs from the reference's sequential one, in double either way).
template <int K>
__global__ __launch_bounds__(1024) void rms_norm_regs(float4 *__restrict__ x, const float4 *__restrict__ r,
    const float4 *__restrict__ w, float4 *__restrict__ out, int n4, float eps)
{
    __shared__ double part[16];
    const int t = threadIdx.x;
    const size_t row = (size_t)blockIdx.x * n4;
    x += row;
    out += row;
    if (r) r += row;
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
    s = wave_sum(s);
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

// The same for any n and alignment: one workgroup of 256 per row.
__global__ __launch_bounds__(256) void rms_norm(float *__restrict__ x, const float *__restrict__ r,
    const float *__restrict__ w, float *__restrict__ out, int n, float eps)
{
    __shared__ double part[4];
    const int t = threadIdx.x;
    const size_t row = (size_t)blockIdx.x * n;
    x += row;
    out += row;
    if (r) r += row;
    double s = 0.0;
    for (int i = t; i < n; i += 256) {
        float v = x[i];
        if (r) {
            v = v + r[i];
            x[i] = v;
        }
        s += (double)v * v;
    }
    s = wave_sum(s);
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    const double total = part[0] + part[1] + part[2] + part[3];
    const float scale = (float)(1.0 / sqrt(total / (double)n + (double)eps));
    for (int i = t; i < n; i += 256) out[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

// Sum of one double per thread over a workgroup of 64 N threads, the same
// value in every thread: each wavefront's sum (wave_sum), then the
// wavefronts' sums added in order.
template <int N>
__device__ __forceinline__ double group_sum(double s, double *part)
{
    s = wave_sum(s);
    __syncthreads();   // an earlier call's reads of part are done
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    double total = part[0];
#pragma unroll
    for (int q = 1; q < N; ++q) total += part[q];
    return total;
}

// The residual add of a block whose branch output carries its own norm
// (the engine's Gemma post-attention and post-feed-forward norms,
// backend/core/llm_cpu.c:514, :531): per token row of n <= 1024 K elements,
// r' = r * s_r * post (r's RMS scale, the sum of squares in double; post
// null: r' = r), x = (x + r') * oscale written back (the block's output
// scale, :544-547; 1 elsewhere), then out = x * s_x * w as the norm step
// (:83-104). Elements in registers, K per thread; r is not written.
template <int K>
__global__ __launch_bounds__(1024) void post_norm(float *__restrict__ x, const float *__restrict__ r,
    const float *__restrict__ post, float oscale, const float *__restrict__ w, float *__restrict__ out, int n,
    float eps)
{
    __shared__ double part[16];
    const int t = threadIdx.x;
    const size_t row = (size_t)blockIdx.x * n;
    x += row;
    out += row;
    if (r) r += row;
    // Every input loaded before the first use: one memory round trip.
    float v[K], u[K], pw[K], g[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = t + 1024 * k;
        v[k] = i < n ? x[i] : 0.f;
        u[k] = i < n && r ? r[i] : 0.f;
        pw[k] = i < n && post ? post[i] : 1.f;
        g[k] = i < n && w ? w[i] : 1.f;
    }
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) s += (double)u[k] * u[k];
    if (r && post) {
        const float sr = (float)(1.0 / sqrt(group_sum<16>(s, part) / (double)n + (double)eps));
#pragma unroll
        for (int k = 0; k < K; ++k) u[k] = u[k] * sr * pw[k];
    }
    s = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = t + 1024 * k;
        if (i < n) {
            if (r) v[k] = v[k] + u[k];
            v[k] = v[k] * oscale;
            x[i] = v[k];
        }
        s += (double)v[k] * v[k];
    }
    const float sx = (float)(1.0 / sqrt(group_sum<16>(s, part) / (double)n + (double)eps));
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = t + 1024 * k;
        if (i < n) out[i] = v[k] * sx * g[k];
    }
}

constexpr int kHeadWidthMax = 512;   // head width limit of head_norm_rope (two elements per thread)

// The query and key steps of the engine's Gemma attention
// (backend/core/llm_cpu.c:487-500): workgroup (head, token i) takes one head
// of width <= 512, elements j and j + 256 in thread j. Heads [0, heads) are q heads (q
// + i q_stride, normalized in place with q_norm, then rotated); with k,
// heads [heads, heads + kv_heads) are k heads (normalized with k_norm,
// rotated, into the key cache slot of positions[i]) and the next kv_heads
// are v heads (normalized without a weight, into the value cache slot; v may
// be k itself, the engine's copy of the key for layers without a value
// matrix). The norm is the engine's RMS norm per head (:360-363, :83-104);
// the rotation turns the pair (j, j + width / 2) by position * freq[j]
// (:345-358, angles :429-432). A position outside [0, capacity) leaves
// everything alone (the host checks first).
__global__ __launch_bounds__(256) void head_norm_rope(float *__restrict__ q, int q_stride,
    const float *__restrict__ k, int k_stride, const float *__restrict__ v, int v_stride, int heads, int kv_heads,
    int width, const float *__restrict__ q_norm, const float *__restrict__ k_norm, float eps,
    const float *__restrict__ freq, const int *__restrict__ positions, int capacity, float *__restrict__ keys,
    float *__restrict__ values)
{
    __shared__ double part[4];
    __shared__ float row[kHeadWidthMax];
    const int h = blockIdx.x, j = threadIdx.x, half = width / 2;
    const int kind = h < heads ? 0 : h < heads + kv_heads ? 1 : 2;   // q, k, v
    const int hh = kind == 0 ? h : kind == 1 ? h - heads : h - heads - kv_heads;
    const float *src = kind == 0 ? q + (size_t)blockIdx.y * q_stride + (size_t)hh * width
                     : kind == 1 ? k + (size_t)blockIdx.y * k_stride + (size_t)hh * width
                                 : v + (size_t)blockIdx.y * v_stride + (size_t)hh * width;
    const float *g = kind == 0 ? q_norm : kind == 1 ? k_norm : nullptr;
    const int j1 = j + 256;
    // Every load first (none depends on the position; only where k and v
    // go does), then the position: one memory round trip, not three.
    const float x0 = j < width ? src[j] : 0.f, x1 = j1 < width ? src[j1] : 0.f;
    const float g0 = g && j < width ? g[j] : 1.0f, g1 = g && j1 < width ? g[j1] : 1.0f;
    const float f = kind != 2 && j < half ? freq[j] : 0.f;
    __builtin_amdgcn_sched_barrier(0);
    const int position = positions[blockIdx.y];
    const bool stored = position >= 0 && position < capacity;   // else nothing is written
    const size_t slot = (size_t)(stored ? position : 0) * kv_heads * width + (size_t)hh * width;
    float *dst = kind == 0 ? q + (size_t)blockIdx.y * q_stride + (size_t)hh * width
               : kind == 1 ? keys + slot : values + slot;
    const double sq = (double)x0 * x0 + (double)x1 * x1;
    const float scale = (float)(1.0 / sqrt(group_sum<4>(sq, part) / (double)width + (double)eps));
    const float y0 = x0 * scale * g0;
    const float y1 = x1 * scale * g1;
    if (kind == 2) {
        if (stored && j < width) dst[j] = y0;
        if (stored && j1 < width) dst[j1] = y1;
        return;
    }
    // q in place: every element was read before group_sum's barriers.
    if (j < width) row[j] = y0;
    if (j1 < width) row[j1] = y1;
    __syncthreads();
    if (stored && j < half) {
        const float angle = (float)position * f;
        const float c = cosf(angle), s = sinf(angle);
        const float a = row[j], b = row[j + half];
        dst[j] = a * c - b * s;
        dst[j + half] = b * c + a * s;
    }
}

// Logits squashed as the engine's final soft cap (backend/core/llm_cpu.c:
// 562-565): x = cap * tanh(x / cap).
__global__ __launch_bounds__(256) void softcap(float *__restrict__ x, size_t n, float cap)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        x[i] = cap * tanhf(x[i] / cap);
}

// The rotary step of token i = blockIdx.y at position positions[i]: its q
// row (q + i q_stride, heads * width) rotated in place and its k row
// (k + i k_stride, kv_heads * width) rotated into the key cache slot
// keys + position * kv_heads * width, every interleaved pair by angle
// position * freq[j] (backend/core/llm_cpu.c:298-324, angles :429-432); its
// v row copied into the value cache slot. A position outside
// [0, capacity) leaves the rows and the cache alone (the host checks
// first).
__global__ __launch_bounds__(256) void rope_qkv(float *__restrict__ q, int q_stride, const float *__restrict__ k,
    int k_stride, const float *__restrict__ v, int v_stride, int heads, int kv_heads, int width,
    const float *__restrict__ freq, const int *__restrict__ positions, int capacity, float *__restrict__ keys,
    float *__restrict__ values)
{
    const int position = positions[blockIdx.y];
    if (position < 0 || position >= capacity) return;
    const int pairs = width / 2, qn = heads * pairs, kn = kv_heads * pairs, vn = kv_heads * width;
    float *qr = q + (size_t)blockIdx.y * q_stride;
    const float *kr = k + (size_t)blockIdx.y * k_stride, *vr = v + (size_t)blockIdx.y * v_stride;
    float *key = keys + (size_t)position * vn, *value = values + (size_t)position * vn;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < qn + kn + vn; i += gridDim.x * 256) {
        if (i < qn + kn) {
            const bool is_q = i < qn;
            const int e = is_q ? i : i - qn, h = e / pairs, j = e % pairs;
            const float angle = (float)position * freq[j];
            const float c = cosf(angle), s = sinf(angle);
            const float *src = (is_q ? qr : kr) + (size_t)h * width + 2 * j;
            float *dst = (is_q ? qr : key) + (size_t)h * width + 2 * j;
            const float a = src[0], b = src[1];
            dst[0] = a * c - b * s;
            dst[1] = a * s + b * c;
        } else {
            const int e = i - qn - kn;
            value[e] = vr[e];
        }
    }
}

__device__ __forceinline__ float block_reduce(float v, float *red, bool maximum)
{
    v = maximum ? wave_reduce<true>(v) : wave_reduce<false>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int k = 1; k < 4; ++k) r = maximum ? fmaxf(r, red[k]) : r + red[k];
    return r;
}

constexpr int kLdsScores = 8192;   // scores kept in LDS up to this length
constexpr int kMaxWidth = 512;     // head width limit of the attention kernels

// The cached positions [first, first + length) that a token at position p
// attends: [0, p] clamped to max_length, and with a local window of
// `window` positions (0: none) the last `window` of them, as the engine
// bounds a sliding layer's attention (backend/core/llm_cpu.c:486-488).
struct CausalRange {
    int first, length;
};

__device__ __forceinline__ CausalRange causal_range(int p, int max_length, int window)
{
    const int end = p < 0 ? -1 : p >= max_length ? max_length - 1 : p;
    const int first = window > 0 && end >= window ? end - window + 1 : 0;
    return {first, end < 0 ? 0 : end - first + 1};
}

// Attention of query token i = blockIdx.y, head blockIdx.x, over its
// causal range: its q at q + i * q_stride + head * W, its output at
// out + (i * heads + head) * W.
struct AttentionRow {
    int head, kvh, first, length;
    size_t q, out, scores;
};

__device__ __forceinline__ AttentionRow attention_row(const int *positions, int heads, int kv_heads, int width,
    int q_stride, int max_length, int window)
{
    AttentionRow a;
    a.head = blockIdx.x;
    a.kvh = a.head / (heads / kv_heads);
    const CausalRange r = causal_range(positions[blockIdx.y], max_length, window);
    a.first = r.first;
    a.length = r.length;
    a.q = (size_t)blockIdx.y * q_stride + (size_t)a.head * width;
    a.out = ((size_t)blockIdx.y * heads + a.head) * width;
    a.scores = ((size_t)blockIdx.y * heads + a.head) * max_length;
    return a;
}

// Head width W (64, 128, 256 or 512; q, keys, values and out 16-byte aligned):
// scores q.k_t * scale for t < length, a softmax over them,
// out = sum_t p_t v_t (backend/core/llm_cpu.c:491-511). Scores: 16 lanes per
// key row, lane l16 holding float4 columns l16 + 16 c of q and of the row;
// 64 rows in flight per workgroup (four per 16 lanes), reduced across the
// 16 lanes. p_t = e^(s_t - max) / sum as in the reference. Output: thread
// (g, c) sums float4 column c over t = g, g + G, ... (G = 1024 / W groups),
// then the groups add up in order. Scores in LDS (LDS: max_length <=
// kLdsScores), else in the global scratch [count][heads][max_length].
//
// Without a window (WIN false) the causal range starts at row 0, so q, the
// first U key rows per 16 lanes and the first VU value rows per thread are
// requested before the token's position is known: rows up to max_length - 1
// (inside the cache), whatever the range. Rows past the range only feed
// scores that are never kept and values that are replaced by zeros before
// they are weighed (they may hold anything, NaN included). With a window the
// first row depends on the position, which is read first.
template <int W, bool LDS, bool WIN>
__global__ __launch_bounds__(256) void attention_w(const float *__restrict__ q, int q_stride,
    const float *__restrict__ keys, const float *__restrict__ values, float *__restrict__ out,
    float *__restrict__ scores, const int *__restrict__ positions, int heads, int kv_heads, int max_length,
    int window, float scale)
{
    constexpr int C = W / 64;            // float4 per lane per row
    constexpr int U = W <= 128 ? 8 : W <= 256 ? 4 : 2;  // rows per 16 lanes in flight
    constexpr int G = 1024 / W;          // output groups of t (W / 4 float4 columns each)
    constexpr int VU = 8;                // V rows per thread in flight
    __shared__ float lds_scores[LDS ? kLdsScores : 1];
    __shared__ float4 part[256];
    __shared__ float red[4];
    const int head = blockIdx.x, kvh = head / (heads / kv_heads), tid = threadIdx.x;
    const int l16 = tid & 15, row = tid >> 4;
    const int c = tid % (W / 4), g = tid / (W / 4);
    const float4 *q4 = (const float4 *)(q + (size_t)blockIdx.y * q_stride + (size_t)head * W);
    float4 qr[C];
#pragma unroll
    for (int k = 0; k < C; ++k) qr[k] = q4[l16 + 16 * k];
    CausalRange range = {0, 0};
    if constexpr (WIN) {
        range = causal_range(positions[blockIdx.y], max_length, window);
        if (range.length == 0) return;
    }
    // The rows loaded before the length is known: up to `last`.
    const int last = WIN ? range.length - 1 : max_length - 1;
    const int kv4 = kv_heads * (W / 4);  // float4 per cached position
    const float4 *k4 = (const float4 *)(keys + (size_t)range.first * kv_heads * W) + (size_t)kvh * (W / 4);
    // The output phase's first VU rows of this thread (rows g, g + G, ...,
    // column c), requested with the keys: V does not wait for the scores.
    const float4 *v4 = (const float4 *)(values + (size_t)range.first * kv_heads * W) + (size_t)kvh * (W / 4) + c;
    float4 vfirst[VU];
#pragma unroll
    for (int u = 0; u < VU; ++u) {
        const int t = g + G * u;
        vfirst[u] = v4[(size_t)(t < last ? t : last) * kv4];
    }
    float4 kr[U][C];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int t = 16 * u + row, tt = t < last ? t : last;
#pragma unroll
        for (int k = 0; k < C; ++k) kr[u][k] = k4[(size_t)tt * kv4 + l16 + 16 * k];
    }
    if constexpr (!WIN) {
        // Read after the loads above are issued (no return before them: a
        // token without positions skips the loops and the store below).
        __builtin_amdgcn_sched_barrier(0);
        range = causal_range(positions[blockIdx.y], max_length, 0);
    }
    const int length = range.length;
    float *sc = LDS ? lds_scores : scores + ((size_t)blockIdx.y * heads + head) * max_length;
    float m = -INFINITY;
    auto chunk_scores = [&](int t0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < C; ++k)
                s += qr[k].x * kr[u][k].x + qr[k].y * kr[u][k].y + qr[k].z * kr[u][k].z + qr[k].w * kr[u][k].w;
            s = row16_reduce<false>(s);
            const int t = t0 + 16 * u + row;
            if (t < length) {
                s = s * scale;
                if (l16 == 0) sc[t] = s;
                m = fmaxf(m, s);
            }
        }
    };
    // The first chunk whatever the length (its rows are loaded; a shorter
    // range keeps fewer of its scores), so its loads are not held behind a
    // test of the length.
    chunk_scores(0);
    for (int t0 = 16 * U; t0 < length; t0 += 16 * U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + 16 * u + row, tt = t < length ? t : length - 1;
#pragma unroll
            for (int k = 0; k < C; ++k) kr[u][k] = k4[(size_t)tt * kv4 + l16 + 16 * k];
        }
        chunk_scores(t0);
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
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int t0 = g; t0 < length; t0 += VU * G) {
        float4 vr[VU];
        float p[VU];
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int t = t0 + G * u, tt = t < length ? t : length - 1;
            vr[u] = t0 == g ? vfirst[u] : v4[(size_t)tt * kv4];
            if (t >= length) vr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            p[u] = t < length ? sc[tt] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            acc.x += p[u] * vr[u].x;
            acc.y += p[u] * vr[u].y;
            acc.z += p[u] * vr[u].z;
            acc.w += p[u] * vr[u].w;
        }
    }
    part[tid] = acc;
    __syncthreads();
    if (tid < W / 4 && length > 0) {
        float4 o = part[tid];
#pragma unroll
        for (int k = 1; k < G; ++k) {
            const float4 b = part[k * (W / 4) + tid];
            o = make_float4(o.x + b.x, o.y + b.y, o.z + b.z, o.w + b.w);
        }
        ((float4 *)(out + ((size_t)blockIdx.y * heads + head) * W))[tid] = o;
    }
}

// The same for any even width up to kMaxWidth and any 4-byte alignment.
// Scores: 16 lanes per key row (lanes striding the width), reduced across
// the 16. Output: up to width 256, 256 / width groups of threads each sum a
// strided share of t per element, then the groups add up; wider, one thread
// per element and every t.
template <bool LDS>
__global__ __launch_bounds__(256) void attention(const float *__restrict__ q, int q_stride,
    const float *__restrict__ keys, const float *__restrict__ values, float *__restrict__ out,
    float *__restrict__ scores, const int *__restrict__ positions, int heads, int kv_heads, int width,
    int max_length, int window, float scale)
{
    __shared__ float lds_scores[LDS ? kLdsScores : 1];
    __shared__ float qs[kMaxWidth];
    __shared__ float part[256];
    __shared__ float red[4];
    const AttentionRow a = attention_row(positions, heads, kv_heads, width, q_stride, max_length, window);
    const int tid = threadIdx.x, length = a.length;
    if (length == 0) return;
    const size_t kvdim = (size_t)kv_heads * width;
    keys += (size_t)a.first * kvdim;
    values += (size_t)a.first * kvdim;
    float *sc = LDS ? lds_scores : scores + a.scores;
    for (int j = tid; j < width; j += 256) qs[j] = q[a.q + j];
    __syncthreads();
    const int l16 = tid & 15, row = tid >> 4;   // 16 rows in flight per workgroup
    const float *kb = keys + (size_t)a.kvh * width;
    float m = -INFINITY;
    for (int t0 = 0; t0 < length; t0 += 16) {
        const int t = t0 + row;
        float s = 0.f;
        if (t < length) {
            const float *kr = kb + (size_t)t * kvdim;
            for (int j = l16; j < width; j += 16) s += qs[j] * kr[j];
        }
        s = row16_reduce<false>(s);
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
    if (width > 256) {
        // Wider heads: thread j sums columns j, j + 256 over every t in order.
        const float *vb = values + (size_t)a.kvh * width;
        for (int j = tid; j < width; j += 256) {
            float acc = 0.f;
            for (int t = 0; t < length; ++t) acc += sc[t] * vb[(size_t)t * kvdim + j];
            out[a.out + j] = acc;
        }
        return;
    }
    const int groups = 256 / width, g = tid / width, j = tid % width;
    if (g < groups) {
        const float *vb = values + (size_t)a.kvh * width + j;
        float acc = 0.f;
        for (int t = g; t < length; t += groups) acc += sc[t] * vb[(size_t)t * kvdim];
        part[tid] = acc;
    }
    __syncthreads();
    if (tid < width) {
        float acc = part[tid];
        for (int k = 1; k < groups; ++k) acc += part[k * width + tid];
        out[a.out + tid] = acc;
    }
}

// ---- attention split over the cached positions (long contexts) ------------
//
// One token's attention reads its KV head's whole history, and one
// workgroup per (query head, token) leaves most of the chip idle past a few
// hundred positions. Here workgroup (kv head, split s, token) takes the
// positions [s C, (s + 1) C) of the token's causal range (C = ceil(length /
// splits)) for all G query heads that share the KV head, so every cached K
// and V row is read once per token: per head g the chunk's scores
// q_g . k_t * scale, their maximum m, e_t = e^(s_t - m), l = sum e_t and
// o = sum e_t v_t, unnormalized (the engine's order within the chunk,
// backend/core/llm_cpu.c:491-511). attention_combine then forms
// out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s. A split
// past the range writes m = -inf, l = 0, o = 0. Partials: o at
// partials[((i heads + head) splits + s) W], m and l after all of them
// ([count][heads][splits][2]).
constexpr int kSplitMaxChunk = 1024;   // positions per split (scores in LDS)

template <int W, int G>
__global__ __launch_bounds__(256) void attention_split(const float *__restrict__ q, int q_stride,
    const float *__restrict__ keys, const float *__restrict__ values, float *__restrict__ partials,
    const int *__restrict__ positions, int heads, int kv_heads, int max_length, int window, int splits, float scale)
{
    constexpr int C = W / 64;          // float4 per lane per row
    constexpr int U = 4;               // rows per 16 lanes in flight
    constexpr int NG = 1024 / W;       // output groups of t (W / 4 float4 columns each)
    static_assert(NG * W <= kSplitMaxChunk, "the groups' partial outputs fit the scores' LDS");
    __shared__ __align__(16) float sc[G * kSplitMaxChunk];   // scores, then the groups' partial outputs
    const int kvh = blockIdx.x, sp = blockIdx.y, tok = blockIdx.z, tid = threadIdx.x;
    const CausalRange range = causal_range(positions[tok], max_length, window);
    const int length = range.length;
    keys += (size_t)range.first * kv_heads * W;
    values += (size_t)range.first * kv_heads * W;
    const int chunk = (length + splits - 1) / splits;
    const int c0 = sp * chunk, n = length - c0 < chunk ? length - c0 : chunk;
    const size_t base = ((size_t)tok * heads + (size_t)kvh * G) * splits + sp;   // partial row of head g: + g splits
    float *ml = partials + (size_t)gridDim.z * heads * splits * W;
    if (n <= 0) {
        // Nothing of the range here: an empty partial.
        for (int i = tid; i < G * W; i += 256) partials[(base + (size_t)(i / W) * splits) * W + i % W] = 0.f;
        if (tid < G) {
            ml[2 * (base + (size_t)tid * splits)] = -INFINITY;
            ml[2 * (base + (size_t)tid * splits) + 1] = 0.f;
        }
        return;
    }
    const int kv4 = kv_heads * (W / 4);
    const int l16 = tid & 15, row = tid >> 4;
    float4 qr[G][C];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float4 *q4 = (const float4 *)(q + (size_t)tok * q_stride + (size_t)(kvh * G + g) * W);
#pragma unroll
        for (int c = 0; c < C; ++c) qr[g][c] = q4[l16 + 16 * c];
    }
    const float4 *k4 = (const float4 *)keys + (size_t)kvh * (W / 4);
    // The output phase's first VU rows per thread (thread (group, float4
    // column) takes rows group, group + NG, ...), requested now: V does not
    // wait for the scores.
    constexpr int VU = 8;
    const int col = tid % (W / 4), grp = tid / (W / 4);
    const float4 *v4 = (const float4 *)values + (size_t)kvh * (W / 4) + col;
    float4 vfirst[VU];
#pragma unroll
    for (int u = 0; u < VU; ++u) {
        const int t = grp + NG * u;
        vfirst[u] = v4[(size_t)(c0 + (t < n ? t : n - 1)) * kv4];
    }
    for (int t0 = 0; t0 < n; t0 += 16 * U) {
        float4 kr[U][C];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + 16 * u + row, tt = c0 + (t < n ? t : n - 1);
#pragma unroll
            for (int c = 0; c < C; ++c) kr[u][c] = k4[(size_t)tt * kv4 + l16 + 16 * c];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + 16 * u + row;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float s = 0.f;
#pragma unroll
                for (int c = 0; c < C; ++c)
                    s += qr[g][c].x * kr[u][c].x + qr[g][c].y * kr[u][c].y + qr[g][c].z * kr[u][c].z +
                         qr[g][c].w * kr[u][c].w;
                s = row16_reduce<false>(s);
                if (t < n && l16 == 0) sc[g * kSplitMaxChunk + t] = s * scale;
            }
        }
    }
    __syncthreads();
    // Per head: maximum, e_t and their sum; wavefront w takes heads w, w + 4.
    __shared__ float mls[2 * G];
    const int lane = tid & 63, wave = tid >> 6;
    for (int g = wave; g < G; g += 4) {
        float *s = sc + g * kSplitMaxChunk;
        float m = -INFINITY;
        for (int t = lane; t < n; t += 64) m = fmaxf(m, s[t]);
        m = wave_reduce<true>(m);
        float sum = 0.f;
        for (int t = lane; t < n; t += 64) {
            const float e = expf(s[t] - m);
            s[t] = e;
            sum += e;
        }
        sum = wave_reduce<false>(sum);
        if (lane == 0) {
            mls[2 * g] = m;
            mls[2 * g + 1] = sum;
        }
    }
    __syncthreads();
    // o_g = sum_t e_t v_t: thread (group, float4 column) over t = group,
    // group + NG, ...; every V row is read once for all G heads. Eight rows
    // in flight per thread (each loop trip's loads issue before their first
    // use; the first trip's were requested with the keys); every thread
    // adds its rows in increasing t.
    float4 acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int t0 = grp; t0 < n; t0 += NG * VU) {
        float4 v[VU];
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int t = t0 + NG * u;
            v[u] = t0 == grp ? vfirst[u] : v4[(size_t)(c0 + (t < n ? t : n - 1)) * kv4];
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int t = t0 + NG * u;
            if (t >= n) break;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float e = sc[g * kSplitMaxChunk + t];
                acc[g].x += e * v[u].x;
                acc[g].y += e * v[u].y;
                acc[g].z += e * v[u].z;
                acc[g].w += e * v[u].w;
            }
        }
    }
    __syncthreads();   // the e_t are read; their LDS takes the groups' sums
    float4 *part = (float4 *)sc;   // [g][grp][W / 4]
#pragma unroll
    for (int g = 0; g < G; ++g) part[(g * NG + grp) * (W / 4) + col] = acc[g];
    __syncthreads();
    for (int i = tid; i < G * (W / 4); i += 256) {
        const int g = i / (W / 4), c = i % (W / 4);
        float4 o = part[(g * NG) * (W / 4) + c];
        for (int k = 1; k < NG; ++k) {
            const float4 b = part[(g * NG + k) * (W / 4) + c];
            o = make_float4(o.x + b.x, o.y + b.y, o.z + b.z, o.w + b.w);
        }
        ((float4 *)(partials + (base + (size_t)g * splits) * W))[c] = o;
    }
    if (tid < G) {
        ml[2 * (base + (size_t)tid * splits)] = mls[2 * tid];
        ml[2 * (base + (size_t)tid * splits) + 1] = mls[2 * tid + 1];
    }
}

constexpr int kCombineOnce = 64;   // splits whose partials one thread holds in registers

// out[i][head] from the `splits` partials of (token i, head): thread s <
// splits forms the split's weight f_s = e^(m_s - M) / L (M = max m, L =
// sum_s l_s e^(m_s - M), an empty split weighs 0), then thread j < width
// adds f_s o_s[j] over the splits in order, all their loads requested at
// once (splits <= 256; the ABI's larger counts run in rounds of 256).

template <bool WIDE>
__global__ __launch_bounds__(256) void attention_combine(const float *__restrict__ partials,
    float *__restrict__ out, const int *__restrict__ positions, int heads, int width, int max_length, int splits)
{
    __shared__ float f[256];
    __shared__ float red[8];
    const int head = blockIdx.x, tok = blockIdx.y, tid = threadIdx.x;
    if (positions[tok] < 0 || max_length <= 0) return;
    const size_t base = ((size_t)tok * heads + head) * splits;
    const float2 *ml = (const float2 *)(partials + (size_t)gridDim.y * heads * splits * width) + base;
    if (splits <= kCombineOnce) {
        // Up to kCombineOnce splits: every load at once (thread j's column of
        // every split with the splits' m and l), so the combination waits for
        // one memory round trip; the same arithmetic in the same order as the
        // rounds below.
        const float2 v = tid < splits ? ml[tid] : make_float2(-INFINITY, 0.f);
        const float *po = partials + base * width + (tid < width ? tid : width - 1);
        float pv[kCombineOnce];
#pragma unroll
        for (int u = 0; u < kCombineOnce; ++u) pv[u] = po[(size_t)(u < splits ? u : splits - 1) * width];
        float m = v.x;
        m = wave_reduce<true>(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float e = v.x == -INFINITY ? 0.f : expf(v.x - m);
        float l = v.y * e;
        l = wave_reduce<false>(l);
        if ((tid & 63) == 0) red[4 + (tid >> 6)] = l;
        __syncthreads();
        f[tid] = e / (red[4] + red[5] + red[6] + red[7]);
        __syncthreads();
        if (tid < width) {
            float acc = 0.f;
#pragma unroll
            for (int u = 0; u < kCombineOnce; ++u)
                if (u < splits) acc += f[u] * pv[u];
            out[((size_t)tok * heads + head) * width + tid] = acc;
        }
        if constexpr (WIDE) {
            // Heads wider than the workgroup: column tid + 256, same weights.
            const int c = tid + 256;
            if (c < width) {
#pragma unroll
                for (int u = 0; u < kCombineOnce; ++u)
                    pv[u] = partials[(base + (u < splits ? u : splits - 1)) * width + c];
                float acc = 0.f;
#pragma unroll
                for (int u = 0; u < kCombineOnce; ++u)
                    if (u < splits) acc += f[u] * pv[u];
                out[((size_t)tok * heads + head) * width + c] = acc;
            }
        }
        return;
    }
    float acc = 0.f, acc2 = 0.f;   // columns tid and (wide heads) tid + 256
    for (int s0 = 0; s0 < splits; s0 += 256) {
        const int ns = splits - s0 < 256 ? splits - s0 : 256;
        const float2 v = tid < ns ? ml[s0 + tid] : make_float2(-INFINITY, 0.f);
        // The maximum and the weighted sum of the l over all splits (the
        // first round covers every split when splits <= 256).
        float m = v.x;
        m = wave_reduce<true>(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        if (splits > 256) {
            // More than one round: the other rounds' maxima too.
            for (int s = 0; s < splits; ++s)
                if (s < s0 || s >= s0 + ns) m = fmaxf(m, ml[s].x);
        }
        const float e = v.x == -INFINITY ? 0.f : expf(v.x - m);
        float l = v.y * e;
        l = wave_reduce<false>(l);
        __syncthreads();
        if ((tid & 63) == 0) red[4 + (tid >> 6)] = l;
        __syncthreads();
        float total = red[4] + red[5] + red[6] + red[7];
        if (splits > 256)
            for (int s = 0; s < splits; ++s)
                if (s < s0 || s >= s0 + ns) {
                    const float2 w = ml[s];
                    if (w.x != -INFINITY) total += w.y * expf(w.x - m);
                }
        f[tid] = e / total;
        __syncthreads();
        if (tid < width) {
            const float *po = partials + (base + s0) * width + tid;
            constexpr int SU = 16;
            for (int k0 = 0; k0 < ns; k0 += SU) {
                float pv[SU];
#pragma unroll
                for (int u = 0; u < SU; ++u) pv[u] = po[(size_t)(k0 + u < ns ? k0 + u : ns - 1) * width];
#pragma unroll
                for (int u = 0; u < SU; ++u)
                    if (k0 + u < ns) acc += f[k0 + u] * pv[u];
            }
        }
        if constexpr (WIDE) {
            if (tid + 256 < width) {
                const float *po = partials + (base + s0) * width + tid + 256;
                constexpr int SU = 16;
                for (int k0 = 0; k0 < ns; k0 += SU) {
                    float pv[SU];
#pragma unroll
                    for (int u = 0; u < SU; ++u) pv[u] = po[(size_t)(k0 + u < ns ? k0 + u : ns - 1) * width];
#pragma unroll
                    for (int u = 0; u < SU; ++u)
                        if (k0 + u < ns) acc2 += f[k0 + u] * pv[u];
                }
            }
        }
        __syncthreads();
    }
    if (tid < width) out[((size_t)tok * heads + head) * width + tid] = acc;
    if constexpr (WIDE)
        if (tid + 256 < width) out[((size_t)tok * heads + head) * width + tid + 256] = acc2;
}

template <int W, int G>
void launch_split_wg(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *partials, const int *positions, int count, int heads, int kv_heads, int max_length, int window, int splits,
    float scale, hipStream_t s)
{
    hipLaunchKernelGGL((attention_split<W, G>), dim3((unsigned)kv_heads, (unsigned)splits, (unsigned)count),
                       dim3(256), 0, s, q, q_stride, keys, values, partials, positions, heads, kv_heads, max_length,
                       window, splits, scale);
    hipLaunchKernelGGL((attention_combine<(W > 256)>), dim3((unsigned)heads, (unsigned)count), dim3(256), 0, s,
                       partials, out, positions, heads, W, max_length, splits);
}

template <int W>
hipError_t launch_split_w(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *partials, const int *positions, int count, int heads, int kv_heads, int max_length, int window, int splits,
    float scale, hipStream_t s)
{
    switch (heads / kv_heads) {
    case 1: launch_split_wg<W, 1>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                  max_length, window, splits, scale, s); break;
    case 2: launch_split_wg<W, 2>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                  max_length, window, splits, scale, s); break;
    case 4:
        if constexpr (W <= 256) {
            launch_split_wg<W, 4>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                  max_length, window, splits, scale, s);
            break;
        }
        return hipErrorInvalidValue;
    default:
        if constexpr (W <= 128) {
            launch_split_wg<W, 8>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                  max_length, window, splits, scale, s);
            break;
        }
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// out[i][j] = silu(gate[i][j]) * up[i][j] for token i = blockIdx.y (rows at
// i times their strides), silu(x) = x / (1 + e^-x)
// (backend/core/llm_cpu.c:336-341); four elements per thread where n and the
// strides are multiples of 4 and the rows 16-byte aligned. out may be gate
// itself for one token.
__device__ __forceinline__ float silu_times(float x, float u) { return x / (1.0f + expf(-x)) * u; }

// GELU with the tanh approximation times u, the engine's Gemma gate
// (backend/core/llm_cpu.c:329-341), in its operation order.
__device__ __forceinline__ float gelu_times(float x, float u)
{
    return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x))) * u;
}

template <bool GELU>
__device__ __forceinline__ float gated(float x, float u) { return GELU ? gelu_times(x, u) : silu_times(x, u); }

template <bool GELU>
__global__ __launch_bounds__(256) void silu_mul4(const float4 *gate, int gate_stride4, const float4 *up,
    int up_stride4, float4 *out, int n4)
{
    const float4 *g = gate + (size_t)blockIdx.y * gate_stride4, *u = up + (size_t)blockIdx.y * up_stride4;
    float4 *o = out + (size_t)blockIdx.y * n4;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n4; i += gridDim.x * 256) {
        const float4 a = g[i], b = u[i];
        o[i] = make_float4(gated<GELU>(a.x, b.x), gated<GELU>(a.y, b.y), gated<GELU>(a.z, b.z),
                           gated<GELU>(a.w, b.w));
    }
}

// The same over rows that hold gate and up in 16-element blocks (row i of
// 2n values at gu + 2 n i: gate element j at 32 (j / 16) + j % 16, up
// element j 16 further), out rows of n.
template <bool GELU>
__global__ __launch_bounds__(256) void silu_pairs(const float *__restrict__ gu, float *__restrict__ out, int n)
{
    const float *row = gu + (size_t)blockIdx.y * 2 * n;
    float *o = out + (size_t)blockIdx.y * n;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
        const int at = 32 * (j >> 4) + (j & 15);
        o[j] = gated<GELU>(row[at], row[at + 16]);
    }
}

template <bool GELU>
__global__ __launch_bounds__(256) void silu_mul(const float *gate, int gate_stride, const float *up, int up_stride,
    float *out, int n)
{
    const float *g = gate + (size_t)blockIdx.y * gate_stride, *u = up + (size_t)blockIdx.y * up_stride;
    float *o = out + (size_t)blockIdx.y * n;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) o[i] = gated<GELU>(g[i], u[i]);
}

// step[0] = token, step[1] = position: one decode token's ids, written on
// the stream so that a recorded sequence of launches can read them.
__global__ void set_step(uint32_t *step, uint32_t token, int position)
{
    if (threadIdx.x == 0) {
        step[0] = token;
        step[1] = (uint32_t)position;
    }
}

unsigned grid_of(long n) { return (unsigned)(n < 256 * 1024 ? (n + 255) / 256 : 1024); }

// The greedy choice of each of `count` rows of n logits, as the engine's
// sampler makes it at temperature 0 (backend/core/llm_cpu.c:896-904) after
// the suppressed tokens are masked (backend/core/llm_cpu.c:570-574): the
// first index of the largest value among the entries whose bit in `mask` is
// clear (one bit per index, word i / 32, bit i % 32; null: none masked).
// 0xFFFFFFFF when the row holds a non-finite value anywhere (the engine
// rejects non-finite model output before it masks), or when every entry is
// masked. One workgroup per row: each thread scans
// its indices in increasing order (a later equal value never replaces an
// earlier one), then the pairs (value, index) meet with the larger value, or
// on equal values the smaller index, winning.
__global__ __launch_bounds__(1024) void greedy(const float *__restrict__ logits, int n,
    const uint32_t *__restrict__ mask, uint32_t *__restrict__ ids)
{
    __shared__ float sv[16];
    __shared__ int si[16];
    const float *row = logits + (size_t)blockIdx.x * n;
    float best = -INFINITY;
    int at = 0x7FFFFFFF;
    int bad = 0;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float v = row[i];
        bad |= !(__builtin_fabsf(v) <= 3.40282347e38f);
        const bool masked = mask && ((mask[i >> 5] >> (i & 31)) & 1u);
        if (!masked && v > best) {
            best = v;
            at = i;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(at, o, 64);
        if (ov > best || (ov == best && oi < at)) {
            best = ov;
            at = oi;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = best;
        si[wave] = at;
    }
    bad = __syncthreads_or(bad);
    if (threadIdx.x != 0) return;
    for (int q = 1; q < 16; ++q)
        if (sv[q] > best || (sv[q] == best && si[q] < at)) {
            best = sv[q];
            at = si[q];
        }
    ids[blockIdx.x] = bad || !(best > -INFINITY) ? 0xFFFFFFFFu : (uint32_t)at;
}

}  // namespace

hipError_t launch_set_step(uint32_t *step, uint32_t token, int position, hipStream_t s)
{
    hipLaunchKernelGGL(set_step, dim3(1), dim3(64), 0, s, step, token, position);
    return hipGetLastError();
}

hipError_t launch_embed(const uint8_t *w, unsigned type, size_t row_bytes, int rows, const uint32_t *tokens, int count,
    int cols, float *out, float scale, hipStream_t s)
{
    hipLaunchKernelGGL(embed, dim3(grid_of(cols), (unsigned)count), dim3(256), 0, s, w, type, row_bytes, rows, tokens,
                       cols, out, scale);
    return hipGetLastError();
}

hipError_t launch_rms_norm(float *x, const float *r, const float *w, float *out, int n, int count, float eps,
    hipStream_t s)
{
    const bool regs = (n & 3) == 0 && n <= 4 * 4096 &&
                      (((uintptr_t)x | (uintptr_t)r | (uintptr_t)w | (uintptr_t)out) & 15u) == 0;
    const int n4 = n / 4;
    const dim3 grid((unsigned)count);
    if (regs && n4 <= 1024)
        hipLaunchKernelGGL(rms_norm_regs<1>, grid, dim3(1024), 0, s, (float4 *)x, (const float4 *)r, (const float4 *)w,
                           (float4 *)out, n4, eps);
    else if (regs && n4 <= 2048)
        hipLaunchKernelGGL(rms_norm_regs<2>, grid, dim3(1024), 0, s, (float4 *)x, (const float4 *)r, (const float4 *)w,
                           (float4 *)out, n4, eps);
    else if (regs)
        hipLaunchKernelGGL(rms_norm_regs<4>, grid, dim3(1024), 0, s, (float4 *)x, (const float4 *)r, (const float4 *)w,
                           (float4 *)out, n4, eps);
    else
        hipLaunchKernelGGL(rms_norm, grid, dim3(256), 0, s, x, r, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_post_norm(float *x, const float *r, const float *post, float oscale, const float *w, float *out,
    int n, int count, float eps, hipStream_t s)
{
    const dim3 grid((unsigned)count);
    if (n <= 1024)
        hipLaunchKernelGGL(post_norm<1>, grid, dim3(1024), 0, s, x, r, post, oscale, w, out, n, eps);
    else if (n <= 2048)
        hipLaunchKernelGGL(post_norm<2>, grid, dim3(1024), 0, s, x, r, post, oscale, w, out, n, eps);
    else if (n <= 4096)
        hipLaunchKernelGGL(post_norm<4>, grid, dim3(1024), 0, s, x, r, post, oscale, w, out, n, eps);
    else if (n <= 8192)
        hipLaunchKernelGGL(post_norm<8>, grid, dim3(1024), 0, s, x, r, post, oscale, w, out, n, eps);
    else if (n <= kPostNormMax)
        hipLaunchKernelGGL(post_norm<16>, grid, dim3(1024), 0, s, x, r, post, oscale, w, out, n, eps);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_head_norm_rope(float *q, int q_stride, const float *k, int k_stride, const float *v, int v_stride,
    int count, int heads, int kv_heads, int width, const float *q_norm, const float *k_norm, float eps,
    const float *freq, const int *positions, int capacity, float *keys, float *values, hipStream_t s)
{
    if (width > kHeadWidthMax || width % 2) return hipErrorInvalidValue;
    const int rows = heads + (k ? 2 * kv_heads : 0);
    hipLaunchKernelGGL(head_norm_rope, dim3((unsigned)rows, (unsigned)count), dim3(256), 0, s, q, q_stride, k,
                       k_stride, v, v_stride, heads, kv_heads, width, q_norm, k_norm, eps, freq, positions, capacity,
                       keys, values);
    return hipGetLastError();
}

hipError_t launch_softcap(float *x, size_t n, float cap, hipStream_t s)
{
    hipLaunchKernelGGL(softcap, dim3(grid_of((long)(n < (size_t)1 << 30 ? n : (size_t)1 << 30))), dim3(256), 0, s, x,
                       n, cap);
    return hipGetLastError();
}

hipError_t launch_rope_qkv(float *q, int q_stride, const float *k, int k_stride, const float *v, int v_stride,
    int count, int heads, int kv_heads, int width, const float *freq, const int *positions, int capacity, float *keys,
    float *values, hipStream_t s)
{
    const long n = (long)(heads + kv_heads) * (width / 2) + (long)kv_heads * width;
    hipLaunchKernelGGL(rope_qkv, dim3(grid_of(n), (unsigned)count), dim3(256), 0, s, q, q_stride, k, k_stride, v,
                       v_stride, heads, kv_heads, width, freq, positions, capacity, keys, values);
    return hipGetLastError();
}

template <int W>
void launch_attention_w(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *scores, const int *positions, int count, int heads, int kv_heads, int max_length, int window, float scale,
    hipStream_t s)
{
    const dim3 grid((unsigned)heads, (unsigned)count);
    if (max_length <= kLdsScores && window == 0)
        hipLaunchKernelGGL((attention_w<W, true, false>), grid, dim3(256), 0, s, q, q_stride, keys, values, out, scores,
                           positions, heads, kv_heads, max_length, window, scale);
    else if (max_length <= kLdsScores)
        hipLaunchKernelGGL((attention_w<W, true, true>), grid, dim3(256), 0, s, q, q_stride, keys, values, out, scores,
                           positions, heads, kv_heads, max_length, window, scale);
    else if (window == 0)
        hipLaunchKernelGGL((attention_w<W, false, false>), grid, dim3(256), 0, s, q, q_stride, keys, values, out,
                           scores, positions, heads, kv_heads, max_length, window, scale);
    else
        hipLaunchKernelGGL((attention_w<W, false, true>), grid, dim3(256), 0, s, q, q_stride, keys, values, out,
                           scores, positions, heads, kv_heads, max_length, window, scale);
}

hipError_t launch_attention(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *scores, const int *positions, int count, int heads, int kv_heads, int width, int max_length, int window,
    float scale, hipStream_t s)
{
    if (width > kMaxWidth) return hipErrorInvalidValue;
    const bool aligned = (q_stride & 3) == 0 &&
                         (((uintptr_t)q | (uintptr_t)keys | (uintptr_t)values | (uintptr_t)out) & 15u) == 0;
    const dim3 grid((unsigned)heads, (unsigned)count);
    if (aligned && width == 128)
        launch_attention_w<128>(q, q_stride, keys, values, out, scores, positions, count, heads, kv_heads, max_length,
                                window, scale, s);
    else if (aligned && width == 64)
        launch_attention_w<64>(q, q_stride, keys, values, out, scores, positions, count, heads, kv_heads, max_length,
                               window, scale, s);
    else if (aligned && width == 256)
        launch_attention_w<256>(q, q_stride, keys, values, out, scores, positions, count, heads, kv_heads, max_length,
                                window, scale, s);
    else if (aligned && width == 512)
        launch_attention_w<512>(q, q_stride, keys, values, out, scores, positions, count, heads, kv_heads, max_length,
                                window, scale, s);
    else if (max_length <= kLdsScores)
        hipLaunchKernelGGL(attention<true>, grid, dim3(256), 0, s, q, q_stride, keys, values, out, scores, positions,
                           heads, kv_heads, width, max_length, window, scale);
    else
        hipLaunchKernelGGL(attention<false>, grid, dim3(256), 0, s, q, q_stride, keys, values, out, scores, positions,
                           heads, kv_heads, width, max_length, window, scale);
    return hipGetLastError();
}

bool attention_split_supported(int heads, int kv_heads, int width, int max_length, int splits)
{
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads || splits < 1 || splits > 4096 || max_length <= 0) return false;
    const int g = heads / kv_heads;
    if (width != 64 && width != 128 && width != 256 && width != 512) return false;
    if (g != 1 && g != 2 && g != 4 && !(g == 8 && width <= 128)) return false;
    if (width == 512 && g > 2) return false;
    return (max_length + splits - 1) / splits <= kSplitMaxChunk;
}

hipError_t launch_attention_split(const float *q, int q_stride, const float *keys, const float *values, float *out,
    float *partials, const int *positions, int count, int heads, int kv_heads, int width, int max_length, int window,
    int splits, float scale, hipStream_t s)
{
    if (!attention_split_supported(heads, kv_heads, width, max_length, splits) || (q_stride & 3) ||
        (((uintptr_t)q | (uintptr_t)keys | (uintptr_t)values | (uintptr_t)partials) & 15u))
        return hipErrorInvalidValue;
    if (width == 128)
        return launch_split_w<128>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                   max_length, window, splits, scale, s);
    if (width == 64)
        return launch_split_w<64>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                  max_length, window, splits, scale, s);
    if (width == 512)
        return launch_split_w<512>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                                   max_length, window, splits, scale, s);
    return launch_split_w<256>(q, q_stride, keys, values, out, partials, positions, count, heads, kv_heads,
                               max_length, window, splits, scale, s);
}

hipError_t launch_greedy(const float *logits, int n, int count, const uint32_t *mask, uint32_t *ids, hipStream_t s)
{
    hipLaunchKernelGGL(greedy, dim3((unsigned)count), dim3(1024), 0, s, logits, n, mask, ids);
    return hipGetLastError();
}

hipError_t launch_silu_pairs(const float *gu, float *out, int n, int count, hipStream_t s)
{
    hipLaunchKernelGGL(silu_pairs<false>, dim3(grid_of(n), (unsigned)count), dim3(256), 0, s, gu, out, n);
    return hipGetLastError();
}

hipError_t launch_gelu_pairs(const float *gu, float *out, int n, int count, hipStream_t s)
{
    hipLaunchKernelGGL(silu_pairs<true>, dim3(grid_of(n), (unsigned)count), dim3(256), 0, s, gu, out, n);
    return hipGetLastError();
}

template <bool GELU>
hipError_t launch_gated(const float *gate, int gate_stride, const float *up, int up_stride, float *out, int n,
    int count, hipStream_t s)
{
    if (((n | gate_stride | up_stride) & 3) == 0 && (((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) & 15u) == 0)
        hipLaunchKernelGGL(silu_mul4<GELU>, dim3(grid_of(n / 4), (unsigned)count), dim3(256), 0, s,
                           (const float4 *)gate, gate_stride / 4, (const float4 *)up, up_stride / 4, (float4 *)out,
                           n / 4);
    else
        hipLaunchKernelGGL(silu_mul<GELU>, dim3(grid_of(n), (unsigned)count), dim3(256), 0, s, gate, gate_stride, up,
                           up_stride, out, n);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *gate, int gate_stride, const float *up, int up_stride, float *out, int n,
    int count, hipStream_t s)
{
    return launch_gated<false>(gate, gate_stride, up, up_stride, out, n, count, s);
}

hipError_t launch_gelu_mul(const float *gate, int gate_stride, const float *up, int up_stride, float *out, int n,
    int count, hipStream_t s)
{
    return launch_gated<true>(gate, gate_stride, up, up_stride, out, n, count, s);
}

}  // namespace fy
