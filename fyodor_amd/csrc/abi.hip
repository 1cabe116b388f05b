// extern "C" entry points of libfyodor_hip.so (declared in include/fyodor_hip.h).
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
#include "../../include/fyodor_hip.h"
#include "formats.h"
#include "kernels.h"

namespace {

using namespace fy;

// Widest block-format row: eight activation rows of it stay below 2^31 bytes.
constexpr size_t kMaxTiledCols = (size_t)1 << 26;

// Same acceptance rules as the provider's request validation
// (backend/core/vendor.c:59-80) applied to packed storage, plus what the
// block-format kernels can address: they reach the whole matrix through one
// buffer resource with a 32-bit range and 32-bit tile offsets, and a batch of
// up to eight activation rows through another, so a block-format matrix
// above INT32_MAX bytes, or rows above 2^26 columns, are declined (the
// caller computes them elsewhere) rather than read with wrapped offsets.
bool storage_bytes(unsigned type, size_t rows, size_t cols, size_t *bytes)
{
    format_info f;
    if (!format_of(type, &f)) return false;
    if (!rows || !cols || rows > INT_MAX || cols > INT_MAX || cols % f.block) return false;
    const size_t blocks = cols / f.block;
    if (blocks > SIZE_MAX / f.bytes) return false;
    const size_t row = blocks * f.bytes;
    if (rows > SIZE_MAX / row) return false;
    const bool tiled = type != F32 && type != F16 && type != BF16;
    if (tiled && (rows * row > (size_t)INT32_MAX || cols > kMaxTiledCols)) return false;
    *bytes = rows * row;
    return true;
}

// Batches above the small-N kernels' 8 columns go to the prefill GEMM (every
// block format), except small batches of matrices the row-balanced small-N
// kernel takes: those stay memory-bound, and launches of 8 tokens each beat
// the GEMM's activation split and sparse grid up to a batch measured per
// shape (MI355X, 50 calls over rotating weights, GEMM / 8-token launches):
// Q4_K 14336 x 4096 at 16 tokens 32.0 / 22.3 us, at 24 32.6 / 33.0; Q4_K and
// Q8_0 4096 x 4096 at 32 31.4 / 26.2 and 40.7 / 25.6, at 40 31.1 / 32.6;
// Q6_K 4096 x 14336 (its int8 GEMM starts slow on wide rows) at 48
// 203.9 / 152.7, at 64 203.9 / 201.9. The Q6_K output head (128256 x 4096)
// keeps the GEMM from 9 tokens on (173 / 198 us).
bool use_prefill(unsigned type, size_t rows, size_t cols, size_t batch)
{
    if (batch <= 8 || !(type == Q4_K || type == Q6_K || type == Q8_0 || type == Q4_0)) return false;
    size_t chunked = 0;
    if (type == Q6_K) chunked = cols > 4096 ? 56 : 0;
    else chunked = rows >= 8192 ? 20 : 32;
    return batch > chunked || !smalln_rows_supported(type, (int)rows, (int)cols, 8);
}

int status(hipError_t e)
{
    return e == hipSuccess ? 0 : -(int)(e > 0 ? e : 1);
}

// One token of a quantized matrix: the batch-1 matvec where it exists, else
// the small-N kernel at batch 1.
hipError_t launch_token(unsigned type, const uint8_t *w, const float *x, float *y, int rows, int cols, hipStream_t s)
{
    if (matvec_supported(type, rows, cols)) return launch_matvec(type, w, x, y, rows, cols, s);
    return launch_smalln(type, w, x, y, rows, cols, 1, nullptr, s);
}

int matmul_impl(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x, uintptr_t y, size_t batch,
    uintptr_t workspace, size_t workspace_bytes, uintptr_t stream)
{
    size_t b;
    if (!w || !x || !y || !batch || batch > INT_MAX || !storage_bytes(type, rows, cols, &b)) return 1;
    // 16-byte weight and activation loads, 4-byte outputs.
    if ((w & 15u) || (x & 15u) || (y & 3u)) return 1;
    const bool dense = type == F32 || type == F16 || type == BF16;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *wp = (const uint8_t *)w;
    const bool fits = workspace && !(workspace & 15u);
    // The GEMM needs its workspace; without one (or a short one) the batch is
    // run 8 columns at a time instead.
    if (use_prefill(type, rows, cols, batch) && fits && workspace_bytes >= prefill_workspace(type, (int)cols, (int)batch))
        return status(launch_prefill(type, wp, (const float *)x, (float *)y, (int)rows, (int)cols, (int)batch,
                                     (void *)workspace, s));
    if (dense && dense_gemm_supported(type, (int)rows, (int)cols, (int)batch))
        return status(launch_dense_gemm(type, wp, (const float *)x, (float *)y, (int)rows, (int)cols, (int)batch,
                                        fits ? (void *)workspace : nullptr, fits ? workspace_bytes : 0, s));
    for (size_t done = 0; done < batch; done += 8) {
        const int n = (int)(batch - done < 8 ? batch - done : 8);
        const float *xp = (const float *)x + done * cols;
        float *yp = (float *)y + done * rows;
        if (dense) {
            const int st = status(launch_dense(type, wp, xp, yp, (int)rows, (int)cols, n, s));
            if (st) return st;
        } else if (n == 1) {
            const int st = status(launch_token(type, wp, xp, yp, (int)rows, (int)cols, s));
            if (st) return st;
        } else if (smalln_rows_supported(type, (int)rows, (int)cols, n)) {
            const int st = status(launch_smalln_rows(type, wp, xp, yp, (int)rows, (int)cols, n, s));
            if (st) return st;
        } else if ((fits && workspace_bytes >= smalln_workspace((int)cols, n))) {
            const int st = status(launch_smalln(type, wp, xp, yp, (int)rows, (int)cols, n, (void *)workspace, s));
            if (st) return st;
        } else {
            // No room for the activation digits of several tokens: one at a time.
            for (int k = 0; k < n; ++k) {
                const int st = status(launch_token(type, wp, xp + (size_t)k * cols, yp + (size_t)k * rows,
                                                   (int)rows, (int)cols, s));
                if (st) return st;
            }
        }
    }
    return 0;
}


// ---- the allocation-free entry point ---------------------------------------
//
// Scratch of nya_hip_matmul_static: a fixed device array, one copy per GPU
// (the runtime places it when it loads this library's code on the device and
// keeps it until the process ends). In host code `scratch` names a host-side
// stand-in, not device memory: its device address is looked up once per
// device with hipGetSymbolAddress, with that device current, and only that
// address is handed to kernels.
constexpr size_t kStaticScratchBytes = NYA_HIP_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch[kMaxDevices];

// The current device's copy of `scratch`, or nullptr if it cannot be found.
void *static_scratch()
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> hold(g_scratch_lock);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_scratch[dev] = p;
    }
    return g_scratch[dev];
}

// Tokens per call of the prefill GEMM whose workspace fits the array (a
// multiple of its 32-token tiles), or 0 if not even 32 do.
size_t static_chunk_tokens(unsigned type, size_t cols)
{
    // Whole 64-token blocks: the workspace rounds the batch up to them.
    const size_t per64 = prefill_workspace(type, (int)cols, 64);
    return per64 ? kStaticScratchBytes / per64 * 64 : 0;
}

}  // namespace

extern "C" {

NYA_HIP_EXPORT unsigned nya_hip_abi_version(void) { return NYA_HIP_ABI_VERSION; }

NYA_HIP_EXPORT int nya_hip_weight_bytes(unsigned type, size_t rows, size_t cols, size_t *bytes)
{
    size_t b;
    if (!bytes || !storage_bytes(type, rows, cols, &b)) return 1;
    *bytes = b;
    return 0;
}

NYA_HIP_EXPORT int nya_hip_weight_layout(unsigned type)
{
    format_info f;
    if (!format_of(type, &f)) return -1;
    return type == F32 || type == F16 || type == BF16 ? 0 : 1;
}

NYA_HIP_EXPORT int nya_hip_weight_pack(void *dst, const void *src, unsigned type, size_t rows, size_t cols)
{
    size_t b;
    if (!dst || !src || !storage_bytes(type, rows, cols, &b)) return 1;
    pack_tiles((uint8_t *)dst, (const uint8_t *)src, type, rows, cols);
    return 0;
}

NYA_HIP_EXPORT int nya_hip_workspace_bytes(unsigned type, size_t rows, size_t cols, size_t batch, size_t *bytes)
{
    size_t b;
    if (!bytes || !batch || batch > INT_MAX || !storage_bytes(type, rows, cols, &b)) return 1;
    const bool dense = type == F32 || type == F16 || type == BF16;
    const int n = batch < 8 ? (int)batch : 8;
    if (dense)
        *bytes = dense_gemm_supported(type, (int)rows, (int)cols, (int)batch)
                     ? dense_gemm_workspace((int)rows, (int)cols, (int)batch) : 0;
    else
        *bytes = use_prefill(type, rows, cols, batch) ? prefill_workspace(type, (int)cols, (int)batch)
               : smalln_rows_supported(type, (int)rows, (int)cols, n) ? 0 : smalln_workspace((int)cols, n);
    return 0;
}

NYA_HIP_EXPORT int nya_hip_matmul(uintptr_t w, unsigned type, size_t rows, size_t cols,
    uintptr_t x, uintptr_t y, size_t batch, uintptr_t workspace, size_t workspace_bytes, uintptr_t stream)
{
    return matmul_impl(w, type, rows, cols, x, y, batch, workspace, workspace_bytes, stream);
}

NYA_HIP_EXPORT int nya_hip_matmul_static(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t y, size_t batch, uintptr_t stream)
{
    size_t b;
    if (!w || !x || !y || !batch || batch > INT_MAX || !storage_bytes(type, rows, cols, &b)) return 1;
    if ((w & 15u) || (x & 15u) || (y & 3u)) return 1;
    void *ws = static_scratch();
    if (!ws) return -(int)hipErrorInvalidSymbol;
    // The prefill GEMM runs in token chunks whose workspace fits the array
    // (every token is independent of the others): `parts` chunks of nearly
    // equal size, each above half the array's capacity (at least 32 tokens),
    // so every chunk stays on the GEMM and every token gets the same result
    // as through nya_hip_matmul. Where not even 64 tokens of the GEMM's
    // workspace fit (rows of about 254k columns and more), the batch runs
    // as 8-token launches, as nya_hip_matmul does with a short workspace.
    // Every other path needs at most a few hundred KiB (the small-N digits
    // of one 16384-column chunk); matmul_impl itself falls back to launches
    // without scratch where even that would not fit.
    size_t parts = 1;
    if (use_prefill(type, rows, cols, batch)) {
        const size_t fit = static_chunk_tokens(type, cols);
        if (fit < 64) return matmul_impl(w, type, rows, cols, x, y, batch, (uintptr_t)ws, kStaticScratchBytes, stream);
        parts = (batch + fit - 1) / fit;
    }
    for (size_t part = 0, done = 0; part < parts; ++part) {
        const size_t n = batch / parts + (part < batch % parts ? 1 : 0);
        const int st = matmul_impl(w, type, rows, cols, x + done * cols * sizeof(float),
                                   y + done * rows * sizeof(float), n, (uintptr_t)ws, kStaticScratchBytes, stream);
        if (st) return st;
        done += n;
    }
    return 0;
}

NYA_HIP_EXPORT int nya_hip_matvec_gated(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t gate,
    uintptr_t up, uintptr_t y, uintptr_t stream)
{
    size_t b;
    if (!w || !gate || !up || !y || !storage_bytes(type, rows, cols, &b)) return 1;
    if ((w & 15u) || (gate & 15u) || (up & 15u) || (y & 3u)) return 1;
    if (!matvec_gated_supported(type, (int)rows, (int)cols)) return 1;
    return status(launch_matvec_gated(type, (const uint8_t *)w, (const float *)gate, (const float *)up, (float *)y,
                                      (int)rows, (int)cols, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_normed(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t r, uintptr_t norm, float eps, uintptr_t hout, uintptr_t y, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_normed_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!x || !norm || !y || (r && !hout) || ((w | x | r | norm | hout) & 15u) || (y & 3u)) return 1;
    if (r && hout < r + 4 * cols && r < hout + 4 * cols) return 1;
    if (r && hout < x + 4 * cols && x < hout + 4 * cols) return 1;
    return status(launch_matvec_normed(type, (const uint8_t *)w, (const float *)x, (const float *)r,
                                       (const float *)norm, (float *)hout, eps, (float *)y, (int)rows, (int)cols,
                                       (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_swiglu(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t hidden, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_swiglu_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!x || !hidden || (w & 15u) || (x & 15u) || (hidden & 3u)) return 1;
    return status(launch_matvec_swiglu(type, (const uint8_t *)w, (const float *)x, (float *)hidden, (int)rows,
                                       (int)cols, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_geglu(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t hidden, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_swiglu_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!x || !hidden || (w & 15u) || (x & 15u) || (hidden & 3u)) return 1;
    return status(launch_matvec_geglu(type, (const uint8_t *)w, (const float *)x, (float *)hidden, (int)rows,
                                      (int)cols, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_residual(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x,
    uintptr_t res, uintptr_t norm, uintptr_t hn, uintptr_t parts, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_residual_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!x || !res || !norm || !hn || !parts || ((w | x) & 15u) || ((res | norm | hn) & 3u) || (parts & 7u)) return 1;
    // hn and the partial sums are written while other workgroups read x.
    if (hn < x + 4 * cols && x < hn + 4 * rows) return 1;
    if (parts < x + 4 * cols && x < parts + 8 * NYA_HIP_NORM_PARTS) return 1;
    if (hn < res + 4 * rows && res < hn + 4 * rows) return 1;
    return status(launch_matvec_residual(type, (const uint8_t *)w, (const float *)x, (float *)res,
                                         (const float *)norm, (float *)hn, (double *)parts, (int)rows, (int)cols,
                                         (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_swiglu_scaled(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t hn,
    uintptr_t parts, float eps, uintptr_t hidden, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_swiglu_scaled_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!hn || !parts || !hidden || ((w | hn) & 15u) || (parts & 7u) || (hidden & 3u)) return 1;
    return status(launch_matvec_swiglu_scaled(type, (const uint8_t *)w, (const float *)hn, (const double *)parts,
                                              eps, (float *)hidden, (int)rows, (int)cols, (hipStream_t)stream));
}

NYA_HIP_EXPORT const char *nya_hip_kernel_name(unsigned type, size_t rows, size_t cols, size_t batch)
{
    size_t b;
    if (!batch || batch > INT_MAX || !storage_bytes(type, rows, cols, &b)) return NULL;
    if (type == F32 || type == F16 || type == BF16)
        return dense_gemm_supported(type, (int)rows, (int)cols, (int)batch) ? "dense_gemm" : "skinny_dense";
    if (use_prefill(type, rows, cols, batch)) return prefill_kernel(type);
    if (batch == 1 && matvec_supported(type, (int)rows, (int)cols)) return matvec_kernel(type, (int)rows, (int)cols);
    // Batches above 8 outside the GEMM run 8 tokens per launch.
    const int n = batch < 8 ? (int)batch : 8;
    return smalln_rows_supported(type, (int)rows, (int)cols, n) ? "smalln_rows" : "smalln_mfma";
}

NYA_HIP_EXPORT int nya_hip_copy(uintptr_t dst, uintptr_t src, size_t bytes, uintptr_t stream)
{
    if (!dst || !src || (dst & 15u) || (src & 15u) || (bytes & 15u)) return 1;
    return status(launch_copy((uint4 *)dst, (const uint4 *)src, bytes / 16, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_read(uintptr_t src, size_t bytes, uintptr_t sink, uintptr_t stream)
{
    if (!src || !sink || !bytes || (src & 15u) || (sink & 3u) || (bytes & 15u)) return 1;
    return status(launch_read((const uint4 *)src, bytes / 16, (unsigned *)sink, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_read_shaped(uintptr_t src, size_t bytes, uintptr_t sink, int waves, int depth,
    int per_cu, int mode, uintptr_t stream)
{
    if (!src || !sink || !bytes || (src & 15u) || (sink & 3u) || (bytes & 15u)) return 1;
    const hipError_t e = launch_read_shaped((const uint4 *)src, bytes / 16, (unsigned *)sink, waves, depth, per_cu,
                                            mode, (hipStream_t)stream);
    return e == hipErrorInvalidValue ? 1 : status(e);
}

// ---- resident decoder steps ----------------------------------------------

// fp32 device vectors: non-null and 4-byte aligned.
static bool vec(uintptr_t p) { return p && !(p & 3u); }
static bool count_ok(size_t n) { return n && n <= (size_t)INT_MAX; }
// Tokens per call: the second grid dimension.
static bool tokens_ok(size_t count) { return count && count <= 65535; }

NYA_HIP_EXPORT int nya_hip_step(uintptr_t step, unsigned token, size_t position, uintptr_t stream)
{
    if (!vec(step) || position > (size_t)INT_MAX) return 1;
    return status(launch_set_step((uint32_t *)step, token, (int)position, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_embed(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t tokens, size_t count,
    uintptr_t out, float scale, uintptr_t stream)
{
    format_info f;
    if (!w || !vec(tokens) || !vec(out) || !format_of(type, &f) || !count_ok(rows) || !count_ok(cols) ||
        cols % f.block || !tokens_ok(count) || !isfinite(scale))
        return 1;
    const size_t row_bytes = cols / f.block * f.bytes;
    return status(launch_embed((const uint8_t *)w, type, row_bytes, (int)rows, (const uint32_t *)tokens, (int)count,
                               (int)cols, (float *)out, scale, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_rms_norm(uintptr_t x, uintptr_t residual, uintptr_t weight, uintptr_t out, size_t n,
    size_t count, float epsilon, uintptr_t stream)
{
    if (!vec(x) || !vec(out) || (residual & 3u) || (weight & 3u) || !count_ok(n) || !tokens_ok(count) ||
        !(epsilon >= 0.f))
        return 1;
    return status(launch_rms_norm((float *)x, (const float *)residual, (const float *)weight, (float *)out, (int)n,
                                  (int)count, epsilon, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_post_norm(uintptr_t x, uintptr_t residual, uintptr_t post, float output_scale,
    uintptr_t weight, uintptr_t out, size_t n, size_t count, float epsilon, uintptr_t stream)
{
    if (!vec(x) || !vec(out) || (residual & 3u) || (post & 3u) || (post && !residual) || (weight & 3u) ||
        !count_ok(n) || n > (size_t)kPostNormMax || !tokens_ok(count) || !(epsilon >= 0.f) || !isfinite(output_scale))
        return 1;
    return status(launch_post_norm((float *)x, (const float *)residual, (const float *)post, output_scale,
                                   (const float *)weight, (float *)out, (int)n, (int)count, epsilon,
                                   (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_head_norm_rope(uintptr_t q, size_t q_stride, uintptr_t k, size_t k_stride, uintptr_t v,
    size_t v_stride, size_t count, size_t heads, size_t kv_heads, size_t width, uintptr_t q_norm, uintptr_t k_norm,
    float epsilon, uintptr_t frequencies, uintptr_t positions, size_t capacity, uintptr_t keys, uintptr_t values,
    uintptr_t stream)
{
    if (!vec(q) || !vec(q_norm) || !vec(frequencies) || !vec(positions) || !tokens_ok(count) || !count_ok(heads) ||
        !count_ok(kv_heads) || !count_ok(width) || width % 2 || width > 512 || !count_ok(capacity) ||
        heads > 65535 || kv_heads > 65535 || heads + 2 * kv_heads > 65535 || !(epsilon >= 0.f) ||
        q_stride < heads * width || q_stride > (size_t)INT_MAX || capacity > (size_t)INT_MAX / (kv_heads * width))
        return 1;
    if (k && (!vec(k) || !vec(v) || !vec(k_norm) || !vec(keys) || !vec(values) || k_stride < kv_heads * width ||
              v_stride < kv_heads * width || k_stride > (size_t)INT_MAX || v_stride > (size_t)INT_MAX))
        return 1;
    return status(launch_head_norm_rope((float *)q, (int)q_stride, (const float *)k, (int)k_stride,
                                        (const float *)v, (int)v_stride, (int)count, (int)heads, (int)kv_heads,
                                        (int)width, (const float *)q_norm, (const float *)k_norm, epsilon,
                                        (const float *)frequencies, (const int *)positions, (int)capacity,
                                        (float *)keys, (float *)values, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_softcap(uintptr_t x, size_t n, float cap, uintptr_t stream)
{
    if (!vec(x) || !n || !(cap > 0.f) || !isfinite(cap)) return 1;
    return status(launch_softcap((float *)x, n, cap, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_rope_qkv(uintptr_t q, size_t q_stride, uintptr_t k, size_t k_stride, uintptr_t v,
    size_t v_stride, size_t count, size_t heads, size_t kv_heads, size_t width, uintptr_t frequencies,
    uintptr_t positions, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    if (!vec(q) || !vec(k) || !vec(v) || !vec(frequencies) || !vec(positions) || !vec(keys) || !vec(values) ||
        !tokens_ok(count) || !count_ok(heads) || !count_ok(kv_heads) || !count_ok(width) || width % 2 ||
        !count_ok(capacity) || heads > (size_t)INT_MAX / width || kv_heads > (size_t)INT_MAX / width ||
        q_stride < heads * width || k_stride < kv_heads * width || v_stride < kv_heads * width ||
        q_stride > (size_t)INT_MAX || k_stride > (size_t)INT_MAX || v_stride > (size_t)INT_MAX)
        return 1;
    return status(launch_rope_qkv((float *)q, (int)q_stride, (const float *)k, (int)k_stride, (const float *)v,
                                  (int)v_stride, (int)count, (int)heads, (int)kv_heads, (int)width,
                                  (const float *)frequencies, (const int *)positions, (int)capacity, (float *)keys,
                                  (float *)values, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_attention(uintptr_t q, size_t q_stride, uintptr_t keys, uintptr_t values, uintptr_t out,
    uintptr_t scores, uintptr_t positions, size_t count, size_t heads, size_t kv_heads, size_t width,
    size_t max_length, size_t window, float scale, uintptr_t stream)
{
    if (!vec(q) || !vec(keys) || !vec(values) || !vec(out) || !vec(positions) || (scores & 3u) ||
        !tokens_ok(count) || !count_ok(heads) || !count_ok(kv_heads) || !count_ok(width) || width > 512 ||
        !count_ok(max_length) || heads % kv_heads || kv_heads > (size_t)INT_MAX / width ||
        q_stride < heads * width || q_stride > (size_t)INT_MAX || (max_length > 8192 && !scores) ||
        heads > (size_t)INT_MAX / max_length || window > (size_t)INT_MAX)
        return 1;
    return status(launch_attention((const float *)q, (int)q_stride, (const float *)keys, (const float *)values,
                                   (float *)out, (float *)scores, (const int *)positions, (int)count, (int)heads,
                                   (int)kv_heads, (int)width, (int)max_length, (int)window, scale,
                                   (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_attention_split(uintptr_t q, size_t q_stride, uintptr_t keys, uintptr_t values,
    uintptr_t out, uintptr_t partials, uintptr_t positions, size_t count, size_t heads, size_t kv_heads, size_t width,
    size_t max_length, size_t window, size_t splits, float scale, uintptr_t stream)
{
    if (!q)   // the shape query
        return count_ok(heads) && count_ok(kv_heads) && count_ok(width) && count_ok(max_length) &&
                       count_ok(splits) && heads <= 4096 && splits <= 4096 && max_length <= (size_t)INT_MAX &&
                       attention_split_supported((int)heads, (int)kv_heads, (int)width, (int)max_length, (int)splits)
                   ? 0 : 1;
    if (!vec(q) || !vec(keys) || !vec(values) || !vec(out) || !vec(positions) || !partials || !tokens_ok(count) ||
        !count_ok(heads) || !count_ok(kv_heads) || !count_ok(width) || !count_ok(max_length) || !count_ok(splits) ||
        q_stride < heads * width || q_stride > (size_t)INT_MAX || heads > 4096 || splits > 4096 ||
        max_length > (size_t)INT_MAX || window > (size_t)INT_MAX ||
        !attention_split_supported((int)heads, (int)kv_heads, (int)width, (int)max_length, (int)splits) ||
        (q_stride & 3u) || ((q | keys | values | partials) & 15u))
        return 1;
    return status(launch_attention_split((const float *)q, (int)q_stride, (const float *)keys, (const float *)values,
                                         (float *)out, (float *)partials, (const int *)positions, (int)count,
                                         (int)heads, (int)kv_heads, (int)width, (int)max_length, (int)window,
                                         (int)splits, scale, (hipStream_t)stream));
}

// A matrix of q|k|v rows [first_row, first_row + rows) of heads + 2 kv_heads
// heads of width: all of them, or one part (even first row).
static bool qkv_part_ok(size_t rows, size_t first_row, size_t heads, size_t kv_heads, size_t width)
{
    return count_ok(heads) && count_ok(kv_heads) && count_ok(width) && width % 2 == 0 && heads <= 65536 &&
           kv_heads <= 65536 && (heads + 2 * kv_heads) <= (size_t)INT_MAX / width && first_row % 2 == 0 &&
           first_row < (heads + 2 * kv_heads) * width && rows <= (heads + 2 * kv_heads) * width - first_row;
}

NYA_HIP_EXPORT int nya_hip_matvec_normed_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row,
    uintptr_t x, uintptr_t r, uintptr_t norm, float eps, uintptr_t hout, uintptr_t y, uintptr_t positions,
    uintptr_t frequencies, size_t heads, size_t kv_heads, size_t width, size_t capacity, uintptr_t keys,
    uintptr_t values, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_normed_rope_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!qkv_part_ok(rows, first_row, heads, kv_heads, width) || !count_ok(capacity)) return 1;
    if (!x || !norm || !y || (r && !hout) || !vec(positions) || !vec(frequencies) || !vec(keys) || !vec(values) ||
        ((w | x | r | norm | hout) & 15u) || (y & 3u))
        return 1;
    if (r && hout < r + 4 * cols && r < hout + 4 * cols) return 1;
    if (r && hout < x + 4 * cols && x < hout + 4 * cols) return 1;
    return status(launch_matvec_normed_rope(type, (const uint8_t *)w, (const float *)x, (const float *)r,
                                            (const float *)norm, (float *)hout, eps, (float *)y, (int)rows, (int)cols,
                                            (int)first_row, (const int *)positions, (const float *)frequencies,
                                            (float *)keys, (float *)values, (int)(heads * width),
                                            (int)(kv_heads * width), (int)width, (int)capacity, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_scaled_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row,
    uintptr_t hn, uintptr_t parts, float eps, uintptr_t y, uintptr_t positions, uintptr_t frequencies, size_t heads,
    size_t kv_heads, size_t width, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type, rows, cols, &b) || !matvec_normed_rope_supported(type, (int)rows, (int)cols)) return 1;
    if (!w) return 0;   // the shape query
    if (!qkv_part_ok(rows, first_row, heads, kv_heads, width) || !count_ok(capacity)) return 1;
    if (!hn || !parts || !y || !vec(positions) || !vec(frequencies) || !vec(keys) || !vec(values) ||
        ((w | hn) & 15u) || (parts & 7u) || (y & 3u))
        return 1;
    return status(launch_matvec_scaled_rope(type, (const uint8_t *)w, (const float *)hn, (const double *)parts, eps,
                                            (float *)y, (int)rows, (int)cols, (int)first_row, (const int *)positions,
                                            (const float *)frequencies, (float *)keys, (float *)values,
                                            (int)(heads * width), (int)(kv_heads * width), (int)width, (int)capacity,
                                            (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_matvec_rope_pair(uintptr_t w0, unsigned type0, size_t rows0, uintptr_t w1, unsigned type1,
    size_t rows1, size_t cols, uintptr_t x, uintptr_t r, uintptr_t norm, uintptr_t hout, uintptr_t parts, float eps,
    uintptr_t y, uintptr_t positions, uintptr_t frequencies, size_t heads, size_t kv_heads, size_t width,
    size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    size_t b;
    if (!storage_bytes(type0, rows0, cols, &b) || !storage_bytes(type1, rows1, cols, &b) ||
        !matvec_rope_pair_supported(type0, (int)rows0, type1, (int)rows1, (int)cols))
        return 1;
    if (!w0) return 0;   // the shape query
    if (!w1 || !qkv_part_ok(rows0 + rows1, 0, heads, kv_heads, width) ||
        rows0 + rows1 != (heads + 2 * kv_heads) * width || !count_ok(capacity) || !x || !y || !vec(positions) ||
        !vec(frequencies) || !vec(keys) || !vec(values) || ((w0 | w1 | x) & 15u) || (y & 3u))
        return 1;
    if (parts) {
        if (parts & 7u) return 1;
        r = norm = hout = 0;
    } else {
        if (!norm || (r && !hout) || ((r | norm | hout) & 15u)) return 1;
        if (r && hout < r + 4 * cols && r < hout + 4 * cols) return 1;
        if (r && hout < x + 4 * cols && x < hout + 4 * cols) return 1;
    }
    return status(launch_matvec_rope_pair(type0, (const uint8_t *)w0, (int)rows0, type1, (const uint8_t *)w1,
                                          (int)rows1, (int)cols, (const float *)x, (const float *)r,
                                          (const float *)norm, (float *)hout, (const double *)parts, eps, (float *)y,
                                          (const int *)positions, (const float *)frequencies, (float *)keys,
                                          (float *)values, (int)(heads * width), (int)(kv_heads * width), (int)width,
                                          (int)capacity, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_greedy(uintptr_t logits, size_t n, size_t count, uintptr_t mask, uintptr_t ids,
    uintptr_t stream)
{
    if (!vec(logits) || !vec(ids) || (mask & 3u) || !count_ok(n) || !tokens_ok(count)) return 1;
    return status(launch_greedy((const float *)logits, (int)n, (int)count, (const uint32_t *)mask, (uint32_t *)ids,
                                (hipStream_t)stream));
}

static bool pairs_ok(uintptr_t gu, uintptr_t out, size_t n, size_t count)
{
    if (!vec(gu) || !vec(out) || !count_ok(n) || n % 16 || n > (size_t)INT_MAX / 2 || !tokens_ok(count)) return false;
    const uintptr_t in_end = gu + 8 * n * count, out_end = out + 4 * n * count;
    return !(gu < out_end && out < in_end);   // not overlapping
}

NYA_HIP_EXPORT int nya_hip_silu_pairs(uintptr_t gu, uintptr_t out, size_t n, size_t count, uintptr_t stream)
{
    if (!pairs_ok(gu, out, n, count)) return 1;
    return status(launch_silu_pairs((const float *)gu, (float *)out, (int)n, (int)count, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_gelu_pairs(uintptr_t gu, uintptr_t out, size_t n, size_t count, uintptr_t stream)
{
    if (!pairs_ok(gu, out, n, count)) return 1;
    return status(launch_gelu_pairs((const float *)gu, (float *)out, (int)n, (int)count, (hipStream_t)stream));
}

// The checks of the gated activations: one token may be rewritten in place
// (out = gate); across tokens the output must not overlap either input.
static bool gated_ok(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride, uintptr_t out, size_t n,
    size_t count)
{
    if (!vec(gate) || !vec(up) || !vec(out) || !count_ok(n) || !tokens_ok(count) || gate_stride < n ||
        up_stride < n || gate_stride > (size_t)INT_MAX || up_stride > (size_t)INT_MAX)
        return false;
    const size_t out_end = out + count * n * sizeof(float);
    const size_t gate_end = gate + ((count - 1) * gate_stride + n) * sizeof(float);
    const size_t up_end = up + ((count - 1) * up_stride + n) * sizeof(float);
    return !(count > 1 && ((out < gate_end && gate < out_end) || (out < up_end && up < out_end)));
}

NYA_HIP_EXPORT int nya_hip_silu_mul(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride,
    uintptr_t out, size_t n, size_t count, uintptr_t stream)
{
    if (!gated_ok(gate, gate_stride, up, up_stride, out, n, count)) return 1;
    return status(launch_silu_mul((const float *)gate, (int)gate_stride, (const float *)up, (int)up_stride,
                                  (float *)out, (int)n, (int)count, (hipStream_t)stream));
}

NYA_HIP_EXPORT int nya_hip_gelu_mul(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride,
    uintptr_t out, size_t n, size_t count, uintptr_t stream)
{
    if (!gated_ok(gate, gate_stride, up, up_stride, out, n, count)) return 1;
    return status(launch_gelu_mul((const float *)gate, (int)gate_stride, (const float *)up, (int)up_stride,
                                  (float *)out, (int)n, (int)count, (hipStream_t)stream));
}

}  // extern "C"
