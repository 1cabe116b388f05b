/* Test-only stand-in for the HIP runtime and libfyodor_hip.so, used to test
 * the C provider's ownership, layout, error propagation and cache behaviour
 * on the CPU (the reference tests its provider the same way:
 * backend/tests/mock_vendor.c, backend/tests/test_vendor.c).
 *
 * "Device" memory is host memory. Every fallible call can be made to fail
 * once with nya_mock_arm_fault(n) (the n-th fallible call from now fails);
 * nya_mock_outstanding() counts allocations and streams not yet released. The
 * matmul computes in double from GGUF element values (the oracle's decoder).
 * Its Q8_0 device layout XORs every byte with 0x5A, so a provider that
 * uploads GGUF bytes where the packed copy belongs produces wrong results. */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define API __attribute__((visibility("default")))

/* ---- HIP runtime ----------------------------------------------------------
 * The entry points the provider resolves, with the signatures and status
 * values of hip/hip_runtime_api.h (ROCm 7.2): hipSuccess 0,
 * hipErrorInvalidValue 1, hipErrorOutOfMemory 2, hipErrorInvalidDevice 101.
 * One device (index 0) with 1 GiB; memory of either kind is calloc'ed host
 * memory; copies run at once on the calling thread. */
typedef int hipError_t;
typedef void *hipStream_t;

enum { OK = 0, INVALID_VALUE = 1, OUT_OF_MEMORY = 2, INVALID_DEVICE = 101 };
enum { H2D = 1, D2H = 2 };            /* hipMemcpyKind */
enum { STREAM_NON_BLOCKING = 1 };     /* hipStreamNonBlocking */

float orc_value(const unsigned char *data, unsigned type, size_t index);

static struct {
    int d2h;            /* device-to-host copy calls so far */
    int outstanding;    /* allocations (device, pinned) and streams not yet released */
    int armed;          /* the armed-th fallible call from now fails (0: none) */
    int fallible;       /* fallible calls made so far */
    int current;        /* current device */
} state;

/* Every call that can fail in HIP passes here first. */
static int injected_fault(void)
{
    ++state.fallible;
    return state.armed > 0 && --state.armed == 0;
}

static void *obtain(size_t bytes)
{
    void *p = calloc(1, bytes ? bytes : 1);
    if (p) ++state.outstanding;
    return p;
}

static void give_back(void *p)
{
    if (!p) return;
    --state.outstanding;
    free(p);
}

API void nya_mock_arm_fault(int n) { state.armed = n; }
API int nya_mock_outstanding(void) { return state.outstanding; }
API int nya_mock_calls(void) { return state.fallible; }
API int nya_mock_d2h_copies(void) { return state.d2h; }

API hipError_t hipInit(unsigned flags)
{
    if (injected_fault()) return INVALID_DEVICE;
    return flags ? INVALID_VALUE : OK;
}

API hipError_t hipGetDeviceCount(int *count)
{
    if (injected_fault()) return INVALID_DEVICE;
    *count = 1;
    return OK;
}

API hipError_t hipGetDevice(int *device)
{
    if (injected_fault()) return INVALID_DEVICE;
    *device = state.current;
    return OK;
}

API hipError_t hipSetDevice(int device)
{
    if (injected_fault() || device != 0) return INVALID_DEVICE;
    state.current = device;
    return OK;
}

API hipError_t hipMemGetInfo(size_t *free_bytes, size_t *total_bytes)
{
    if (injected_fault()) return INVALID_VALUE;
    *free_bytes = *total_bytes = (size_t)1 << 30;
    return OK;
}

API hipError_t hipMalloc(void **ptr, size_t size)
{
    if (injected_fault()) return OUT_OF_MEMORY;
    *ptr = obtain(size);
    return *ptr ? OK : OUT_OF_MEMORY;
}

API hipError_t hipFree(void *ptr)
{
    give_back(ptr);
    return OK;
}

/* Flags: none, or mapped (0x2) and coherent (0x40000000), alone or
 * together; anything else is refused. */
API hipError_t hipHostMalloc(void **ptr, size_t size, unsigned flags)
{
    if (flags & ~(0x2u | 0x40000000u)) return INVALID_VALUE;
    if (injected_fault()) return OUT_OF_MEMORY;
    *ptr = obtain(size);
    return *ptr ? OK : OUT_OF_MEMORY;
}

/* Host memory is device memory here: the same address. */
API hipError_t hipHostGetDevicePointer(void **device, void *host, unsigned flags)
{
    if (!device || !host || flags) return INVALID_VALUE;
    *device = host;
    return OK;
}

API hipError_t hipHostFree(void *ptr)
{
    give_back(ptr);
    return OK;
}

API hipError_t hipMemcpyAsync(void *dst, const void *src, size_t bytes, int kind, hipStream_t stream)
{
    if (injected_fault()) return INVALID_VALUE;
    if (!stream || (kind != H2D && kind != D2H)) return INVALID_VALUE;
    if (kind == D2H) ++state.d2h;
    memcpy(dst, src, bytes);
    return OK;
}

API hipError_t hipStreamCreateWithFlags(hipStream_t *stream, unsigned flags)
{
    if (injected_fault()) return OUT_OF_MEMORY;
    if (flags != STREAM_NON_BLOCKING) return INVALID_VALUE;
    *stream = obtain(1);
    return *stream ? OK : OUT_OF_MEMORY;
}

API hipError_t hipStreamDestroy(hipStream_t stream)
{
    give_back(stream);
    return OK;
}

API hipError_t hipStreamSynchronize(hipStream_t stream)
{
    if (injected_fault()) return INVALID_VALUE;
    return stream ? OK : INVALID_VALUE;
}

/* ---- kernel library ---- */
static int blocks(unsigned type, size_t *block, size_t *bytes)
{
    switch (type) {
    case 0: *block = 1; *bytes = 4; return 0;
    case 1: case 30: *block = 1; *bytes = 2; return 0;
    case 2: *block = 32; *bytes = 18; return 0;
    case 8: *block = 32; *bytes = 34; return 0;
    case 12: *block = 256; *bytes = 144; return 0;
    case 14: *block = 256; *bytes = 210; return 0;
    default: return -1;
    }
}

/* A type the mock library declines (as the real one declines shapes it
 * cannot address), or -1 for none. */
static int declined_type = -1;
API void nya_mock_decline_type(int type) { declined_type = type; }

API unsigned nya_hip_abi_version(void) { return 2; }
API int nya_hip_weight_bytes(unsigned type, size_t rows, size_t cols, size_t *out)
{
    size_t block, bytes;
    if (!out || (int)type == declined_type || blocks(type, &block, &bytes) || !rows || !cols || cols % block) return 1;
    *out = rows * (cols / block) * bytes;
    return 0;
}
API int nya_hip_weight_layout(unsigned type)
{
    size_t block, bytes;
    if (blocks(type, &block, &bytes)) return -1;
    return type == 8 ? 1 : 0;
}
API int nya_hip_weight_pack(void *dst, const void *src, unsigned type, size_t rows, size_t cols)
{
    size_t n;
    if (injected_fault() || nya_hip_weight_bytes(type, rows, cols, &n)) return 1;
    for (size_t i = 0; i < n; ++i) ((unsigned char *)dst)[i] = ((const unsigned char *)src)[i] ^ 0x5A;
    return 0;
}
API int nya_hip_workspace_bytes(unsigned type, size_t rows, size_t cols, size_t batch, size_t *out)
{
    size_t n;
    if (!out || !batch || nya_hip_weight_bytes(type, rows, cols, &n)) return 1;
    /* The real library's GEMM asks for scratch above 8 tokens; the stand-in
     * computes without any, unless a test sets a size to report. */
    const char *ws = getenv("MOCK_HIP_GEMM_WORKSPACE");
    *out = ws && batch > 8 ? (size_t)strtoull(ws, NULL, 10) : 0;
    return 0;
}
API int nya_hip_matmul(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x, uintptr_t y,
    size_t batch, uintptr_t workspace, size_t workspace_bytes, uintptr_t stream)
{
    (void)workspace; (void)workspace_bytes;
    size_t n;
    if (!w || !x || !y || !stream || nya_hip_weight_bytes(type, rows, cols, &n)) return 1;
    if (injected_fault()) return -1;
    const unsigned char *data = (const unsigned char *)w;
    unsigned char *plain = NULL;
    if (type == 8) {
        plain = malloc(n);
        if (!plain) return -2;
        for (size_t i = 0; i < n; ++i) plain[i] = data[i] ^ 0x5A;
        data = plain;
    }
    const float *in = (const float *)x;
    float *out = (float *)y;
    for (size_t b = 0; b < batch; ++b)
        for (size_t r = 0; r < rows; ++r) {
            double sum = 0;
            for (size_t k = 0; k < cols; ++k) sum += (double)orc_value(data, type, r * cols + k) * in[b * cols + k];
            out[b * rows + r] = (float)sum;
        }
    free(plain);
    return 0;
}
/* The gated down product of one token: silu(gate) * up formed as the step
 * forms it, then the mock product; the quantized types on whole 256-column
 * groups only, as the library. */
API int nya_hip_matvec_gated(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t gate, uintptr_t up,
    uintptr_t y, uintptr_t stream)
{
    if (!gate || !up || (type != 2 && type != 8 && type != 12 && type != 14) || cols % 256) return 1;
    float *v = malloc(cols * sizeof(float));
    if (!v) return -2;
    for (size_t i = 0; i < cols; ++i) {
        const float x = ((const float *)gate)[i], u = ((const float *)up)[i];
        v[i] = x / (1.0f + expf(-x)) * u;
    }
    const int rc = nya_hip_matmul(w, type, rows, cols, (uintptr_t)v, y, 1, 0, 0, stream);
    free(v);
    return rc;
}

/* The interleaved gate|up product of one token with the gated SiLU as its
 * output; the shapes the library takes on 256 CUs (Q4_K, more than 32 rows
 * per CU); w == 0 queries. */
API int nya_hip_matvec_swiglu(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x, uintptr_t hidden,
    uintptr_t stream)
{
    if (type != 12 || rows % 32 || cols % 256 || cols > 16384 || rows <= 32 * 256) return 1;
    if (!w) return 0;
    if (!x || !hidden) return 1;
    float *y = malloc(rows * sizeof(float));
    if (!y) return -2;
    int rc = nya_hip_matmul(w, type, rows, cols, x, (uintptr_t)y, 1, 0, 0, stream);
    for (size_t j = 0; !rc && j < rows / 2; ++j) {
        const float g = y[32 * (j / 16) + j % 16], u = y[32 * (j / 16) + 16 + j % 16];
        ((float *)hidden)[j] = g / (1.0f + expf(-g)) * u;
    }
    free(y);
    return rc;
}

/* The same with Gemma's GELU gate. */
API int nya_hip_matvec_geglu(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x, uintptr_t hidden,
    uintptr_t stream)
{
    if (nya_hip_matvec_swiglu(0, type, rows, cols, 0, 0, stream)) return 1;
    if (!w) return 0;
    if (!x || !hidden) return 1;
    float *y = malloc(rows * sizeof(float));
    if (!y) return -2;
    int rc = nya_hip_matmul(w, type, rows, cols, x, (uintptr_t)y, 1, 0, 0, stream);
    for (size_t j = 0; !rc && j < rows / 2; ++j) {
        const float g = y[32 * (j / 16) + j % 16], u = y[32 * (j / 16) + 16 + j % 16];
        ((float *)hidden)[j] = 0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g))) * u;
    }
    free(y);
    return rc;
}

API int nya_hip_gelu_pairs(uintptr_t gu, uintptr_t out, size_t n, size_t count, uintptr_t stream)
{
    if (!gu || !out || !n || n % 16 || !count || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t t = 0; t < count; ++t)
        for (size_t j = 0; j < n; ++j) {
            const float *row = (const float *)gu + 2 * n * t;
            const float g = row[32 * (j / 16) + j % 16], u = row[32 * (j / 16) + 16 + j % 16];
            ((float *)out)[t * n + j] =
                0.5f * g * (1.0f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g))) * u;
        }
    return 0;
}

/* One token's product added into the residual, with h * norm and 256 partial
 * sums of squares (rows in 256 runs of ceil(rows / 256), zeros past the last
 * run); the shapes the library takes on 256 CUs. w == 0 queries. */
API int nya_hip_matvec_residual(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x, uintptr_t res,
    uintptr_t norm, uintptr_t hn, uintptr_t parts, uintptr_t stream)
{
    if ((type != 2 && type != 8 && type != 12 && type != 14) || cols % 256 || cols > 20480 || rows > 64 * 256)
        return 1;
    if (!w) return 0;
    if (!x || !res || !norm || !hn || !parts) return 1;
    float *y = malloc(rows * sizeof(float));
    if (!y) return -2;
    const int rc = nya_hip_matmul(w, type, rows, cols, x, (uintptr_t)y, 1, 0, 0, stream);
    const size_t run = (rows + 255) / 256;
    double *ps = (double *)parts;
    for (size_t j = 0; j < 256; ++j) ps[j] = 0.0;
    for (size_t i = 0; !rc && i < rows; ++i) {
        float *h = (float *)res + i;
        *h += y[i];
        ((float *)hn)[i] = *h * ((const float *)norm)[i];
        ps[i / run] += (double)*h * *h;
    }
    free(y);
    return rc;
}

/* The interleaved gate|up product of hn scaled by the norm of the partial
 * sums: the mock SwiGLU product of hn * scale; its shapes. w == 0 queries. */
API int nya_hip_matvec_swiglu_scaled(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t hn,
    uintptr_t parts, float eps, uintptr_t hidden, uintptr_t stream)
{
    if (nya_hip_matvec_swiglu(0, type, rows, cols, 0, 0, stream)) return 1;
    if (!w) return 0;
    if (!hn || !parts || !hidden) return 1;
    double total = 0.0;
    for (size_t j = 0; j < 256; ++j) total += ((const double *)parts)[j];
    const float scale = (float)(1.0 / sqrt(total / (double)cols + (double)eps));
    float *xn = malloc(cols * sizeof(float));
    if (!xn) return -2;
    for (size_t i = 0; i < cols; ++i) xn[i] = ((const float *)hn)[i] * scale;
    const int rc = nya_hip_matvec_swiglu(w, type, rows, cols, (uintptr_t)xn, hidden, stream);
    free(xn);
    return rc;
}

API int nya_hip_silu_pairs(uintptr_t gu, uintptr_t out, size_t n, size_t count, uintptr_t stream)
{
    if (!gu || !out || !n || n % 16 || !count || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t t = 0; t < count; ++t)
        for (size_t j = 0; j < n; ++j) {
            const float *row = (const float *)gu + 2 * n * t;
            const float g = row[32 * (j / 16) + j % 16], u = row[32 * (j / 16) + 16 + j % 16];
            ((float *)out)[t * n + j] = g / (1.0f + expf(-g)) * u;
        }
    return 0;
}

API const char *nya_hip_kernel_name(unsigned type, size_t rows, size_t cols, size_t batch)
{
    (void)type; (void)rows; (void)cols; (void)batch;
    return "mock_matmul";
}

/* ---- resident decoder steps (include/fyodor_hip.h), computed at once on
 * the calling thread in the order the engine's CPU forward uses. */
static size_t mock_row_bytes(unsigned type, size_t cols)
{
    size_t block, bytes;
    if (blocks(type, &block, &bytes) || cols % block) return 0;
    return cols / block * bytes;
}

/* nya_hip_copy: 16-byte aligned pointers and a 16-byte multiple. */
API int nya_hip_copy(uintptr_t dst, uintptr_t src, size_t bytes, uintptr_t stream)
{
    (void)stream;
    if (!dst || !src || (dst & 15u) || (src & 15u) || (bytes & 15u)) return 1;
    memmove((void *)dst, (const void *)src, bytes);
    return 0;
}

API int nya_hip_step(uintptr_t step, unsigned token, size_t position, uintptr_t stream)
{
    if (!step || !stream) return 1;
    if (injected_fault()) return -1;
    ((uint32_t *)step)[0] = token;
    ((uint32_t *)step)[1] = (uint32_t)position;
    return 0;
}

API int nya_hip_embed(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t tokens, size_t count,
    uintptr_t out, float scale, uintptr_t stream)
{
    if (!w || !tokens || !out || !rows || !cols || !count || !stream || !isfinite(scale)) return 1;
    if (injected_fault()) return -1;
    const size_t rb = mock_row_bytes(type, cols);
    if (!rb) return 1;
    for (size_t t = 0; t < count; ++t) {
        const uint32_t token = ((const uint32_t *)tokens)[t];
        for (size_t i = 0; i < cols; ++i)
            ((float *)out)[t * cols + i] =
                token < rows ? orc_value((const unsigned char *)w + token * rb, type, i) * scale : 0.0f;
    }
    return 0;
}

API int nya_hip_rms_norm(uintptr_t x, uintptr_t residual, uintptr_t weight, uintptr_t out, size_t n, size_t count,
    float eps, uintptr_t stream)
{
    if (!x || !out || !n || !count || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t t = 0; t < count; ++t) {
        float *v = (float *)x + t * n, *o = (float *)out + t * n;
        const float *r = residual ? (const float *)residual + t * n : NULL, *wt = (const float *)weight;
        double sum = 0.0;
        for (size_t i = 0; i < n; ++i) {
            if (r) v[i] = v[i] + r[i];
            sum += (double)v[i] * v[i];
        }
        const float scale = (float)(1.0 / sqrt(sum / (double)n + eps));
        for (size_t i = 0; i < n; ++i) o[i] = v[i] * scale * (wt ? wt[i] : 1.0f);
    }
    return 0;
}

API int nya_hip_rope_qkv(uintptr_t q, size_t q_stride, uintptr_t k, size_t k_stride, uintptr_t v, size_t v_stride,
    size_t count, size_t heads, size_t kv_heads, size_t width, uintptr_t freq, uintptr_t positions, size_t capacity,
    uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    if (!q || !k || !v || !freq || !positions || !keys || !values || !count || !heads || !kv_heads || !width ||
        width % 2 || !capacity || !stream)
        return 1;
    if (injected_fault()) return -1;
    const size_t kvd = kv_heads * width;
    for (size_t t = 0; t < count; ++t) {
        const int position = ((const int *)positions)[t];
        if (position < 0 || (size_t)position >= capacity) continue;
        float *qr = (float *)q + t * q_stride;
        const float *kr = (const float *)k + t * k_stride, *vr = (const float *)v + t * v_stride;
        float *key = (float *)keys + (size_t)position * kvd, *value = (float *)values + (size_t)position * kvd;
        for (size_t h = 0; h < heads + kv_heads; ++h)
            for (size_t j = 0; j < width / 2; ++j) {
                const float angle = (float)position * ((const float *)freq)[j];
                const float c = cosf(angle), s = sinf(angle);
                const float *p = h < heads ? qr + h * width + 2 * j : kr + (h - heads) * width + 2 * j;
                float *o = h < heads ? qr + h * width + 2 * j : key + (h - heads) * width + 2 * j;
                const float a = p[0], b = p[1];
                o[0] = a * c - b * s;
                o[1] = a * s + b * c;
            }
        memcpy(value, vr, kvd * sizeof(float));
    }
    return 0;
}

/* The positions [*first, *first + length) a token at p attends: [0, p]
 * within max_length, the last `window` of them when window > 0. */
static size_t mock_range(int p, size_t max_length, size_t window, size_t *first)
{
    *first = 0;
    if (p < 0) return 0;
    const size_t end = (size_t)p >= max_length ? max_length - 1 : (size_t)p;
    if (window && end >= window) *first = end - window + 1;
    return end - *first + 1;
}

API int nya_hip_attention(uintptr_t q, size_t q_stride, uintptr_t keys, uintptr_t values, uintptr_t out,
    uintptr_t scores, uintptr_t positions, size_t count, size_t heads, size_t kv_heads, size_t width,
    size_t max_length, size_t window, float scale, uintptr_t stream)
{
    (void)scores;
    if (!q || !keys || !values || !out || !positions || !count || !heads || !kv_heads || heads % kv_heads ||
        !width || !max_length || !stream)
        return 1;
    if (injected_fault()) return -1;
    const size_t kvdim = kv_heads * width;
    float *sc = malloc(max_length * sizeof(float));
    if (!sc) return -1;
    for (size_t i = 0; i < count; ++i) {
        size_t first;
        const size_t length = mock_range(((const int *)positions)[i], max_length, window, &first);
        const float *kb = (const float *)keys + first * kvdim, *vb = (const float *)values + first * kvdim;
        for (size_t h = 0; h < heads && length; ++h) {
            const float *qh = (const float *)q + i * q_stride + h * width;
            const size_t kvh = h / (heads / kv_heads);
            float m = -INFINITY, sum = 0.f;
            for (size_t t = 0; t < length; ++t) {
                const float *k = kb + t * kvdim + kvh * width;
                float s = 0.f;
                for (size_t j = 0; j < width; ++j) s += qh[j] * k[j];
                sc[t] = s * scale;
                if (sc[t] > m) m = sc[t];
            }
            for (size_t t = 0; t < length; ++t) {
                sc[t] = expf(sc[t] - m);
                sum += sc[t];
            }
            for (size_t t = 0; t < length; ++t) sc[t] /= sum;
            for (size_t j = 0; j < width; ++j) {
                float acc = 0.f;
                for (size_t t = 0; t < length; ++t) acc += sc[t] * vb[t * kvdim + kvh * width + j];
                ((float *)out)[(i * heads + h) * width + j] = acc;
            }
        }
    }
    free(sc);
    return 0;
}

/* The split form: the same result computed through per-split partial
 * softmaxes, written to `partials` first ([count][heads][splits][width],
 * then [count][heads][splits][2] maxima and sums) and combined from there,
 * so the plan's scratch sizing and arguments are exercised. q == 0 is the
 * shape query. */
API int nya_hip_attention_split(uintptr_t q, size_t q_stride, uintptr_t keys, uintptr_t values, uintptr_t out,
    uintptr_t partials, uintptr_t positions, size_t count, size_t heads, size_t kv_heads, size_t width,
    size_t max_length, size_t window, size_t splits, float scale, uintptr_t stream)
{
    if (!heads || !kv_heads || heads % kv_heads || !width || !max_length || !splits ||
        (max_length + splits - 1) / splits > 1024)
        return 1;
    if (!q) return 0;
    if (!keys || !values || !out || !partials || !positions || !count || !stream) return 1;
    if (injected_fault()) return -1;
    const size_t kvdim = kv_heads * width;
    float *o = (float *)partials, *ml = o + count * heads * splits * width;
    for (size_t i = 0; i < count; ++i) {
        size_t first;
        const size_t length = mock_range(((const int *)positions)[i], max_length, window, &first);
        if (!length) continue;
        const float *kb = (const float *)keys + first * kvdim, *vb = (const float *)values + first * kvdim;
        const size_t chunk = (length + splits - 1) / splits;
        for (size_t h = 0; h < heads; ++h) {
            const float *qh = (const float *)q + i * q_stride + h * width;
            const size_t kvh = h / (heads / kv_heads);
            for (size_t sp = 0; sp < splits; ++sp) {
                const size_t row = (i * heads + h) * splits + sp, c0 = sp * chunk;
                const size_t c1 = c0 + chunk < length ? c0 + chunk : length;
                float m = -INFINITY, l = 0.f;
                for (size_t t = c0; t < c1; ++t) {
                    const float *k = kb + t * kvdim + kvh * width;
                    float sdot = 0.f;
                    for (size_t j = 0; j < width; ++j) sdot += qh[j] * k[j];
                    if (sdot * scale > m) m = sdot * scale;
                }
                for (size_t j = 0; j < width; ++j) o[row * width + j] = 0.f;
                for (size_t t = c0; t < c1; ++t) {
                    const float *k = kb + t * kvdim + kvh * width;
                    float sdot = 0.f;
                    for (size_t j = 0; j < width; ++j) sdot += qh[j] * k[j];
                    const float e = expf(sdot * scale - m);
                    l += e;
                    for (size_t j = 0; j < width; ++j) o[row * width + j] += e * vb[t * kvdim + kvh * width + j];
                }
                ml[2 * row] = c0 < c1 ? m : -INFINITY;
                ml[2 * row + 1] = l;
            }
            float mx = -INFINITY;
            for (size_t sp = 0; sp < splits; ++sp)
                if (ml[2 * ((i * heads + h) * splits + sp)] > mx) mx = ml[2 * ((i * heads + h) * splits + sp)];
            for (size_t j = 0; j < width; ++j) {
                float num = 0.f, den = 0.f;
                for (size_t sp = 0; sp < splits; ++sp) {
                    const size_t row = (i * heads + h) * splits + sp;
                    if (ml[2 * row] == -INFINITY) continue;
                    const float f = expf(ml[2 * row] - mx);
                    den += ml[2 * row + 1] * f;
                    num += o[row * width + j] * f;
                }
                ((float *)out)[(i * heads + h) * width + j] = num / den;
            }
        }
    }
    return 0;
}

API int nya_hip_silu_mul(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride, uintptr_t out,
    size_t n, size_t count, uintptr_t stream)
{
    if (!gate || !up || !out || !n || !count || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t t = 0; t < count; ++t)
        for (size_t i = 0; i < n; ++i) {
            const float x = ((const float *)gate)[t * gate_stride + i], u = ((const float *)up)[t * up_stride + i];
            ((float *)out)[t * n + i] = x / (1.0f + expf(-x)) * u;
        }
    return 0;
}

API int nya_hip_gelu_mul(uintptr_t gate, size_t gate_stride, uintptr_t up, size_t up_stride, uintptr_t out,
    size_t n, size_t count, uintptr_t stream)
{
    if (!gate || !up || !out || !n || !count || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t t = 0; t < count; ++t)
        for (size_t i = 0; i < n; ++i) {
            const float x = ((const float *)gate)[t * gate_stride + i], u = ((const float *)up)[t * up_stride + i];
            ((float *)out)[t * n + i] = 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x))) * u;
        }
    return 0;
}

/* One row's RMS norm as the engine's (sum of squares in double). */
static void mock_norm(float *out, const float *in, const float *w, size_t n, float eps)
{
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) sum += (double)in[i] * in[i];
    const float scale = (float)(1.0 / sqrt(sum / (double)n + eps));
    for (size_t i = 0; i < n; ++i) out[i] = in[i] * scale * (w ? w[i] : 1.0f);
}

API int nya_hip_post_norm(uintptr_t x, uintptr_t residual, uintptr_t post, float output_scale, uintptr_t weight,
    uintptr_t out, size_t n, size_t count, float eps, uintptr_t stream)
{
    if (!x || !out || !n || n > 16384 || !count || !stream || (post && !residual)) return 1;
    if (injected_fault()) return -1;
    float *r = malloc(n * sizeof(float));
    if (!r) return -2;
    for (size_t t = 0; t < count; ++t) {
        float *v = (float *)x + t * n;
        if (residual) {
            const float *rr = (const float *)residual + t * n;
            if (post) mock_norm(r, rr, (const float *)post, n, eps);
            else memcpy(r, rr, n * sizeof(float));
            for (size_t i = 0; i < n; ++i) v[i] += r[i];
        }
        for (size_t i = 0; i < n; ++i) v[i] *= output_scale;
        mock_norm((float *)out + t * n, v, (const float *)weight, n, eps);
    }
    free(r);
    return 0;
}

API int nya_hip_head_norm_rope(uintptr_t q, size_t q_stride, uintptr_t k, size_t k_stride, uintptr_t v,
    size_t v_stride, size_t count, size_t heads, size_t kv_heads, size_t width, uintptr_t q_norm, uintptr_t k_norm,
    float eps, uintptr_t freq, uintptr_t positions, size_t capacity, uintptr_t keys, uintptr_t values,
    uintptr_t stream)
{
    if (!q || !q_norm || !freq || !positions || !count || !heads || !kv_heads || !width || width % 2 || width > 512 ||
        !capacity || !stream || (k && (!v || !k_norm || !keys || !values)))
        return 1;
    if (injected_fault()) return -1;
    const size_t kvd = kv_heads * width, half = width / 2;
    float row[512];
    for (size_t t = 0; t < count; ++t) {
        const int position = ((const int *)positions)[t];
        if (position < 0 || (size_t)position >= capacity) continue;
        for (size_t h = 0; h < heads + (k ? 2 * kv_heads : 0); ++h) {
            const int kind = h < heads ? 0 : h < heads + kv_heads ? 1 : 2;
            const size_t hh = kind == 0 ? h : kind == 1 ? h - heads : h - heads - kv_heads;
            const float *src = kind == 0 ? (const float *)q + t * q_stride + hh * width
                             : kind == 1 ? (const float *)k + t * k_stride + hh * width
                                         : (const float *)v + t * v_stride + hh * width;
            float *dst = kind == 0 ? (float *)q + t * q_stride + hh * width
                       : (kind == 1 ? (float *)keys : (float *)values) + (size_t)position * kvd + hh * width;
            mock_norm(row, src, kind == 0 ? (const float *)q_norm : kind == 1 ? (const float *)k_norm : NULL, width,
                      eps);
            if (kind == 2) {
                memcpy(dst, row, width * sizeof(float));
                continue;
            }
            for (size_t j = 0; j < half; ++j) {
                const float angle = (float)position * ((const float *)freq)[j];
                const float c = cosf(angle), s = sinf(angle), a = row[j], b = row[j + half];
                dst[j] = a * c - b * s;
                dst[j + half] = b * c + a * s;
            }
        }
    }
    return 0;
}

API int nya_hip_softcap(uintptr_t x, size_t n, float cap, uintptr_t stream)
{
    if (!x || !n || !(cap > 0.0f) || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t i = 0; i < n; ++i) ((float *)x)[i] = cap * tanhf(((float *)x)[i] / cap);
    return 0;
}

API int nya_hip_greedy(uintptr_t logits, size_t n, size_t count, uintptr_t mask, uintptr_t ids, uintptr_t stream)
{
    if (!logits || !ids || !n || !count || !stream) return 1;
    if (injected_fault()) return -1;
    for (size_t t = 0; t < count; ++t) {
        const float *row = (const float *)logits + t * n;
        const uint32_t *m = (const uint32_t *)mask;
        int bad = 0;
        size_t best = n;
        for (size_t i = 0; i < n; ++i) {
            if (!isfinite(row[i])) bad = 1;
            if (m && ((m[i / 32] >> (i % 32)) & 1u)) continue;
            if (best == n || row[i] > row[best]) best = i;
        }
        ((uint32_t *)ids)[t] = bad || best == n ? 0xFFFFFFFFu : (uint32_t)best;
    }
    return 0;
}

/* One token's product of the normalized residual: the mock norm (into hout
 * when r is given, x left as it is) and the mock product; the shapes the
 * library takes on 256 CUs. w == 0 queries. */
API int nya_hip_matvec_normed(uintptr_t w, unsigned type, size_t rows, size_t cols, uintptr_t x, uintptr_t r,
    uintptr_t norm, float eps, uintptr_t hout, uintptr_t y, uintptr_t stream)
{
    if ((type != 2 && type != 8 && type != 12 && type != 14) || cols % 256 || cols > 4096 || rows > 32 * 256) return 1;
    if (!w) return 0;
    if (!x || !norm || !y || (r && !hout)) return 1;
    float *xn = malloc(cols * sizeof(float));
    if (!xn) return -2;
    uintptr_t h = x;
    if (r) {
        memcpy((void *)hout, (const void *)x, cols * sizeof(float));
        h = hout;
    }
    int rc = nya_hip_rms_norm(h, r, norm, (uintptr_t)xn, cols, 1, eps, stream);
    if (!rc) rc = nya_hip_matmul(w, type, rows, cols, (uintptr_t)xn, y, 1, 0, 0, stream);
    free(xn);
    return rc;
}

/* The rotary step over q|k|v rows [first_row, first_row + rows) held in y
 * (y[i] is row first_row + i), as nya_hip_rope_qkv treats those rows. */
static void mock_rope_part(float *y, size_t first_row, size_t rows, size_t heads, size_t kv_heads, size_t width,
    const float *freq, int position, size_t capacity, float *keys, float *values)
{
    if (position < 0 || (size_t)position >= capacity) return;
    const size_t qd = heads * width, kvd = kv_heads * width;
    for (size_t i = 0; i < rows; i += 2) {
        const size_t row = first_row + i;
        if (row >= qd + kvd) {
            values[(size_t)position * kvd + row - qd - kvd] = y[i];
            values[(size_t)position * kvd + row + 1 - qd - kvd] = y[i + 1];
            continue;
        }
        const size_t e = row < qd ? row : row - qd;
        const float angle = (float)position * freq[(e % width) / 2];
        const float c = cosf(angle), sn = sinf(angle), a = y[i], b = y[i + 1];
        const float o0 = a * c - b * sn, o1 = a * sn + b * c;
        if (row < qd) {
            y[i] = o0;
            y[i + 1] = o1;
        } else {
            keys[(size_t)position * kvd + e] = o0;
            keys[(size_t)position * kvd + e + 1] = o1;
        }
    }
}

/* The normed q|k|v product (or one part of its rows) with the rotary step:
 * the two mock steps. */
API int nya_hip_matvec_normed_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row, uintptr_t x,
    uintptr_t r, uintptr_t norm, float eps, uintptr_t hout, uintptr_t y, uintptr_t positions, uintptr_t freq,
    size_t heads, size_t kv_heads, size_t width, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    if (nya_hip_matvec_normed(0, type, rows, cols, 0, 0, 0, eps, 0, 0, stream) || rows % 2 ||
        ((rows + 255) / 256) % 2)
        return 1;
    if (!w) return 0;
    if (!heads || !kv_heads || !width || width % 2 || first_row % 2 ||
        first_row + rows > (heads + 2 * kv_heads) * width)
        return 1;
    int rc = nya_hip_matvec_normed(w, type, rows, cols, x, r, norm, eps, hout, y, stream);
    if (!rc)
        mock_rope_part((float *)y, first_row, rows, heads, kv_heads, width, (const float *)freq,
                       ((const int *)positions)[0], capacity, (float *)keys, (float *)values);
    return rc;
}

/* Both parts of q|k|v stored in two types (Q4_K then Q6_K) in one call:
 * the per-part mock steps; the shapes the library takes on 256 CUs (its
 * workgroup split between the parts by bytes). */
API int nya_hip_matvec_scaled_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row,
    uintptr_t hn, uintptr_t parts, float eps, uintptr_t y, uintptr_t positions, uintptr_t freq, size_t heads,
    size_t kv_heads, size_t width, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream);

API int nya_hip_matvec_rope_pair(uintptr_t w0, unsigned type0, size_t rows0, uintptr_t w1, unsigned type1,
    size_t rows1, size_t cols, uintptr_t x, uintptr_t r, uintptr_t norm, uintptr_t hout, uintptr_t parts, float eps,
    uintptr_t y, uintptr_t positions, uintptr_t freq, size_t heads, size_t kv_heads, size_t width, size_t capacity,
    uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    if (type0 != 12 || type1 != 14 || !rows0 || !rows1 || rows0 % 2 || rows1 % 2 || cols % 256 || cols > 4096)
        return 1;
    /* The stand-in runs the per-part steps: each part must take them. */
    if (nya_hip_matvec_normed_rope(0, type0, rows0, cols, 0, 0, 0, 0, eps, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, stream) ||
        nya_hip_matvec_normed_rope(0, type1, rows1, cols, 0, 0, 0, 0, eps, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, stream))
        return 1;
    /* The library's split: the 256 CUs shared by the parts' bytes. */
    const double b0 = (double)rows0 * (cols / 256) * 144, b1 = (double)rows1 * (cols / 256) * 210;
    size_t wgs1 = (size_t)(256 * b1 / (b0 + b1) + 0.5);
    wgs1 = wgs1 < 1 ? 1 : wgs1 > 255 ? 255 : wgs1;
    size_t rw1 = (rows1 + wgs1 - 1) / wgs1;
    rw1 += rw1 % 2;
    wgs1 = (rows1 + rw1 - 1) / rw1;
    const size_t wgs0 = 256 - wgs1;
    size_t rw0 = (rows0 + wgs0 - 1) / wgs0;
    rw0 += rw0 % 2;
    if (rw0 > 32 || rw1 > 32) return 1;
    if (!w0) return 0;
    if (!w1 || !x || !y || rows0 + rows1 != (heads + 2 * kv_heads) * width) return 1;
    if (parts) {
        for (int k = 0; k < 2; ++k) {
            const int rc = nya_hip_matvec_scaled_rope(k ? w1 : w0, k ? type1 : type0, k ? rows1 : rows0, cols,
                                                      k ? rows0 : 0, x, parts, eps, y + (k ? 4 * rows0 : 0),
                                                      positions, freq, heads, kv_heads, width, capacity, keys, values,
                                                      stream);
            if (rc) return rc;
        }
        return 0;
    }
    int rc = nya_hip_matvec_normed_rope(w0, type0, rows0, cols, 0, x, r, norm, eps, hout, y, positions, freq, heads,
                                        kv_heads, width, capacity, keys, values, stream);
    if (!rc)
        rc = nya_hip_matvec_normed_rope(w1, type1, rows1, cols, rows0, r ? hout : x, 0, norm, eps, 0, y + 4 * rows0,
                                        positions, freq, heads, kv_heads, width, capacity, keys, values, stream);
    return rc;
}

API int nya_hip_matvec_scaled_rope(uintptr_t w, unsigned type, size_t rows, size_t cols, size_t first_row,
    uintptr_t hn, uintptr_t parts, float eps, uintptr_t y, uintptr_t positions, uintptr_t freq, size_t heads,
    size_t kv_heads, size_t width, size_t capacity, uintptr_t keys, uintptr_t values, uintptr_t stream)
{
    if (nya_hip_matvec_normed_rope(0, type, rows, cols, 0, 0, 0, 0, eps, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, stream))
        return 1;
    if (!w) return 0;
    if (!hn || !parts || !y || !heads || !kv_heads || !width || width % 2 || first_row % 2 ||
        first_row + rows > (heads + 2 * kv_heads) * width)
        return 1;
    double total = 0.0;
    for (size_t j = 0; j < 256; ++j) total += ((const double *)parts)[j];
    const float scale = (float)(1.0 / sqrt(total / (double)cols + (double)eps));
    float *xn = malloc(cols * sizeof(float));
    if (!xn) return -2;
    for (size_t i = 0; i < cols; ++i) xn[i] = ((const float *)hn)[i] * scale;
    int rc = nya_hip_matmul(w, type, rows, cols, (uintptr_t)xn, y, 1, 0, 0, stream);
    free(xn);
    if (!rc)
        mock_rope_part((float *)y, first_row, rows, heads, kv_heads, width, (const float *)freq,
                       ((const int *)positions)[0], capacity, (float *)keys, (float *)values);
    return rc;
}
