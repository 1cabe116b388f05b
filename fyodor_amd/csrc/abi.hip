// extern "C" entry points of libfyodor_hip.so (declared in include/fyodor_hip.h).
#include <limits.h>
#include <stdint.h>
#include <string.h>
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

// Batches above the small-N kernels' 8 columns go to the prefill GEMM
// (every block format).
bool use_prefill(unsigned type, size_t cols, size_t batch)
{
    (void)cols;
    return batch > 8 && (type == Q4_K || type == Q6_K || type == Q8_0 || type == Q4_0);
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
    if (use_prefill(type, cols, batch) && fits && workspace_bytes >= prefill_workspace(type, (int)cols, (int)batch))
        return status(launch_prefill(type, wp, (const float *)x, (float *)y, (int)rows, (int)cols, (int)batch,
                                     (void *)workspace, s));
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
    *bytes = use_prefill(type, cols, batch) ? prefill_workspace(type, (int)cols, (int)batch)
           : dense || smalln_rows_supported(type, (int)rows, (int)cols, n) ? 0 : smalln_workspace((int)cols, n);
    return 0;
}

NYA_HIP_EXPORT int nya_hip_matmul(uintptr_t w, unsigned type, size_t rows, size_t cols,
    uintptr_t x, uintptr_t y, size_t batch, uintptr_t workspace, size_t workspace_bytes, uintptr_t stream)
{
    return matmul_impl(w, type, rows, cols, x, y, batch, workspace, workspace_bytes, stream);
}

NYA_HIP_EXPORT const char *nya_hip_kernel_name(unsigned type, size_t rows, size_t cols, size_t batch)
{
    size_t b;
    if (!batch || batch > INT_MAX || !storage_bytes(type, rows, cols, &b)) return NULL;
    if (type == F32 || type == F16 || type == BF16) return "skinny_dense";
    if (use_prefill(type, cols, batch)) return prefill_kernel(type);
    if (batch == 1 && matvec_supported(type, (int)rows, (int)cols)) return matvec_kernel(type, (int)rows, (int)cols);
    return smalln_rows_supported(type, (int)rows, (int)cols, (int)batch) ? "smalln_rows" : "smalln_mfma";
}

NYA_HIP_EXPORT int nya_hip_copy(uintptr_t dst, uintptr_t src, size_t bytes, uintptr_t stream)
{
    if (!dst || !src || (dst & 15u) || (src & 15u) || (bytes & 15u)) return 1;
    return status(launch_copy((uint4 *)dst, (const uint4 *)src, bytes / 16, (hipStream_t)stream));
}

}  // extern "C"
