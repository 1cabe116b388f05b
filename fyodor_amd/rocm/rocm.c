/* ROCm provider for the engine's compute layer: quantized GGUF matrices are
 * kept packed in HBM and multiplied by the gfx950 kernels of
 * libfyodor_hip.so. Replaces the reference provider (rocm/rocm.c:1-199),
 * which expanded weights to F32 on the host and called rocblas_sgemm.
 *
 * Kept from the reference contract (backend/include/compute_backend.h:12-29):
 *  - the vtable, name "rocm" and capabilities MATVEC|QUANTIZED|MATMUL;
 *  - synchronous calls on host buffers: W [rows][cols] GGUF row-major,
 *    X [batch][cols], Y [batch][rows]; each call returns after Y is written;
 *  - weights are borrowed, immutable and cached by source address in an LRU
 *    bounded by free VRAM minus max(10 %, 256 MiB) or NYA_ROCM_CACHE_MIB;
 *  - an unsupported type or shape declines (-1) and leaves the provider
 *    usable; any runtime error prints one line, marks the provider failed so
 *    the engine reports "cpu", and returns -1 for the caller to recompute;
 *  - the calling thread's device is saved and restored around every call;
 *  - creation probes a real 2x2 dispatch before it succeeds.
 *
 * Environment: NYA_ROCM_HIP_LIBRARY, NYA_ROCM_KERNEL_LIBRARY,
 * NYA_ROCM_DEVICE, NYA_ROCM_CACHE_MIB. Host code is C; it needs neither a
 * HIP compiler nor HIP headers. */
#include "compute_backend.h"
#include "vendor.h"
#include "abi.h"
#include <errno.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct nya_rocm {
    nya_rocm_api api;
    void *hip_library, *kernel_library;
    void *input, *output, *workspace;
    size_t input_bytes, output_bytes, workspace_bytes;
    hipStream_t stream;
    int device, failed;
    nya_vendor_cache cache;
    nya_compute_stats stats;
} nya_rocm;

/* rocm/rocm.c:21-26: every runtime failure is sticky. */
static int checked(nya_rocm *c, long long status, const char *operation)
{
    if (!status) return 0;
    fprintf(stderr, "ROCm %s failed: status %lld; reverting to CPU execution\n", operation, status);
    c->failed = 1;
    return -1;
}

/* Kernel library calls: 0 enqueued, 1 declined before enqueue (not a
 * failure), negative HIP failure. */
static int launched(nya_rocm *c, int status, const char *operation)
{
    if (status == 0) { ++c->stats.kernel_launches; return 0; }
    if (status > 0) return 1;
    return checked(c, status, operation);
}

static void release_weight(void *state, void *value)
{
    nya_rocm *c = state;
    if (value) (void)checked(c, c->api.deallocate(value), "free weight");
}

static int enter(nya_rocm *c, int *previous)
{
    if (checked(c, c->api.get_device(previous), "get device")) return -1;
    return checked(c, c->api.set_device(c->device), "select device");
}

static void release_scratch(nya_rocm *c, void **buffer, size_t *bytes, const char *operation)
{
    if (*buffer) (void)checked(c, c->api.deallocate(*buffer), operation);
    *buffer = NULL;
    *bytes = 0;
}

/* rocm/rocm.c:37-58: release every owned resource even when the device is
 * lost or selecting it fails. */
static void destroy(void *state)
{
    nya_rocm *c = state;
    if (!c) return;
    if (c->stream) {
        int previous = 0, selected = !enter(c, &previous);
        (void)checked(c, c->api.synchronize(c->stream), "synchronize during cleanup");
        nya_vendor_clear(&c->cache, release_weight, c);
        release_scratch(c, &c->input, &c->input_bytes, "free input");
        release_scratch(c, &c->output, &c->output_bytes, "free output");
        release_scratch(c, &c->workspace, &c->workspace_bytes, "free workspace");
        (void)checked(c, c->api.stream_destroy(c->stream), "destroy stream");
        if (selected) (void)checked(c, c->api.set_device(previous), "restore device");
    }
    nya_vendor_close(c->kernel_library);
    nya_vendor_close(c->hip_library);
    free(c);
}

/* Grows one persistent scratch buffer. Every public call synchronizes before
 * returning, so the old buffer is idle and may be freed first. */
static int grow(nya_rocm *c, void **buffer, size_t *bytes, size_t want, const char *operation)
{
    if (want <= *bytes) return 0;
    release_scratch(c, buffer, bytes, operation);
    if (c->failed || checked(c, c->api.allocate(buffer, want), operation)) { *buffer = NULL; return -1; }
    *bytes = want;
    return 0;
}

/* rocm/rocm.c:59-81, plus the kernel workspace. Scratch never shrinks and is
 * charged to the same budget as cached weights. */
static int buffers(nya_rocm *c, size_t input, size_t output, size_t workspace)
{
    size_t want_input = input > c->input_bytes ? input : c->input_bytes;
    size_t want_output = output > c->output_bytes ? output : c->output_bytes;
    size_t want_work = workspace > c->workspace_bytes ? workspace : c->workspace_bytes;
    if (want_input == c->input_bytes && want_output == c->output_bytes && want_work == c->workspace_bytes) return 0;
    if (want_input > SIZE_MAX - want_output || want_work > SIZE_MAX - want_input - want_output ||
        nya_vendor_reserve(&c->cache, 0, want_input + want_output + want_work, release_weight, c))
        return checked(c, -1, "scratch budget");
    if (grow(c, &c->input, &c->input_bytes, want_input, "allocate input")) return -1;
    if (grow(c, &c->output, &c->output_bytes, want_output, "allocate output")) return -1;
    if (grow(c, &c->workspace, &c->workspace_bytes, want_work, "allocate workspace")) return -1;
    return c->failed ? -1 : 0;
}

/* rocm/rocm.c:82-110: cache lookup, else reserve, convert to the device
 * layout on the host when it differs from GGUF, upload and synchronize. */
static nya_vendor_weight *weight(nya_rocm *c, const void *source, size_t rows, size_t cols,
    unsigned type, size_t bytes)
{
    nya_vendor_weight *w = nya_vendor_find(&c->cache, source, rows, cols, type);
    if (w) return w;
    size_t scratch = c->input_bytes + c->output_bytes + c->workspace_bytes;
    if (nya_vendor_reserve(&c->cache, bytes, scratch, release_weight, c)) {
        (void)checked(c, -1, "weight budget");
        return NULL;
    }
    int layout = c->api.weight_layout(type);
    w = calloc(1, sizeof(*w));
    void *packed = layout == 1 ? malloc(bytes) : NULL;
    if (!w || layout < 0 || (layout == 1 && !packed)) {
        free(w); free(packed);
        (void)checked(c, -1, "allocate host weight");
        return NULL;
    }
    if (packed && c->api.weight_pack(packed, source, type, rows, cols)) {
        (void)checked(c, -1, "pack weight");
        goto failure;
    }
    if (checked(c, c->api.allocate(&w->value, bytes), "allocate weight")) goto failure;
    if (checked(c, c->api.copy_async(w->value, packed ? packed : source, bytes, NYA_HIP_H2D, c->stream),
        "upload weight")) goto failure;
    ++c->stats.uploads;
    /* The packed copy belongs to this call: finish the upload before freeing. */
    ++c->stats.synchronizations;
    if (checked(c, c->api.synchronize(c->stream), "finish weight upload")) goto failure;
    free(packed);
    w->source = source; w->rows = rows; w->columns = cols; w->type = type; w->bytes = bytes;
    nya_vendor_insert(&c->cache, w);
    return w;
failure:
    (void)checked(c, c->api.synchronize(c->stream), "drain failed upload");
    release_weight(c, w->value);
    free(w);
    free(packed);
    return NULL;
}

static int matmul(void *state, const void *source, size_t rows, size_t cols,
    unsigned type, const float *x, float *y, size_t batch)
{
    nya_rocm *c = state;
    size_t expanded, xb, yb, wb, sb;
    /* Declines: nothing is touched and the provider stays active. */
    if (!c || c->failed || !source || !x || !y ||
        nya_vendor_matrix(rows, cols, batch, type, &expanded, &xb, &yb) ||
        c->api.weight_bytes(type, rows, cols, &wb) ||
        c->api.workspace_bytes(type, rows, cols, batch, &sb)) return -1;
    int previous = 0, result = -1;
    if (enter(c, &previous)) return -1;
    if (buffers(c, xb, yb, sb)) goto done;
    nya_vendor_weight *w = weight(c, source, rows, cols, type, wb);
    if (!w || c->failed) goto done;
    if (checked(c, c->api.copy_async(c->input, x, xb, NYA_HIP_H2D, c->stream), "upload input")) goto done;
    ++c->stats.uploads;
    if (launched(c, c->api.matmul((uintptr_t)w->value, type, rows, cols, (uintptr_t)c->input,
        (uintptr_t)c->output, batch, (uintptr_t)c->workspace, c->workspace_bytes, (uintptr_t)c->stream),
        "quantized matmul")) goto done;
    ++c->stats.external_matmul_calls;
    if (checked(c, c->api.copy_async(y, c->output, yb, NYA_HIP_D2H, c->stream), "download output")) goto done;
    ++c->stats.downloads;
    result = 0;
done:
    ++c->stats.synchronizations;
    if (checked(c, c->api.synchronize(c->stream), "finish matrix")) result = -1;
    if (checked(c, c->api.set_device(previous), "restore device")) result = -1;
    return result;
}

static int matvec(void *c, const void *w, size_t rows, size_t cols, unsigned type, const float *x, float *y)
{
    return matmul(c, w, rows, cols, type, x, y, 1);
}

static int active(const void *state)
{
    const nya_rocm *c = state;
    return c && !c->failed;
}

/* rocm/rocm.c:141-146; kind 0 = the provider's own kernels. */
static void stats(const void *state, nya_compute_stats *out)
{
    const nya_rocm *c = state;
    *out = c->stats;
    out->weights_bytes = c->cache.bytes;
    out->scratch_bytes = c->input_bytes + c->output_bytes + c->workspace_bytes;
    out->external_matmul_kind = 0;
}

static int resolve(nya_rocm *c)
{
#define HIP(field, name) if (nya_vendor_symbol(c->hip_library, name, &c->api.field, sizeof(c->api.field))) return -1
#define KERNEL(field, name) if (nya_vendor_symbol(c->kernel_library, name, &c->api.field, sizeof(c->api.field))) return -1
    HIP(init, "hipInit"); HIP(device_count, "hipGetDeviceCount");
    HIP(get_device, "hipGetDevice"); HIP(set_device, "hipSetDevice");
    HIP(memory_info, "hipMemGetInfo"); HIP(allocate, "hipMalloc"); HIP(deallocate, "hipFree");
    HIP(copy_async, "hipMemcpyAsync"); HIP(stream_create, "hipStreamCreateWithFlags");
    HIP(stream_destroy, "hipStreamDestroy"); HIP(synchronize, "hipStreamSynchronize");
    KERNEL(kernel_version, "nya_hip_abi_version"); KERNEL(weight_bytes, "nya_hip_weight_bytes");
    KERNEL(weight_layout, "nya_hip_weight_layout"); KERNEL(weight_pack, "nya_hip_weight_pack");
    KERNEL(workspace_bytes, "nya_hip_workspace_bytes"); KERNEL(matmul, "nya_hip_matmul");
#undef HIP
#undef KERNEL
    return c->api.kernel_version() == NYA_HIP_KERNEL_ABI ? 0 : -1;
}

/* rocm/rocm.c:147-192 */
static void *create(void)
{
    nya_rocm *c = calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->hip_library = nya_vendor_open(getenv("NYA_ROCM_HIP_LIBRARY"), "libamdhip64.so");
    c->kernel_library = nya_vendor_open(getenv("NYA_ROCM_KERNEL_LIBRARY"), "libfyodor_hip.so");
    if (!c->hip_library || !c->kernel_library || resolve(c)) goto unavailable;
    int count = 0, previous = 0;
    if (checked(c, c->api.init(0), "initialize HIP") ||
        checked(c, c->api.device_count(&count), "enumerate devices") || count < 1) goto unavailable;
    const char *device = getenv("NYA_ROCM_DEVICE");
    if (device) {
        char *end = NULL;
        errno = 0;
        unsigned long value = strtoul(device, &end, 10);
        if (errno || device[0] < '0' || device[0] > '9' || *end || value >= (unsigned long)count) goto unavailable;
        c->device = (int)value;
    }
    if (enter(c, &previous)) goto unavailable;
    size_t available = 0, total = 0;
    int failed = checked(c, c->api.memory_info(&available, &total), "query memory") ||
        !(c->cache.limit = nya_vendor_budget(available, "NYA_ROCM_CACHE_MIB")) ||
        checked(c, c->api.stream_create(&c->stream, NYA_HIP_STREAM_NON_BLOCKING), "create stream");
    if (checked(c, c->api.set_device(previous), "restore initial device") || failed) goto unavailable;
    /* A device can enumerate while its kernels cannot run: dispatch once. */
    static const float probe_w[] = {1, 2, 3, 4}, probe_x[] = {1, 1};
    float probe_y[2] = {0, 0};
    if (matvec(c, probe_w, 2, 2, 0, probe_x, probe_y) || probe_y[0] != 3 || probe_y[1] != 7) goto unavailable;
    memset(&c->stats, 0, sizeof(c->stats));
    return c;
unavailable:
    fprintf(stderr, "ROCm unavailable: verify HIP, the kernel library, device selection and memory budget; CPU remains available\n");
    destroy(c);
    return NULL;
}

const nya_backend_interface *nya_rocm_backend(void)
{
    static const nya_backend_interface api = {
        .type = NYA_BACKEND_ROCM, .name = "rocm",
        .capabilities = NYA_COMPUTE_MATVEC | NYA_COMPUTE_QUANTIZED | NYA_COMPUTE_MATMUL,
        .create = create, .destroy = destroy, .active = active,
        .matvec = matvec, .matmul = matmul, .context_stats = stats};
    return &api;
}
