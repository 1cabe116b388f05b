/* ROCm provider for the engine's compute layer on one MI355X: quantized
 * GGUF matrices stay packed in HBM and are multiplied by the gfx950 kernels
 * of libfyodor_hip.so (the reference provider, rocm/rocm.c, expanded them
 * to F32 on the host and called rocblas_sgemm).
 *
 * Resources, per session (one context = one device, one stream):
 *  - a device arena holding the three per-call buffers, x | y | kernel
 *    workspace, each region starting on a 256-byte boundary; one allocation
 *    that only grows;
 *  - a pinned (page-locked) host staging area, x | y: x is DMA-copied from
 *    it, and y is either DMA-copied into it or, up to 1 MiB, written into it
 *    by the kernel itself (pinned host memory is device-accessible);
 *  - the weight cache (vendor.c): device copies of caller weights in the
 *    kernel library's layout, keyed by source address, least recently used
 *    first out, charged with the arena against one budget.
 * A call stages x, enqueues upload, kernel (and download) on the stream and
 * waits once; weights are uploaded (and waited for) only on a cache miss.
 *
 * Behaviour kept from the engine's provider contract
 * (backend/include/compute_backend.h:12-29, backend/include/compute.h):
 *  - vtable, name "rocm", capabilities MATVEC | QUANTIZED | MATMUL;
 *  - synchronous calls on host buffers, W [rows][cols] GGUF row-major,
 *    X [batch][cols], Y [batch][rows]; the call returns after Y is written;
 *  - the cache budget is free VRAM minus max(10 %, 256 MiB) or
 *    NYA_ROCM_CACHE_MIB;
 *  - an unsupported type or shape declines (-1) with nothing touched and the
 *    provider still active; a runtime failure prints one line, makes the
 *    provider inactive for good (the engine then reports "cpu") and returns
 *    -1 for the caller to recompute on the CPU;
 *  - the calling thread's current device is restored after every call;
 *  - creation runs one real 2x2 dispatch before reporting success.
 *
 * Environment: NYA_ROCM_HIP_LIBRARY, NYA_ROCM_KERNEL_LIBRARY,
 * NYA_ROCM_DEVICE, NYA_ROCM_CACHE_MIB. Plain C; no HIP headers. */
#include "compute_backend.h"
#include "llm_internal.h"
#include "vendor.h"
#include "abi.h"
#include <errno.h>
#include <limits.h>
#include <math.h>
#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define REGION_ALIGN ((size_t)256)
/* Outputs up to this size are written by the kernel into pinned host memory. */
#define DIRECT_OUTPUT_BYTES ((size_t)1 << 20)

/* One region of the arena or of the staging area: how many bytes the
 * largest request so far needed (what the budget and the statistics
 * count), and where it starts. */
typedef struct region {
    size_t need;
    size_t offset;
} region;

typedef struct session {
    nya_hip_runtime hip;
    nya_kernel_library kern;
    nya_resident_ops resident;  /* optional: resident plans need them */
    bool has_resident;
    nya_hip_graphs graphs;      /* optional: resident decode tokens as one graph */
    bool has_graphs;
    void *hip_module, *kernel_module;
    int device;
    bool broken;
    hipStream_t stream;
    unsigned char *arena;       /* device: x | y | workspace */
    size_t arena_bytes;
    region dx, dy, dw;
    unsigned char *staging;     /* pinned host: x | y */
    size_t staging_bytes;
    nya_vendor_cache weights;
    nya_compute_stats counters;
} session;

static size_t round_up(size_t v) { return (v + REGION_ALIGN - 1) / REGION_ALIGN * REGION_ALIGN; }

/* A runtime failure: report it once per failing call and retire the
 * session. Returns -1 so call sites can `return broke(...)`. */
static int broke(session *s, long long status, const char *what)
{
    fprintf(stderr, "ROCm provider: %s returned status %lld; the provider retires and the CPU kernels take over\n", what, status);
    s->broken = true;
    return -1;
}

/* Runs one HIP call; nonzero status retires the session. */
static int hip_ok(session *s, hipError_t status, const char *what)
{
    return status == hipSuccess ? 0 : broke(s, (long long)status, what);
}

/* ---- device selection ---------------------------------------------------- */

/* Makes the session's device current, remembering the caller's. */
static int borrow_device(session *s, int *callers)
{
    if (hip_ok(s, s->hip.get_device(callers), "device query")) return -1;
    return hip_ok(s, s->hip.set_device(s->device), "device selection");
}

static int return_device(session *s, int callers)
{
    return hip_ok(s, s->hip.set_device(callers), "return to the caller's device");
}

/* ---- arena and staging ------------------------------------------------------ */

static void drop_weight(void *opaque, void *device_copy)
{
    session *s = opaque;
    if (device_copy) (void)hip_ok(s, s->hip.device_free(device_copy), "release of a weight copy");
}

static size_t region_bytes(const session *s)
{
    return s->dx.need + s->dy.need + s->dw.need;
}

/* Lays the three device regions out for the larger of the current and the
 * requested sizes; grows the arena and the staging area when the layout no
 * longer fits. Every call waits for its stream before returning, so nothing
 * is in flight in the old buffers when they are replaced. */
static int fit_buffers(session *s, size_t x_bytes, size_t y_bytes, size_t w_bytes)
{
    region dx = {x_bytes > s->dx.need ? x_bytes : s->dx.need, 0};
    region dy = {y_bytes > s->dy.need ? y_bytes : s->dy.need, 0};
    region dw = {w_bytes > s->dw.need ? w_bytes : s->dw.need, 0};
    if (dx.need > SIZE_MAX / 4 || dy.need > SIZE_MAX / 4 || dw.need > SIZE_MAX / 4)
        return broke(s, -1, "scratch size");
    dy.offset = round_up(dx.need);
    dw.offset = dy.offset + round_up(dy.need);
    const size_t arena = dw.offset + round_up(dw.need);
    const size_t staging = round_up(dx.need) + round_up(dy.need);
    if (arena > s->arena_bytes) {
        /* The weights give way first: the arena is charged to the same budget. */
        if (nya_vendor_reserve(&s->weights, 0, arena, drop_weight, s)) return broke(s, -1, "arena budget");
        if (s->arena && hip_ok(s, s->hip.device_free(s->arena), "free scratch")) return -1;
        s->arena = NULL;
        s->arena_bytes = 0;
        void *p = NULL;
        if (hip_ok(s, s->hip.device_alloc(&p, arena), "allocate scratch")) return -1;
        s->arena = p;
        s->arena_bytes = arena;
    }
    if (staging > s->staging_bytes) {
        if (s->staging && hip_ok(s, s->hip.pinned_free(s->staging), "free staging")) return -1;
        s->staging = NULL;
        s->staging_bytes = 0;
        void *p = NULL;
        if (hip_ok(s, s->hip.pinned_alloc(&p, staging, 0), "allocate staging")) return -1;
        s->staging = p;
        s->staging_bytes = staging;
    }
    s->dx = dx;
    s->dy = dy;
    s->dw = dw;
    return s->broken ? -1 : 0;
}

/* ---- weights ---------------------------------------------------------------- */

/* The device copy of a caller's weights: a cache hit, or a new copy in the
 * kernel library's layout (packed on the host when it differs from GGUF),
 * uploaded and waited for, then cached. NULL on failure (session retired). */
static void *device_weights(session *s, const void *source, size_t rows, size_t cols, unsigned type, size_t bytes)
{
    nya_vendor_weight *hit = nya_vendor_find(&s->weights, source, rows, cols, type);
    if (hit) return hit->value;
    if (nya_vendor_reserve(&s->weights, bytes, s->arena_bytes, drop_weight, s)) {
        (void)broke(s, -1, "cache budget");
        return NULL;
    }
    const int layout = s->kern.weight_layout(type);
    nya_vendor_weight *entry = calloc(1, sizeof(*entry));
    unsigned char *packed = layout == 1 ? malloc(bytes) : NULL;
    void *copy = NULL;
    if (!entry || layout < 0 || (layout == 1 && !packed)) {
        (void)broke(s, -1, "host weight buffer");
        goto fail;
    }
    if (packed && s->kern.weight_pack(packed, source, type, rows, cols)) {
        (void)broke(s, -1, "pack weight");
        goto fail;
    }
    if (hip_ok(s, s->hip.device_alloc(&copy, bytes), "device copy of a weight")) goto fail;
    if (hip_ok(s, s->hip.copy_async(copy, packed ? packed : source, bytes, hipMemcpyHostToDevice, s->stream),
               "weight copy to the device")) goto drain;
    ++s->counters.uploads;
    /* The host copy belongs to this call: the upload must end first. */
    ++s->counters.synchronizations;
    if (hip_ok(s, s->hip.stream_wait(s->stream), "wait for the weight copy")) goto fail;
    free(packed);
    entry->source = source;
    entry->rows = rows;
    entry->columns = cols;
    entry->type = type;
    entry->bytes = bytes;
    entry->value = copy;
    nya_vendor_insert(&s->weights, entry);
    return copy;
drain:
    /* A copy that may have been enqueued reads `packed`: wait before freeing. */
    (void)hip_ok(s, s->hip.stream_wait(s->stream), "wait after a failed weight copy");
fail:
    drop_weight(s, copy);
    free(entry);
    free(packed);
    return NULL;
}

/* ---- one request -------------------------------------------------------------- */

/* Y[batch][rows] = X[batch][cols] . W^T. */
static int run(void *opaque, const void *source, size_t rows, size_t cols, unsigned type, const float *x, float *y,
    size_t batch)
{
    session *s = opaque;
    size_t f32_bytes, x_bytes, y_bytes, w_bytes, ws_bytes;
    /* Declines (the request is unsupported): nothing touched, still active. */
    if (!s || s->broken || !source || !x || !y) return -1;
    if (nya_vendor_matrix(rows, cols, batch, type, &f32_bytes, &x_bytes, &y_bytes)) return -1;
    if (s->kern.weight_bytes(type, rows, cols, &w_bytes)) return -1;
    if (s->kern.workspace_bytes(type, rows, cols, batch, &ws_bytes)) return -1;

    int callers = 0;
    if (borrow_device(s, &callers)) return -1;
    int status = -1;
    bool waited = false;
    if (fit_buffers(s, x_bytes, y_bytes, ws_bytes)) goto out;
    void *w = device_weights(s, source, rows, cols, type, w_bytes);
    if (!w) goto out;
    unsigned char *px = s->staging, *py = s->staging + round_up(s->dx.need);
    unsigned char *dx = s->arena + s->dx.offset, *dy = s->arena + s->dy.offset, *dw = s->arena + s->dw.offset;
    /* Small outputs go straight from the kernel into the pinned staging area
     * (the device writes host memory over the bus as it finishes), which
     * saves the download's dispatch and its completion wait; large ones
     * (prefill batches) are faster as one DMA copy. */
    const bool direct = y_bytes <= DIRECT_OUTPUT_BYTES;
    memcpy(px, x, x_bytes);
    if (hip_ok(s, s->hip.copy_async(dx, px, x_bytes, hipMemcpyHostToDevice, s->stream), "input copy to the device")) goto out;
    ++s->counters.uploads;
    const int launched = s->kern.matmul((uintptr_t)w, type, rows, cols, (uintptr_t)dx,
                                        (uintptr_t)(direct ? py : dy), batch, ws_bytes ? (uintptr_t)dw : 0, ws_bytes,
                                        (uintptr_t)s->stream);
    if (launched > 0) goto out;   /* declined before enqueueing anything: still active */
    if (launched < 0) {
        (void)broke(s, launched, "quantized matmul");
        goto out;
    }
    ++s->counters.kernel_launches;
    ++s->counters.external_matmul_calls;
    if (!direct && hip_ok(s, s->hip.copy_async(py, dy, y_bytes, hipMemcpyDeviceToHost, s->stream), "output copy to the host"))
        goto out;
    ++s->counters.downloads;
    ++s->counters.synchronizations;
    waited = true;
    if (hip_ok(s, s->hip.stream_wait(s->stream), "wait for the product")) goto out;
    memcpy(y, py, y_bytes);
    status = 0;
out:
    /* Whatever was enqueued is waited for before the call returns. */
    if (!waited && s->stream) {
        ++s->counters.synchronizations;
        (void)hip_ok(s, s->hip.stream_wait(s->stream), "drain failed call");
    }
    if (return_device(s, callers)) status = -1;
    return s->broken ? -1 : status;
}

static int run_one(void *s, const void *w, size_t rows, size_t cols, unsigned type, const float *x, float *y)
{
    return run(s, w, rows, cols, type, x, y, 1);
}

static int alive(const void *opaque)
{
    const session *s = opaque;
    return s && !s->broken;
}

/* kind 0: the provider's own kernels (no vendor BLAS). */
static void report(const void *opaque, nya_compute_stats *out)
{
    const session *s = opaque;
    *out = s->counters;
    out->weights_bytes = s->weights.bytes;
    out->scratch_bytes = region_bytes(s);
    out->external_matmul_kind = 0;
}

/* ---- lifetime ------------------------------------------------------------------- */

/* Releases everything the session owns; every release is attempted even
 * when the device is gone or selecting it fails. */
static void close_session(void *opaque)
{
    session *s = opaque;
    if (!s) return;
    if (s->stream) {
        int callers = 0;
        const bool selected = !borrow_device(s, &callers);
        (void)hip_ok(s, s->hip.stream_wait(s->stream), "final wait before release");
        nya_vendor_clear(&s->weights, drop_weight, s);
        if (s->arena) (void)hip_ok(s, s->hip.device_free(s->arena), "free scratch");
        if (s->staging) (void)hip_ok(s, s->hip.pinned_free(s->staging), "free staging");
        (void)hip_ok(s, s->hip.stream_destroy(s->stream), "stream release");
        if (selected) (void)return_device(s, callers);
    }
    nya_vendor_close(s->kernel_module);
    nya_vendor_close(s->hip_module);
    free(s);
}

/* Resolves both tables; the kernel library must speak this provider's ABI. */
static int bind_all(session *s)
{
    const struct { void *module; const char *symbol; void *slot; size_t size; } table[] = {
        {s->hip_module, "hipInit", &s->hip.init, sizeof s->hip.init},
        {s->hip_module, "hipGetDeviceCount", &s->hip.device_count, sizeof s->hip.device_count},
        {s->hip_module, "hipGetDevice", &s->hip.get_device, sizeof s->hip.get_device},
        {s->hip_module, "hipSetDevice", &s->hip.set_device, sizeof s->hip.set_device},
        {s->hip_module, "hipMemGetInfo", &s->hip.memory_info, sizeof s->hip.memory_info},
        {s->hip_module, "hipMalloc", &s->hip.device_alloc, sizeof s->hip.device_alloc},
        {s->hip_module, "hipFree", &s->hip.device_free, sizeof s->hip.device_free},
        {s->hip_module, "hipHostMalloc", &s->hip.pinned_alloc, sizeof s->hip.pinned_alloc},
        {s->hip_module, "hipHostFree", &s->hip.pinned_free, sizeof s->hip.pinned_free},
        {s->hip_module, "hipMemcpyAsync", &s->hip.copy_async, sizeof s->hip.copy_async},
        {s->hip_module, "hipStreamCreateWithFlags", &s->hip.stream_create, sizeof s->hip.stream_create},
        {s->hip_module, "hipStreamDestroy", &s->hip.stream_destroy, sizeof s->hip.stream_destroy},
        {s->hip_module, "hipStreamSynchronize", &s->hip.stream_wait, sizeof s->hip.stream_wait},
        {s->kernel_module, "nya_hip_abi_version", &s->kern.abi_version, sizeof s->kern.abi_version},
        {s->kernel_module, "nya_hip_weight_bytes", &s->kern.weight_bytes, sizeof s->kern.weight_bytes},
        {s->kernel_module, "nya_hip_weight_layout", &s->kern.weight_layout, sizeof s->kern.weight_layout},
        {s->kernel_module, "nya_hip_weight_pack", &s->kern.weight_pack, sizeof s->kern.weight_pack},
        {s->kernel_module, "nya_hip_workspace_bytes", &s->kern.workspace_bytes, sizeof s->kern.workspace_bytes},
        {s->kernel_module, "nya_hip_matmul", &s->kern.matmul, sizeof s->kern.matmul},
    };
    for (size_t i = 0; i < sizeof table / sizeof table[0]; ++i)
        if (nya_vendor_symbol(table[i].module, table[i].symbol, table[i].slot, table[i].size)) return -1;
    const struct { const char *symbol; void *slot; size_t size; } resident[] = {
        {"nya_hip_step", &s->resident.step, sizeof s->resident.step},
        {"nya_hip_embed", &s->resident.embed, sizeof s->resident.embed},
        {"nya_hip_rms_norm", &s->resident.rms_norm, sizeof s->resident.rms_norm},
        {"nya_hip_rope_qkv", &s->resident.rope_qkv, sizeof s->resident.rope_qkv},
        {"nya_hip_attention", &s->resident.attention, sizeof s->resident.attention},
        {"nya_hip_silu_mul", &s->resident.silu_mul, sizeof s->resident.silu_mul},
        {"nya_hip_greedy", &s->resident.greedy, sizeof s->resident.greedy},
    };
    s->has_resident = true;
    for (size_t i = 0; i < sizeof resident / sizeof resident[0]; ++i)
        if (nya_vendor_symbol(s->kernel_module, resident[i].symbol, resident[i].slot, resident[i].size))
            s->has_resident = false;
    if (nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_gated", &s->resident.matvec_gated,
                          sizeof s->resident.matvec_gated))
        s->resident.matvec_gated = NULL;
    if (nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_normed", &s->resident.matvec_normed,
                          sizeof s->resident.matvec_normed))
        s->resident.matvec_normed = NULL;
    if (nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_normed_rope", &s->resident.matvec_normed_rope,
                          sizeof s->resident.matvec_normed_rope))
        s->resident.matvec_normed_rope = NULL;
    if (nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_swiglu", &s->resident.matvec_swiglu,
                          sizeof s->resident.matvec_swiglu) ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_silu_pairs", &s->resident.silu_pairs,
                          sizeof s->resident.silu_pairs))
        s->resident.matvec_swiglu = NULL, s->resident.silu_pairs = NULL;
    if (!s->resident.matvec_swiglu ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_residual", &s->resident.matvec_residual,
                          sizeof s->resident.matvec_residual) ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_swiglu_scaled", &s->resident.matvec_swiglu_scaled,
                          sizeof s->resident.matvec_swiglu_scaled))
        s->resident.matvec_residual = NULL, s->resident.matvec_swiglu_scaled = NULL;
    if (!s->resident.matvec_residual || !s->resident.matvec_normed_rope ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_scaled_rope", &s->resident.matvec_scaled_rope,
                          sizeof s->resident.matvec_scaled_rope))
        s->resident.matvec_scaled_rope = NULL;
    if (!s->resident.matvec_normed_rope ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_rope_pair", &s->resident.matvec_rope_pair,
                          sizeof s->resident.matvec_rope_pair))
        s->resident.matvec_rope_pair = NULL;
    if (nya_vendor_symbol(s->kernel_module, "nya_hip_attention_split", &s->resident.attention_split,
                          sizeof s->resident.attention_split))
        s->resident.attention_split = NULL;
    const struct { const char *symbol; void *slot; size_t size; } gemma[] = {
        {"nya_hip_post_norm", &s->resident.post_norm, sizeof s->resident.post_norm},
        {"nya_hip_head_norm_rope", &s->resident.head_norm_rope, sizeof s->resident.head_norm_rope},
        {"nya_hip_gelu_mul", &s->resident.gelu_mul, sizeof s->resident.gelu_mul},
        {"nya_hip_softcap", &s->resident.softcap, sizeof s->resident.softcap},
    };
    bool has_gemma = true;
    for (size_t i = 0; i < sizeof gemma / sizeof gemma[0]; ++i)
        if (nya_vendor_symbol(s->kernel_module, gemma[i].symbol, gemma[i].slot, gemma[i].size)) has_gemma = false;
    if (!has_gemma)
        s->resident.post_norm = NULL, s->resident.head_norm_rope = NULL, s->resident.gelu_mul = NULL,
        s->resident.softcap = NULL;
    if (!has_gemma ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_matvec_geglu", &s->resident.matvec_geglu,
                          sizeof s->resident.matvec_geglu) ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_gelu_pairs", &s->resident.gelu_pairs,
                          sizeof s->resident.gelu_pairs))
        s->resident.matvec_geglu = NULL, s->resident.gelu_pairs = NULL;
    if (nya_vendor_symbol(s->hip_module, "hipHostGetDevicePointer", &s->hip.host_device_pointer,
                          sizeof s->hip.host_device_pointer) ||
        nya_vendor_symbol(s->kernel_module, "nya_hip_copy", &s->resident.copy, sizeof s->resident.copy))
        s->hip.host_device_pointer = NULL, s->resident.copy = NULL;
    const struct { const char *symbol; void *slot; size_t size; } graphs[] = {
        {"hipStreamBeginCapture", &s->graphs.begin_capture, sizeof s->graphs.begin_capture},
        {"hipStreamEndCapture", &s->graphs.end_capture, sizeof s->graphs.end_capture},
        {"hipGraphInstantiateWithFlags", &s->graphs.instantiate, sizeof s->graphs.instantiate},
        {"hipGraphLaunch", &s->graphs.launch, sizeof s->graphs.launch},
        {"hipGraphExecDestroy", &s->graphs.exec_destroy, sizeof s->graphs.exec_destroy},
        {"hipGraphDestroy", &s->graphs.destroy, sizeof s->graphs.destroy},
    };
    /* NYA_ROCM_GRAPHS=0 keeps the resident plan on direct launches. */
    const char *use_graphs = getenv("NYA_ROCM_GRAPHS");
    s->has_graphs = !(use_graphs && !strcmp(use_graphs, "0"));
    for (size_t i = 0; s->has_graphs && i < sizeof graphs / sizeof graphs[0]; ++i)
        if (nya_vendor_symbol(s->hip_module, graphs[i].symbol, graphs[i].slot, graphs[i].size)) s->has_graphs = false;
    return s->kern.abi_version() == NYA_KERNEL_ABI ? 0 : -1;
}

/* NYA_ROCM_DEVICE: a decimal index below the device count, else -1. */
static int pick_device(int count)
{
    const char *text = getenv("NYA_ROCM_DEVICE");
    if (!text) return 0;
    if (text[0] < '0' || text[0] > '9') return -1;
    char *end = NULL;
    errno = 0;
    const unsigned long v = strtoul(text, &end, 10);
    return errno || *end || v >= (unsigned long)count ? -1 : (int)v;
}

static void *open_session(void)
{
    session *s = calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->hip_module = nya_vendor_open(getenv("NYA_ROCM_HIP_LIBRARY"), "libamdhip64.so");
    s->kernel_module = nya_vendor_open(getenv("NYA_ROCM_KERNEL_LIBRARY"), "libfyodor_hip.so");
    if (!s->hip_module || !s->kernel_module || bind_all(s)) goto unavailable;
    int count = 0;
    if (hip_ok(s, s->hip.init(0), "HIP initialization") || hip_ok(s, s->hip.device_count(&count), "device count") ||
        count < 1 || (s->device = pick_device(count)) < 0) goto unavailable;
    int callers = 0;
    if (borrow_device(s, &callers)) goto unavailable;
    size_t free_bytes = 0, total = 0;
    bool ready = !hip_ok(s, s->hip.memory_info(&free_bytes, &total), "memory query") &&
                 (s->weights.limit = nya_vendor_budget(free_bytes, "NYA_ROCM_CACHE_MIB")) != 0 &&
                 !hip_ok(s, s->hip.stream_create(&s->stream, NYA_HIP_STREAM_NON_BLOCKING), "stream creation");
    if (return_device(s, callers) || !ready) goto unavailable;
    /* Enumerating a device does not prove its kernels run: one real call. */
    static const float pw[4] = {1, 2, 3, 4}, px[2] = {1, 1};
    float py[2] = {0, 0};
    if (run_one(s, pw, 2, 2, 0, px, py) || py[0] != 3 || py[1] != 7) goto unavailable;
    memset(&s->counters, 0, sizeof(s->counters));
    return s;
unavailable:
    fprintf(stderr, "ROCm unavailable: verify HIP, the kernel library, device selection and memory budget; "
                    "CPU remains available\n");
    close_session(s);
    return NULL;
}

#include "resident.inc"

const nya_backend_interface *nya_rocm_backend(void)
{
    static const nya_backend_interface provider = {
        .type = NYA_BACKEND_ROCM,
        .name = "rocm",
        .capabilities = NYA_COMPUTE_MATVEC | NYA_COMPUTE_QUANTIZED | NYA_COMPUTE_MATMUL | NYA_COMPUTE_RESIDENT,
        .create = open_session,
        .destroy = close_session,
        .active = alive,
        .matvec = run_one,
        .plan_create = plan_open,
        .plan_free = plan_release,
        .plan_token = plan_token,
        .plan_prefill = plan_prefill,
        .plan_stats = plan_report,
        .matmul = run,
        .plan_read_kv = plan_read_kv,
        .context_stats = report,
    };
    return &provider;
}
