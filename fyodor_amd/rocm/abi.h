/* Entry points the ROCm provider resolves at run time, grouped by the shared
 * library that exports them. The HIP members keep the runtime's own names
 * and C types (the reference provider resolves the same ones,
 * rocm/abi.h:8-19); the rocBLAS members of the reference table
 * (rocm/abi.h:20-25) are replaced by the gfx950 kernel library of
 * include/fyodor_hip.h. Building the provider needs neither a HIP compiler
 * nor HIP headers. */
#ifndef NYA_ROCM_ABI_H
#define NYA_ROCM_ABI_H
#include <stddef.h>
#include <stdint.h>
#include "types.h"

/* libamdhip64 */
typedef struct nya_hip_runtime {
    hipError_t (*init)(unsigned);
    hipError_t (*device_count)(int *);
    hipError_t (*get_device)(int *);
    hipError_t (*set_device)(int);
    hipError_t (*memory_info)(size_t *, size_t *);
    hipError_t (*device_alloc)(void **, size_t);
    hipError_t (*device_free)(void *);
    hipError_t (*pinned_alloc)(void **, size_t, unsigned);
    hipError_t (*pinned_free)(void *);
    hipError_t (*copy_async)(void *, const void *, size_t, hipMemcpyKind, hipStream_t);
    hipError_t (*stream_create)(hipStream_t *, unsigned);
    hipError_t (*stream_destroy)(hipStream_t);
    hipError_t (*stream_wait)(hipStream_t);
    /* Optional: the device address of mapped pinned memory; NULL leaves the
     * resident plan downloading its logits with copy_async. */
    hipError_t (*host_device_pointer)(void **, void *, unsigned);
} nya_hip_runtime;

/* libamdhip64's stream capture and graphs. Optional: without them the
 * resident plan launches every step of a token itself. */
typedef struct nya_hip_graphs {
    hipError_t (*begin_capture)(hipStream_t, hipStreamCaptureMode);
    hipError_t (*end_capture)(hipStream_t, hipGraph_t *);
    hipError_t (*instantiate)(hipGraphExec_t *, hipGraph_t, unsigned long long);
    hipError_t (*launch)(hipGraphExec_t, hipStream_t);
    hipError_t (*exec_destroy)(hipGraphExec_t);
    hipError_t (*destroy)(hipGraph_t);
} nya_hip_graphs;

/* libfyodor_hip (include/fyodor_hip.h) */
typedef struct nya_kernel_library {
    unsigned (*abi_version)(void);
    int (*weight_bytes)(unsigned, size_t, size_t, size_t *);
    int (*weight_layout)(unsigned);
    int (*weight_pack)(void *, const void *, unsigned, size_t, size_t);
    int (*workspace_bytes)(unsigned, size_t, size_t, size_t, size_t *);
    int (*matmul)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, size_t, uintptr_t, size_t, uintptr_t);
} nya_kernel_library;

/* libfyodor_hip's resident decoder steps (include/fyodor_hip.h). Optional:
 * without them the provider still multiplies matrices and declines plans. */
typedef struct nya_resident_ops {
    int (*step)(uintptr_t, unsigned, size_t, uintptr_t);
    int (*embed)(uintptr_t, unsigned, size_t, size_t, uintptr_t, size_t, uintptr_t, float, uintptr_t);
    int (*rms_norm)(uintptr_t, uintptr_t, uintptr_t, uintptr_t, size_t, size_t, float, uintptr_t);
    int (*rope_qkv)(uintptr_t, size_t, uintptr_t, size_t, uintptr_t, size_t, size_t, size_t, size_t, size_t,
        uintptr_t, uintptr_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    int (*attention)(uintptr_t, size_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t, size_t, size_t, size_t,
        size_t, size_t, size_t, float, uintptr_t);
    int (*silu_mul)(uintptr_t, size_t, uintptr_t, size_t, uintptr_t, size_t, size_t, uintptr_t);
    int (*greedy)(uintptr_t, size_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    /* Optional within the set: NULL leaves the gated SiLU a step of its own. */
    int (*matvec_gated)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t);
    /* Optional: NULL leaves the attention norm a step of its own. */
    int (*matvec_normed)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, uintptr_t, float, uintptr_t,
        uintptr_t, uintptr_t);
    /* Optional: NULL leaves the rotary step a launch of its own. */
    int (*matvec_normed_rope)(uintptr_t, unsigned, size_t, size_t, size_t, uintptr_t, uintptr_t, uintptr_t, float,
        uintptr_t, uintptr_t, uintptr_t, uintptr_t, size_t, size_t, size_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    /* Optional as a pair: NULL keeps gate and up in two blocks of rows. */
    int (*matvec_swiglu)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    int (*silu_pairs)(uintptr_t, uintptr_t, size_t, size_t, uintptr_t);
    /* Optional as a pair (with matvec_swiglu): NULL leaves the feed-forward
     * norm a step of its own. */
    int (*matvec_residual)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t,
        uintptr_t, uintptr_t);
    int (*matvec_swiglu_scaled)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, float, uintptr_t,
        uintptr_t);
    /* Optional (with matvec_residual and matvec_normed_rope): NULL keeps the
     * attention norm inside every q|k|v workgroup. */
    int (*matvec_scaled_rope)(uintptr_t, unsigned, size_t, size_t, size_t, uintptr_t, uintptr_t, float, uintptr_t,
        uintptr_t, uintptr_t, size_t, size_t, size_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    /* Optional (with matvec_normed_rope): NULL runs q|k|v stored in two
     * types as one rotary launch per part. */
    int (*matvec_rope_pair)(uintptr_t, unsigned, size_t, uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t,
        uintptr_t, uintptr_t, uintptr_t, float, uintptr_t, uintptr_t, uintptr_t, size_t, size_t, size_t, size_t,
        uintptr_t, uintptr_t, uintptr_t);
    /* Optional: NULL keeps attention one workgroup per query head at every
     * length. */
    int (*attention_split)(uintptr_t, size_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t, size_t, size_t,
        size_t, size_t, size_t, size_t, size_t, float, uintptr_t);
    /* Optional as a set: the Gemma steps (per-block post norms and output
     * scale, per-head q/k/v norms with the half-split rotation, the GELU
     * gate, the logit soft cap); NULL declines Gemma models. */
    int (*post_norm)(uintptr_t, uintptr_t, uintptr_t, float, uintptr_t, uintptr_t, size_t, size_t, float, uintptr_t);
    int (*head_norm_rope)(uintptr_t, size_t, uintptr_t, size_t, uintptr_t, size_t, size_t, size_t, size_t, size_t,
        uintptr_t, uintptr_t, float, uintptr_t, uintptr_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    int (*gelu_mul)(uintptr_t, size_t, uintptr_t, size_t, uintptr_t, size_t, size_t, uintptr_t);
    int (*softcap)(uintptr_t, size_t, float, uintptr_t);
    /* Optional as a pair (with the Gemma set): NULL keeps Gemma's gate and
     * up in two blocks of rows and its GELU gate a step of its own. */
    int (*matvec_geglu)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, uintptr_t);
    int (*gelu_pairs)(uintptr_t, uintptr_t, size_t, size_t, uintptr_t);
    /* Optional (with host_device_pointer): the logits written into the
     * mapped pinned staging by the plan's last launch, no copy call. */
    int (*copy)(uintptr_t, uintptr_t, size_t, uintptr_t);
} nya_resident_ops;

#define NYA_KERNEL_ABI 2U
#endif
