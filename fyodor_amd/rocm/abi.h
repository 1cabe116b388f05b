/* Function table the C provider resolves at run time: the HIP runtime
 * members keep the names and C types of the reference table
 * (rocm/abi.h:8-19); the rocBLAS members (rocm/abi.h:20-25) are replaced by
 * the gfx950 kernel library declared in include/fyodor_hip.h. Neither a HIP
 * compiler nor HIP headers are needed to build the provider. */
#ifndef NYA_ROCM_ABI_H
#define NYA_ROCM_ABI_H
#include <stddef.h>
#include <stdint.h>
#include "types.h"

typedef struct nya_rocm_api {
    /* libamdhip64 */
    hipError_t (*init)(unsigned);
    hipError_t (*device_count)(int *);
    hipError_t (*get_device)(int *);
    hipError_t (*set_device)(int);
    hipError_t (*memory_info)(size_t *, size_t *);
    hipError_t (*allocate)(void **, size_t);
    hipError_t (*deallocate)(void *);
    hipError_t (*copy_async)(void *, const void *, size_t, hipMemcpyKind, hipStream_t);
    hipError_t (*stream_create)(hipStream_t *, unsigned);
    hipError_t (*stream_destroy)(hipStream_t);
    hipError_t (*synchronize)(hipStream_t);
    /* libfyodor_hip (include/fyodor_hip.h) */
    unsigned (*kernel_version)(void);
    int (*weight_bytes)(unsigned, size_t, size_t, size_t *);
    int (*weight_layout)(unsigned);
    int (*weight_pack)(void *, const void *, unsigned, size_t, size_t);
    int (*workspace_bytes)(unsigned, size_t, size_t, size_t, size_t *);
    int (*matmul)(uintptr_t, unsigned, size_t, size_t, uintptr_t, uintptr_t, size_t, uintptr_t, size_t, uintptr_t);
} nya_rocm_api;

#define NYA_HIP_H2D hipMemcpyHostToDevice
#define NYA_HIP_D2H hipMemcpyDeviceToHost
#define NYA_HIP_KERNEL_ABI 1U
#endif
