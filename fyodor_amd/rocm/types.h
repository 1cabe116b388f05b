/* The few HIP runtime C types the provider passes through dlsym'ed function
 * pointers. Tags and enumerator values are HIP's own (hip/hip_runtime_api.h,
 * hip/driver_types.h in ROCm 7.2), as in the reference's private copy
 * (rocm/types.h:1-132): matching tags keep the function pointer types
 * compatible with the runtime's, which UBSan's indirect-call check compares.
 * Only the enumerators this provider uses are listed. */
#ifndef NYA_ROCM_TYPES_H
#define NYA_ROCM_TYPES_H

typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorNotInitialized = 3,
    hipErrorNoDevice = 100,
    hipErrorInvalidDevice = 101,
    hipErrorUnknown = 999
} hipError_t;

typedef enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4
} hipMemcpyKind;

typedef struct ihipStream_t *hipStream_t;
typedef struct ihipGraph *hipGraph_t;
typedef struct hipGraphExec *hipGraphExec_t;

typedef enum hipStreamCaptureMode {
    hipStreamCaptureModeGlobal = 0,
    hipStreamCaptureModeThreadLocal = 1,
    hipStreamCaptureModeRelaxed = 2
} hipStreamCaptureMode;

/* hipStreamNonBlocking: the stream does not synchronize with the null
 * stream (rocm/rocm.c:179 passes 1). */
#define NYA_HIP_STREAM_NON_BLOCKING 1U

#endif
