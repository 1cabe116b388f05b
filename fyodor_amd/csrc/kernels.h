// Host-side launchers of the gfx950 kernels (called by abi.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fy {

// Y[n][rows] = sum_k W[row][k] * X[n][k] for n < batch, batch 1..8, W in the
// device layout. Reads every weight byte once per call.
hipError_t launch_skinny(unsigned type, const uint8_t *w, const float *x, float *y,
    int rows, int cols, int batch, hipStream_t stream);
const char *skinny_name(unsigned type, int batch);

}  // namespace fy
