// Launchers for the activation quantisers (quant.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ovh {

// tiled: codes tile-major (act_index), rows of the last 32-row band past M
// written as zero codes (the buffer holds whole 32-row bands)
hipError_t launch_quantize(int64_t M, int64_t K, const float* A, int8_t* aq, float* asc,
                           hipStream_t st, bool tiled = false);
// tiled: codes tile-major (act_index); needs cols % 256 == 0, cols <= 1024 and
// 16-byte aligned x and w (hipErrorInvalidValue otherwise).
hipError_t launch_rmsnorm_quantize(int64_t rows, int64_t cols, const float* x, const float* w,
                                   float eps, int8_t* aq, float* asc, hipStream_t st,
                                   bool tiled = false);
size_t rmsnorm_quantize_smem(int64_t cols);
hipError_t launch_silu_mul_quantize(int64_t M, int64_t K, const float* g, const float* u,
                                    int8_t* aq, float* asc, hipStream_t st);

}  // namespace ovh
