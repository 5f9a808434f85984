// Internal launch interface of the elementwise kernels (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

hipError_t launch_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int dim,
                          float eps, int dtype, hipStream_t stream);
hipError_t launch_rope(const void* x, const void* positions, int pos_bytes, const float* cos_t,
                       const float* sin_t, void* out, int64_t rows, int64_t heads, int dim,
                       int64_t num_positions, int64_t max_positions, int dtype,
                       hipStream_t stream);
hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
                         hipStream_t stream);
hipError_t launch_axpby(const float* x, float* y, float a, float b, int64_t n,
                        hipStream_t stream);

}  // namespace mvllm
