// Internal launch interface of the prefill projection GEMM (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Whether launch_gemm serves y[m, n] = x[m, k] w[n, k]^T (row-major, 16-byte aligned
// rows) in this dtype: bf16 / fp16, n a multiple of 64, k of 64.
bool gemm_supported(int dtype, int64_t m, int64_t n, int64_t k);

// `cus`: the device's compute units (the tile is chosen to fill them); `config` < 0
// picks the tile by size, 0..2 forces one (256 x 128, 128 x 128, 128 x 64: 128-wide
// tiles need n a multiple of 128).
hipError_t launch_gemm(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                       int dtype, int cus, int config, hipStream_t stream);

}  // namespace mvllm
