// Internal interface of the cached hipBLASLt product (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Outcome of blas_linear: kind 0 ok; 1 a HIP runtime error (code = hipError_t); 2 a
// hipBLASLt error (code = hipblasStatus_t); 3 no algorithm for this shape. `what` names
// the failing step.
struct BlasStatus {
  int kind;
  int code;
  const char* what;
};

// Workspace bytes the product may use, held per (device, stream) by the library.
constexpr uint64_t kBlasWorkspaceBytes = 32ull << 20;
// Shapes whose descriptors and algorithm the library keeps; the next new shape past
// this drops them all (each is made again on its next call).
constexpr int kBlasMaxPlans = 4096;

// y [m, n] = x [m, k] w [n, k]^T, row-major, fp16 or bf16 (dtype code), fp32 accumulation,
// on `stream` of the current device.
BlasStatus blas_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                       int dtype, hipStream_t stream);

// Shapes currently kept (for tests).
int blas_plans_cached();

}  // namespace mvllm
