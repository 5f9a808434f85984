// Internal launch interface of the greedy-sampling kernel (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// out[r] = index of the maximum of logits row r (rows x v, rows row_stride elements
// apart), torch.argmax order: NaN above numbers, -0 == +0, first index among equals.
hipError_t launch_argmax(int64_t* out, const void* logits, int64_t rows, int64_t v,
                         int64_t row_stride, int dtype, hipStream_t stream);

}  // namespace mvllm
