// Internal launch interface of the greedy-sampling kernel (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// out[r] = index of the maximum of logits row r (rows x v, rows row_stride elements
// apart), torch.argmax order: NaN above numbers, -0 == +0, first index among equals.
// `workspace`: argmax_workspace_bytes(rows, v) bytes (the segments' best keys).
hipError_t launch_argmax(int64_t* out, const void* logits, int64_t rows, int64_t v,
                         int64_t row_stride, int dtype, void* workspace, hipStream_t stream);
uint64_t argmax_workspace_bytes(int64_t rows, int64_t v);
// Longest row served (64 segments).
int64_t argmax_max_vocab();

}  // namespace mvllm
