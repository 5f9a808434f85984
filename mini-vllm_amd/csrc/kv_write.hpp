// Internal launch interface of the paged KV write (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Whether launch_kv_write serves this (source, pool) storage pair and head dim.
bool kv_write_supported(int src_dtype, int pool_dtype, int head_dim);

hipError_t launch_kv_write(void* k_pool, void* v_pool, float* k_scales, float* v_scales,
                           const void* key, const void* value, const int32_t* slots,
                           int num_tokens, int hk, int head_dim, int block_shift,
                           int64_t num_blocks, int src_dtype, int pool_dtype, hipStream_t stream);

}  // namespace mvllm
