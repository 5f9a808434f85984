// Internal interface of the dense-cache metadata kernel (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// The paged-batch metadata that presents a dense cache to the paged kernels.
struct DenseMeta {
  int32_t* block_tables;  // [batch][max_blocks]: slot id b * slots_per_batch + 16 page
  int32_t* cu_seqlens_q;  // [batch + 1]: b * query_len
  int32_t* context_lens;  // [batch]: kv_len
  int32_t* seq_lens;      // [batch]: query_len
  int batch;
  int max_blocks;         // ceil(kv_len / 16)
  int64_t slots_per_batch;  // batch stride / position stride
  int query_len;
  int kv_len;
};

hipError_t launch_dense_meta(const DenseMeta& meta, hipStream_t stream);

}  // namespace mvllm
