// Dense-cache attention (B x H x L x D tensors) on the paged kernels.
//
// The reference serves its dense-cache model (mini_vllm/model/qwen3_cached.py) with two
// more kernels, csrc/decode_attention.cu (one query token against the whole cache) and
// csrc/flash_prefill.cu (L queries, causal with offset S - L), both reading K/V through
// (batch, head, position) strides so a cache narrowed out of a larger buffer is read in
// place. Their math is the paged kernels' math over a different address map, so this
// library does not keep a second pair of kernels: the paged decode and prefill kernels
// take the pool's slot and head strides as parameters, and a dense cache is presented
// to them as a pool of virtual 16-position pages - sequence b's page i is the 16
// positions from 16 i on, its table entry the slot id of its first position,
// b * (batch stride / position stride) + 16 i, read with a table shift of 0 - with
// every sequence's context the full S and its query length L. This file writes
// that metadata (block tables, cu_seqlens, context and query lengths) into the
// caller's workspace; the host entry then plans and launches as for a paged batch.

#include <algorithm>

#include "common.hpp"
#include "dense.hpp"

namespace mvllm {

namespace {

__global__ void dense_meta_kernel(DenseMeta meta) {
  const int64_t table = static_cast<int64_t>(meta.batch) * meta.max_blocks;
  const int64_t total = table + 3 * static_cast<int64_t>(meta.batch) + 1;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (i < table) {
      const int64_t b = i / meta.max_blocks, page = i % meta.max_blocks;
      meta.block_tables[i] = static_cast<int32_t>(b * meta.slots_per_batch + 16 * page);
    } else {
      const int64_t j = i - table;
      if (j <= meta.batch) {
        meta.cu_seqlens_q[j] = static_cast<int32_t>(j * meta.query_len);
      } else if (j <= 2 * static_cast<int64_t>(meta.batch)) {
        meta.context_lens[j - meta.batch - 1] = meta.kv_len;
      } else {
        meta.seq_lens[j - 2 * meta.batch - 1] = meta.query_len;
      }
    }
  }
}

}  // namespace

hipError_t launch_dense_meta(const DenseMeta& meta, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(meta.batch) * meta.max_blocks + 3 * meta.batch + 1;
  const int blocks = static_cast<int>(std::min<int64_t>((total + 255) / 256, 1024));
  dense_meta_kernel<<<blocks, 256, 0, stream>>>(meta);
  return hipGetLastError();
}

}  // namespace mvllm
