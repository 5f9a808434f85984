// Internal launch interface of the elementwise kernels (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

hipError_t launch_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int dim,
                          float eps, int dtype, hipStream_t stream);
// h_out = T(x + residual) and out = RMSNorm(h_out) in one pass (rows of dim elements,
// every pointer 16-byte aligned); add_rmsnorm_supported says which dims it takes.
bool add_rmsnorm_supported(int dtype, int dim);
hipError_t launch_add_rmsnorm(const void* x, const void* residual, const void* w, void* h_out,
                              void* out, int64_t rows, int dim, float eps, int dtype,
                              hipStream_t stream);
// h_out[i] = the table row of token (index && index[i] >= 0 ? prev[index[i]] : ids[i])
// and out = RMSNorm(h_out) in one pass (the token embedding and the first block's input
// norm; same dims and alignment as the add; a token id outside [0, vocab) gives NaN
// rows).
hipError_t launch_embed_rmsnorm(const void* table, int64_t vocab, const int64_t* ids,
                                const int64_t* index, const int64_t* prev, const void* w,
                                void* h_out, void* out, int64_t rows, int dim, float eps,
                                int dtype, hipStream_t stream);
hipError_t launch_rope(const void* x, const void* positions, int pos_bytes, const float* cos_t,
                       const float* sin_t, void* out, int64_t rows, int64_t heads, int dim,
                       int64_t num_positions, int64_t max_positions, int dtype,
                       hipStream_t stream);
// Whether launch_qk_norm_rope serves this dtype and head dim (D / (16 / elt) lanes
// per head a power of two from 2 to 64).
bool qk_norm_rope_supported(int dtype, int head_dim);
// With k_pool non-null the launch also writes k (as rotated) and v to the paged pools
// [num_slots, hk, dim] of the same dtype at slots[token] (outside [0, num_slots):
// skipped); k_out may then be null.
hipError_t launch_qk_norm_rope(const void* q, const void* k, const void* wq, const void* wk,
                               const void* positions, int pos_bytes, const float* cos_t,
                               const float* sin_t, void* q_out, void* k_out, int64_t tokens,
                               int hq, int hk, int dim, int64_t num_positions,
                               int64_t max_positions, float eps, int dtype, hipStream_t stream,
                               const void* v = nullptr, void* k_pool = nullptr,
                               void* v_pool = nullptr, const int32_t* slots = nullptr,
                               int64_t num_slots = 0, int64_t q_token_stride = 0,
                               int64_t kv_token_stride = 0);
// (Token strides in elements between consecutive tokens of q and of k and v; 0 means
// contiguous, hq * dim and hk * dim.)
// out [rows][cols] = swiglu of the 16-column gate/up interleave [rows][2 cols]; cols a
// multiple of 16, every pointer 16-byte aligned.
hipError_t launch_swiglu_interleaved(const void* gate_up, void* out, int64_t rows, int64_t cols,
                                     int dtype, hipStream_t stream);
hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
                         hipStream_t stream);
hipError_t launch_axpby(const float* x, float* y, float a, float b, int64_t n,
                        hipStream_t stream);

}  // namespace mvllm
