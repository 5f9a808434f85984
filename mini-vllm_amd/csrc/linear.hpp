// Internal launch interface of the skinny projection kernel (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Most rows (x rows, i.e. tokens) one skinny projection serves.
constexpr int64_t kSkinnyMaxRows = 64;
// Longest reduction (x columns) it serves.
constexpr int64_t kSkinnyMaxK = 65536;

// Whether launch_skinny_linear (over packed W) serves y[m, n] = x[m, k] w[n, k]^T in this dtype.
bool skinny_linear_supported(int dtype, int64_t m, int64_t n, int64_t k);

// Whether launch_skinny_linear_residual_rmsnorm serves this shape: K > 1024 (the split
// path) and n a multiple of 512 up to 4096 (whole 8-element chunks on a 64-lane row).
bool skinny_residual_rmsnorm_supported(int dtype, int64_t m, int64_t n, int64_t k);

// Device bytes of fp32 partial sums the projection of a [m, k] x [n, k]^T needs (K >
// 1024; 0 otherwise): caller-owned, contents need not be initialised.
uint64_t skinny_linear_workspace_bytes(int64_t m, int64_t n, int64_t k);

// Elements of W [n, k] packed into the kernel's fragment order (n rounded up to 32).
int64_t skinny_linear_packed_elements(int64_t n, int64_t k);
// Packs row-major W [n, k] (16-bit elements) into that order (rows past n zero).
hipError_t launch_skinny_linear_pack(void* w_packed, const void* w, int64_t n, int64_t k,
                                     hipStream_t stream);

// Epilogues of the skinny projection kernel.
enum LinearEpilogue : int { kLinearPlain = 0, kLinearSplit = 1, kLinearResidual = 2, kLinearSwiglu = 3 };

hipError_t launch_skinny_linear(void* y, const void* x, const void* w, int64_t m, int64_t n,
                                int64_t k, int dtype, void* workspace, hipStream_t stream);
// Columns [0, n0) -> y0 [m, n0], [n0, n0 + n1) -> y1 [m, n1], the last n2 -> y2 [m, n2];
// n0 and n1 multiples of 32.
hipError_t launch_skinny_linear_split(void* y0, void* y1, void* y2, const void* x, const void* w,
                                      int64_t m, int64_t n0, int64_t n1, int64_t n2, int64_t k,
                                      int dtype, void* workspace, hipStream_t stream);
// y = residual + x w^T, each of the two steps rounded to the dtype (residual [m, n]).
hipError_t launch_skinny_linear_residual(void* y, const void* x, const void* w, const void* residual,
                                         int64_t m, int64_t n, int64_t k, int dtype,
                                         void* workspace, hipStream_t stream);
// y [m, n_out] = swiglu(x gate^T, x up^T) with w_gate_up [2 n_out, k] holding gate and up
// rows interleaved in groups of 16; n_out a multiple of 16.
hipError_t launch_skinny_linear_swiglu(void* y, const void* x, const void* w_gate_up, int64_t m,
                                       int64_t n_out, int64_t k, int dtype, void* workspace,
                                       hipStream_t stream);
// h = T(residual + T(x w^T)) and normed = RMSNorm(h) * norm_weight (rounded as the
// RMSNorm kernel rounds), h and normed [m, n].
hipError_t launch_skinny_linear_residual_rmsnorm(void* h_out, void* normed, const void* x,
                                                 const void* w, const void* residual,
                                                 const void* norm_weight, int64_t m, int64_t n,
                                                 int64_t k, float eps, int dtype, void* workspace,
                                                 hipStream_t stream);

}  // namespace mvllm
