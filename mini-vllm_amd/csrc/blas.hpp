// Internal interface of the cached hipBLASLt product (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Outcome of blas_linear / blas_tune: kind 0 ok; 1 a HIP runtime error (code =
// hipError_t); 2 a hipBLASLt error (code = hipblasStatus_t); 3 no algorithm for this
// shape; 4 the stream is being captured (blas_tune only). `what` names the failing step.
struct BlasStatus {
  int kind;
  int code;
  const char* what;
};

// Workspace bytes the product may use: the caller's buffer must hold this many.
constexpr uint64_t kBlasWorkspaceBytes = 32ull << 20;
// Heuristic candidates timed on the first call of a bucket (or exact shape), and the
// timed runs of each.
constexpr int kBlasCandidates = 16;
constexpr int kBlasTimedRuns = 5;
// blas_tune: timed runs of each algorithm in its sweep, and how many of the fastest it
// keeps as extra candidates.
constexpr int kBlasSweepRuns = 3;
constexpr int kBlasPreferred = 12;

// How a kept algorithm was chosen: the heuristic's candidates, how many were timed
// (0: the first was taken untimed, e.g. under graph capture), the kept one's index in
// the heuristic's order, and the first's and the kept one's time per product (us, -1
// when untimed).
struct BlasTuning {
  int candidates = 0;
  int timed = 0;
  int chosen = 0;
  float first_us = -1.0f;
  float chosen_us = -1.0f;
};
// Shapes whose descriptors and algorithm the library keeps; the next new shape past
// this drops them all (each is made again on its next call).
constexpr int kBlasMaxPlans = 4096;

// y [m, n] = x [m, k] w [n, k]^T, row-major, fp16 or bf16 (dtype code), fp32 accumulation,
// on `stream` of the current device, with `workspace` (kBlasWorkspaceBytes) the caller's.
BlasStatus blas_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                       int dtype, void* workspace, hipStream_t stream);

// Times every algorithm hipBLASLt holds that serves y = x w^T at (m, n, k) (one warm-up
// and kBlasSweepRuns runs each, the least of the runs' own times, on the caller's
// operands and stream, one host wait per algorithm) and keeps the kBlasPreferred fastest as extra candidates for every later
// choice of (n, k); choices already made for (n, k) are dropped and made again. Leaves y
// = x w^T. Refused while `stream` is capturing. `timed` = the algorithms timed.
BlasStatus blas_tune(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                     int dtype, void* workspace, hipStream_t stream, int& timed);

// The choice record of the algorithm kept for (current device, dtype, m, n, k); false if
// that shape has not been called.
bool blas_tuning(int64_t m, int64_t n, int64_t k, int dtype, BlasTuning& out);

// Shapes currently kept (for tests).
int blas_plans_cached();

}  // namespace mvllm
