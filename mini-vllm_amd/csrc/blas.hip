// The projections of a prefill chunk through hipBLASLt, with the per-shape set-up kept.
//
// The reference runs every projection through torch (mini_vllm/basics.py:18 linear:
// x @ w.T), which on this part reaches hipBLASLt and, on every call, creates the matmul
// and matrix-layout descriptors and asks the library's heuristic for an algorithm.
// Measured on the MI355X through torch: ~18.5 us of host time per call when the shape was
// seen before and ~72 us when it is new (the heuristic's own lookup), against ~19 us of
// GPU time for a 1460 x 1024 x 4096 bf16 product - an engine iteration that issues 112 of
// them (28 layers x q/k/v, o, gate/up, down) is bound by that host time, not by the GPU.
//
// Here the descriptors are made once per (device, dtype, m, n, k) and kept, and the
// heuristic's first algorithm once per (device, dtype, n, k, 128-row bucket of m): the
// rows of a prefill chunk change from one engine iteration to the next, and a heuristic
// query for each new m costs more host time than the product takes on the GPU. The
// bucket's algorithm is the heuristic's choice for the bucket's largest m, an odd number
// (128 j + 127), so that it assumes nothing of m's alignment; should hipBLASLt refuse
// it for an m of the bucket, that shape asks the heuristic for its own and keeps it.
// An m that is a multiple of 128 (a full 2048-token budget is one) takes its own
// algorithm from the start: the heuristic has aligned kernels for it that the bucket's
// odd m rules out (measured at m = 2048: 6.7 ms per engine iteration with the bucket's
// against 6.2 with the exact shape's).
// A call looks its shape up and issues hipblasLtMatmul. The workspace
// (kBlasWorkspaceBytes, the most any kept algorithm may ask for) is one allocation per
// (device, stream), made on that pair's first call, so concurrent streams never share
// one. The product itself is hipBLASLt's (fp32 accumulation, alpha 1, beta 0).
//
// Row-major y [m, n] = x [m, k] w [n, k]^T is, in hipBLASLt's column-major terms,
// Y (n x m, ld n) = op_T(W: k x n, ld k) * X (k x m, ld k).

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <unordered_map>
#include <utility>

#include "blas.hpp"
#include "common.hpp"

namespace mvllm {

namespace {

constexpr int kBlasDevices = 64;
constexpr int64_t kBucketRows = 128;

struct PlanKey {
  int dev;
  int dtype;
  int64_t m, n, k;
  bool operator==(const PlanKey& o) const {
    return dev == o.dev && dtype == o.dtype && m == o.m && n == o.n && k == o.k;
  }
};

struct PlanKeyHash {
  size_t operator()(const PlanKey& key) const {
    uint64_t h = static_cast<uint64_t>(key.dev) * 0x9E3779B97F4A7C15ull ^ static_cast<uint64_t>(key.dtype);
    for (int64_t v : {key.m, key.n, key.k}) h = (h ^ static_cast<uint64_t>(v)) * 0x100000001B3ull;
    return static_cast<size_t>(h);
  }
};

struct Algo {
  hipblasLtMatmulAlgo_t algo;
  size_t workspace = 0;
};

struct BlasPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  Algo algo;
  bool own_algo = false;  // the bucket's algorithm was refused: this shape's own
};

std::mutex g_blas_mutex;
hipblasLtHandle_t g_handles[kBlasDevices] = {};
std::unordered_map<PlanKey, BlasPlan, PlanKeyHash> g_plans;
// Keyed by (device, dtype, bucket, n, k) in PlanKey's fields (m = the bucket index).
std::unordered_map<PlanKey, Algo, PlanKeyHash> g_algos;
std::map<std::pair<int, hipStream_t>, void*> g_blas_workspaces;

void destroy(BlasPlan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = BlasPlan{};
}

BlasStatus lt_error(hipblasStatus_t s, const char* what) {
  return BlasStatus{2, static_cast<int>(s), what};
}

hipDataType data_type(int dtype) { return dtype == kBF16 ? HIP_R_16BF : HIP_R_16F; }

// The layouts of W (k x n, ld k), X (k x m, ld k) and Y (n x m, ld n).
hipblasStatus_t make_layouts(int dtype, int64_t m, int64_t n, int64_t k, hipblasLtMatrixLayout_t& a,
                             hipblasLtMatrixLayout_t& b, hipblasLtMatrixLayout_t& c) {
  const hipDataType type = data_type(dtype);
  hipblasStatus_t s = hipblasLtMatrixLayoutCreate(&a, type, k, n, k);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&b, type, k, m, k);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&c, type, n, m, n);
  return s;
}

// The heuristic's first algorithm for `desc` at m rows (caller holds the mutex).
BlasStatus heuristic(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t desc, int dtype, int64_t m,
                     int64_t n, int64_t k, Algo& out) {
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasStatus_t s = make_layouts(dtype, m, n, k, a, b, c);
  hipblasLtMatmulPreference_t pref = nullptr;
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatmulPreferenceCreate(&pref);
  const uint64_t max_ws = kBlasWorkspaceBytes;
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                              &max_ws, sizeof(max_ws));
  }
  hipblasLtMatmulHeuristicResult_t result;
  int found = 0;
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulAlgoGetHeuristic(handle, desc, a, b, c, c, pref, 1, &result, &found);
  }
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (a) hipblasLtMatrixLayoutDestroy(a);
  if (b) hipblasLtMatrixLayoutDestroy(b);
  if (c) hipblasLtMatrixLayoutDestroy(c);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "heuristic");
  if (found < 1 || result.state != HIPBLAS_STATUS_SUCCESS || result.workspaceSize > max_ws) {
    return BlasStatus{3, 0, "heuristic found no algorithm"};
  }
  out.algo = result.algo;
  out.workspace = result.workspaceSize;
  return BlasStatus{0, 0, nullptr};
}

// Descriptors for one shape and its bucket's algorithm (caller holds the mutex).
BlasStatus make_plan(hipblasLtHandle_t handle, const PlanKey& key, BlasPlan& plan) {
  hipblasStatus_t s = hipblasLtMatmulDescCreate(&plan.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "matmul descriptor");
  const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  s = hipblasLtMatmulDescSetAttribute(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t));
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulDescSetAttribute(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n));
  }
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "transpose attributes");
  s = make_layouts(key.dtype, key.m, key.n, key.k, plan.a, plan.b, plan.c);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "matrix layouts");
  if (key.m % kBucketRows == 0) {
    // A whole number of buckets (a full token budget: the same m every iteration) has
    // aligned algorithms the bucket's odd m cannot use: the exact shape's own.
    plan.own_algo = true;
    return heuristic(handle, plan.desc, key.dtype, key.m, key.n, key.k, plan.algo);
  }
  const int64_t bucket = key.m / kBucketRows;
  const PlanKey akey{key.dev, key.dtype, bucket, key.n, key.k};
  auto it = g_algos.find(akey);
  if (it == g_algos.end()) {
    Algo algo;
    const BlasStatus st = heuristic(handle, plan.desc, key.dtype, bucket * kBucketRows + kBucketRows - 1,
                                    key.n, key.k, algo);
    if (st.kind != 0) return st;
    it = g_algos.emplace(akey, algo).first;
  }
  plan.algo = it->second;
  return BlasStatus{0, 0, nullptr};
}

}  // namespace

BlasStatus blas_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                       int dtype, hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return BlasStatus{1, static_cast<int>(e), "hipGetDevice"};
  if (dev < 0 || dev >= kBlasDevices) return BlasStatus{1, static_cast<int>(hipErrorInvalidDevice), "device index"};
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  if (g_handles[dev] == nullptr) {
    const hipblasStatus_t s = hipblasLtCreate(&g_handles[dev]);
    if (s != HIPBLAS_STATUS_SUCCESS) {
      g_handles[dev] = nullptr;
      return lt_error(s, "handle");
    }
  }
  const PlanKey key{dev, dtype, m, n, k};
  auto it = g_plans.find(key);
  if (it == g_plans.end()) {
    if (static_cast<int>(g_plans.size()) >= kBlasMaxPlans) {
      for (auto& kv : g_plans) destroy(kv.second);
      g_plans.clear();
      g_algos.clear();
    }
    BlasPlan plan;
    const BlasStatus st = make_plan(g_handles[dev], key, plan);
    if (st.kind != 0) {
      destroy(plan);
      return st;
    }
    it = g_plans.emplace(key, plan).first;
  }
  BlasPlan& plan = it->second;
  void*& slot = g_blas_workspaces[std::make_pair(dev, stream)];
  if (slot == nullptr) {
    e = hipMalloc(&slot, kBlasWorkspaceBytes);
    if (e != hipSuccess) {
      slot = nullptr;
      return BlasStatus{1, static_cast<int>(e), "workspace allocation"};
    }
  }
  const float alpha = 1.0f, beta = 0.0f;
  hipblasStatus_t s = hipblasLtMatmul(g_handles[dev], plan.desc, &alpha, w, plan.a, x, plan.b, &beta,
                                      y, plan.c, y, plan.c, &plan.algo.algo, slot,
                                      kBlasWorkspaceBytes, stream);
  if (s != HIPBLAS_STATUS_SUCCESS && !plan.own_algo) {
    // The bucket's algorithm does not serve this m: the shape's own, kept from now on.
    const BlasStatus st = heuristic(g_handles[dev], plan.desc, dtype, m, n, k, plan.algo);
    if (st.kind != 0) return st;
    plan.own_algo = true;
    s = hipblasLtMatmul(g_handles[dev], plan.desc, &alpha, w, plan.a, x, plan.b, &beta, y, plan.c,
                        y, plan.c, &plan.algo.algo, slot, kBlasWorkspaceBytes, stream);
  }
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "matmul");
  return BlasStatus{0, 0, nullptr};
}

int blas_plans_cached() {
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  return static_cast<int>(g_plans.size());
}

}  // namespace mvllm
