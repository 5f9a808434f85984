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
// algorithm once per (device, dtype, n, k, 128-row bucket of m): the rows of a prefill
// chunk change from one engine iteration to the next, and a heuristic query for each new
// m costs more host time than the product takes on the GPU. The bucket's candidates are
// the heuristic's first kBlasCandidates for the bucket's largest m, an odd number
// (128 j + 127), so that they assume nothing of m's alignment; should hipBLASLt refuse
// the kept one for an m of the bucket, that shape takes the heuristic's first for its
// own m and keeps it. An m that is a multiple of 128 (a full 2048-token budget is one)
// takes candidates for its exact shape: the heuristic has aligned kernels for it that
// the bucket's odd m rules out (measured at m = 2048: 6.7 ms per engine iteration with
// the bucket's against 6.2 with the exact shape's).
// Choosing among the candidates: the heuristic's first is not always the fastest on
// this part, so the first call of a bucket (or exact shape) times every candidate on
// the call's own operands (one warm-up and kBlasTimedRuns runs each, every run between
// its own two HIP events on the caller's stream, the least kept, one host wait) and
// keeps the fastest; a call made while its stream
// is being captured into a graph cannot wait, so it keeps the heuristic's first
// without timing. The record of that choice (candidates, the first's and the kept
// one's time) is kept for reports.
// The heuristic's first 16 are not the library's best on this part either: timing every
// algorithm hipBLASLt holds for a shape (~230 of its ~20000 run at a Qwen3-0.6B
// projection shape) found faster ones. That sweep takes ~0.5 s per shape,
// too long for a first call, so it is an explicit step (blas_tune, at one row count per
// (n, k)): its fastest kBlasPreferred algorithms join the heuristic's candidates of every
// later bucket choice of that (n, k), each checked against the bucket's m first.
// A call looks its shape up and issues hipblasLtMatmul on the caller's workspace
// (kBlasWorkspaceBytes, the most any kept algorithm may ask for; calls on one stream
// may share it, being ordered): the library allocates no device memory. The product
// itself is hipBLASLt's (fp32 accumulation, alpha 1, beta 0).
//
// Row-major y [m, n] = x [m, k] w [n, k]^T is, in hipBLASLt's column-major terms,
// Y (n x m, ld n) = op_T(W: k x n, ld k) * X (k x m, ld k).

#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <mutex>
#include <algorithm>
#include <unordered_map>
#include <utility>
#include <vector>

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
  BlasTuning tuning;  // how it was chosen
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
// Keyed by (device, dtype, 0, n, k): blas_tune's fastest algorithms for that shape.
std::unordered_map<PlanKey, std::vector<Algo>, PlanKeyHash> g_preferred;

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

// The heuristic's first `want` algorithms for `desc` at m rows (caller holds the mutex).
BlasStatus heuristic(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t desc, int dtype, int64_t m,
                     int64_t n, int64_t k, int want, std::vector<Algo>& out) {
  out.clear();
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasStatus_t s = make_layouts(dtype, m, n, k, a, b, c);
  hipblasLtMatmulPreference_t pref = nullptr;
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatmulPreferenceCreate(&pref);
  const uint64_t max_ws = kBlasWorkspaceBytes;
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                              &max_ws, sizeof(max_ws));
  }
  std::vector<hipblasLtMatmulHeuristicResult_t> results(want);
  int found = 0;
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulAlgoGetHeuristic(handle, desc, a, b, c, c, pref, want, results.data(),
                                        &found);
  }
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (a) hipblasLtMatrixLayoutDestroy(a);
  if (b) hipblasLtMatrixLayoutDestroy(b);
  if (c) hipblasLtMatrixLayoutDestroy(c);
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "heuristic");
  for (int i = 0; i < found && i < want; ++i) {
    if (results[i].state != HIPBLAS_STATUS_SUCCESS || results[i].workspaceSize > max_ws) continue;
    Algo algo;
    algo.algo = results[i].algo;
    algo.workspace = results[i].workspaceSize;
    out.push_back(algo);
  }
  if (out.empty()) return BlasStatus{3, 0, "heuristic found no algorithm"};
  return BlasStatus{0, 0, nullptr};
}

struct Call {  // one product's operands
  void* y;
  const void* x;
  const void* w;
  void* workspace;
  hipStream_t stream;
};

hipblasStatus_t matmul(hipblasLtHandle_t handle, const BlasPlan& plan, const Algo& algo,
                       const Call& call) {
  const float alpha = 1.0f, beta = 0.0f;
  return hipblasLtMatmul(handle, plan.desc, &alpha, call.w, plan.a, call.x, plan.b, &beta, call.y,
                         plan.c, call.y, plan.c, &algo.algo, call.workspace, kBlasWorkspaceBytes,
                         call.stream);
}

// Events bracketing each timed run of a candidate.
struct RunEvents {
  hipEvent_t start[kBlasTimedRuns] = {};
  hipEvent_t stop[kBlasTimedRuns] = {};
  bool ok = true;
  RunEvents() {
    for (int r = 0; r < kBlasTimedRuns; ++r) {
      ok = ok && hipEventCreate(&start[r]) == hipSuccess && hipEventCreate(&stop[r]) == hipSuccess;
    }
  }
  ~RunEvents() {
    for (int r = 0; r < kBlasTimedRuns; ++r) {
      if (start[r]) (void)hipEventDestroy(start[r]);
      if (stop[r]) (void)hipEventDestroy(stop[r]);
    }
  }
};

// One warm-up and `runs` (<= kBlasTimedRuns) runs of `algo`, each bracketed by its own
// pair of events, one host wait: the least of the runs' GPU times in ms, or -1 if
// hipBLASLt refuses the algorithm for these operands. Timing each run on its own keeps
// the host out of the figure: back-to-back products of ~20 us are issued about as fast
// as they run, so a pair of events around several of them measures the issue rate, the
// same for every candidate.
float time_runs(hipblasLtHandle_t handle, const BlasPlan& plan, const Algo& algo,
                const Call& call, RunEvents& ev, int runs) {
  if (matmul(handle, plan, algo, call) != HIPBLAS_STATUS_SUCCESS) return -1.0f;
  for (int r = 0; r < runs; ++r) {
    if (hipEventRecord(ev.start[r], call.stream) != hipSuccess ||
        matmul(handle, plan, algo, call) != HIPBLAS_STATUS_SUCCESS ||
        hipEventRecord(ev.stop[r], call.stream) != hipSuccess) {
      return -1.0f;
    }
  }
  if (hipEventSynchronize(ev.stop[runs - 1]) != hipSuccess) return -1.0f;
  float least = -1.0f;
  for (int r = 0; r < runs; ++r) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ev.start[r], ev.stop[r]) != hipSuccess) return -1.0f;
    if (least < 0.0f || ms < least) least = ms;
  }
  return least;
}

// The fastest of `cands` on the call's own operands (time_runs, kBlasTimedRuns runs
// each). A candidate hipBLASLt refuses for this m is skipped. Leaves the kept
// algorithm's record in `best.tuning`. Caller holds the mutex; the stream is not
// capturing.
BlasStatus fastest(hipblasLtHandle_t handle, const BlasPlan& plan, std::vector<Algo>& cands,
                   const Call& call, Algo& best) {
  RunEvents ev;
  if (!ev.ok) return BlasStatus{1, static_cast<int>(hipErrorOutOfMemory), "tuning events"};
  float best_ms = -1.0f, first_ms = -1.0f;
  int best_i = -1, timed = 0;
  for (size_t i = 0; i < cands.size(); ++i) {
    const float ms = time_runs(handle, plan, cands[i], call, ev, kBlasTimedRuns);
    if (ms < 0.0f) continue;
    ++timed;
    if (i == 0) first_ms = ms;
    if (best_i < 0 || ms < best_ms) {
      best_ms = ms;
      best_i = static_cast<int>(i);
    }
  }
  if (best_i < 0) return BlasStatus{3, 0, "no candidate algorithm ran"};
  best = cands[best_i];
  best.tuning = BlasTuning{static_cast<int>(cands.size()), timed, best_i, first_ms * 1e3f,
                           best_ms * 1e3f};
  return BlasStatus{0, 0, nullptr};
}

// The kept algorithm from the heuristic's candidates at `m_heur` rows: timed on the
// call when the stream may wait, else the first.
BlasStatus choose(hipblasLtHandle_t handle, const BlasPlan& plan, int dtype, int64_t m_heur,
                  int64_t n, int64_t k, const Call& call, Algo& out) {
  std::vector<Algo> cands;
  const BlasStatus st = heuristic(handle, plan.desc, dtype, m_heur, n, k, kBlasCandidates, cands);
  if (st.kind != 0) return st;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    const auto pref = g_preferred.find(PlanKey{dev, dtype, 0, n, k});
    if (pref != g_preferred.end() && !pref->second.empty()) {
      // the tuned algorithms that serve the bucket's m join the candidates
      hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
      if (make_layouts(dtype, m_heur, n, k, a, b, c) == HIPBLAS_STATUS_SUCCESS) {
        const float alpha = 1.0f, beta = 0.0f;
        for (Algo cand : pref->second) {
          size_t need = 0;
          if (hipblaslt_ext::matmulIsAlgoSupported(handle, plan.desc, &alpha, a, b, &beta, c, c,
                                                   cand.algo, need) == HIPBLAS_STATUS_SUCCESS &&
              need <= kBlasWorkspaceBytes) {
            cand.workspace = need;
            cands.push_back(cand);
          }
        }
      }
      if (a) hipblasLtMatrixLayoutDestroy(a);
      if (b) hipblasLtMatrixLayoutDestroy(b);
      if (c) hipblasLtMatrixLayoutDestroy(c);
    }
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(call.stream, &capture) != hipSuccess) {
    capture = hipStreamCaptureStatusActive;  // unknown: do not wait
  }
  if (cands.size() > 1 && capture == hipStreamCaptureStatusNone) {
    return fastest(handle, plan, cands, call, out);
  }
  out = cands[0];
  out.tuning = BlasTuning{static_cast<int>(cands.size()), 0, 0, -1.0f, -1.0f};
  return BlasStatus{0, 0, nullptr};
}

// Descriptors for one shape and its kept algorithm (caller holds the mutex): the exact
// shape's for m a multiple of 128, else the bucket's (chosen on its first call).
BlasStatus make_plan(hipblasLtHandle_t handle, const PlanKey& key, const Call& call,
                     BlasPlan& plan) {
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
    return choose(handle, plan, key.dtype, key.m, key.n, key.k, call, plan.algo);
  }
  const int64_t bucket = key.m / kBucketRows;
  const PlanKey akey{key.dev, key.dtype, bucket, key.n, key.k};
  auto it = g_algos.find(akey);
  if (it == g_algos.end()) {
    Algo algo;
    const BlasStatus st = choose(handle, plan, key.dtype, bucket * kBucketRows + kBucketRows - 1,
                                 key.n, key.k, call, algo);
    if (st.kind != 0) return st;
    it = g_algos.emplace(akey, algo).first;
  }
  plan.algo = it->second;
  return BlasStatus{0, 0, nullptr};
}

}  // namespace

BlasStatus blas_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                       int dtype, void* workspace, hipStream_t stream) {
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
  const Call call{y, x, w, workspace, stream};
  const PlanKey key{dev, dtype, m, n, k};
  auto it = g_plans.find(key);
  if (it == g_plans.end()) {
    if (static_cast<int>(g_plans.size()) >= kBlasMaxPlans) {
      for (auto& kv : g_plans) destroy(kv.second);
      g_plans.clear();
      g_algos.clear();
    }
    BlasPlan plan;
    const BlasStatus st = make_plan(g_handles[dev], key, call, plan);
    if (st.kind != 0) {
      destroy(plan);
      return st;
    }
    it = g_plans.emplace(key, plan).first;
  }
  BlasPlan& plan = it->second;
  hipblasStatus_t s = matmul(g_handles[dev], plan, plan.algo, call);
  if (s != HIPBLAS_STATUS_SUCCESS && !plan.own_algo) {
    // The bucket's algorithm does not serve this m: the shape's own (the heuristic's
    // first), kept from now on.
    std::vector<Algo> cands;
    const BlasStatus st = heuristic(g_handles[dev], plan.desc, dtype, m, n, k, 1, cands);
    if (st.kind != 0) return st;
    plan.algo = cands[0];
    plan.algo.tuning = BlasTuning{1, 0, 0, -1.0f, -1.0f};
    plan.own_algo = true;
    s = matmul(g_handles[dev], plan, plan.algo, call);
  }
  if (s != HIPBLAS_STATUS_SUCCESS) return lt_error(s, "matmul");
  return BlasStatus{0, 0, nullptr};
}

bool blas_tuning(int64_t m, int64_t n, int64_t k, int dtype, BlasTuning& out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  const auto it = g_plans.find(PlanKey{dev, dtype, m, n, k});
  if (it == g_plans.end()) return false;
  out = it->second.algo.tuning;
  return true;
}

BlasStatus blas_tune(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                     int dtype, void* workspace, hipStream_t stream, int& timed_out) {
  timed_out = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return BlasStatus{1, static_cast<int>(e), "hipGetDevice"};
  if (dev < 0 || dev >= kBlasDevices) return BlasStatus{1, static_cast<int>(hipErrorInvalidDevice), "device index"};
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &capture);
  if (e != hipSuccess) return BlasStatus{1, static_cast<int>(e), "hipStreamIsCapturing"};
  if (capture != hipStreamCaptureStatusNone) return BlasStatus{4, 0, "the stream is capturing"};
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  if (g_handles[dev] == nullptr) {
    const hipblasStatus_t s = hipblasLtCreate(&g_handles[dev]);
    if (s != HIPBLAS_STATUS_SUCCESS) {
      g_handles[dev] = nullptr;
      return lt_error(s, "handle");
    }
  }
  hipblasLtHandle_t handle = g_handles[dev];
  BlasPlan plan;
  hipblasStatus_t s = hipblasLtMatmulDescCreate(&plan.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulDescSetAttribute(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t));
  }
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblasLtMatmulDescSetAttribute(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n));
  }
  if (s == HIPBLAS_STATUS_SUCCESS) s = make_layouts(dtype, m, n, k, plan.a, plan.b, plan.c);
  std::vector<hipblasLtMatmulHeuristicResult_t> all;
  const hipDataType type = data_type(dtype);
  if (s == HIPBLAS_STATUS_SUCCESS) {
    s = hipblaslt_ext::getAllAlgos(handle, hipblaslt_ext::GemmType::HIPBLASLT_GEMM, HIPBLAS_OP_T,
                                   HIPBLAS_OP_N, type, type, type, type, HIPBLAS_COMPUTE_32F, all);
  }
  if (s != HIPBLAS_STATUS_SUCCESS) {
    destroy(plan);
    return lt_error(s, "algorithm list");
  }
  RunEvents ev;
  if (!ev.ok) {
    destroy(plan);
    return BlasStatus{1, static_cast<int>(hipErrorOutOfMemory), "tuning events"};
  }
  const Call call{y, x, w, workspace, stream};
  const float alpha = 1.0f, beta = 0.0f;
  std::vector<std::pair<float, size_t>> times;
  for (size_t i = 0; i < all.size(); ++i) {
    Algo cand;
    cand.algo = all[i].algo;
    size_t need = 0;
    if (hipblaslt_ext::matmulIsAlgoSupported(handle, plan.desc, &alpha, plan.a, plan.b, &beta,
                                             plan.c, plan.c, cand.algo, need) !=
            HIPBLAS_STATUS_SUCCESS ||
        need > kBlasWorkspaceBytes) {
      continue;
    }
    const float ms = time_runs(handle, plan, cand, call, ev, kBlasSweepRuns);
    if (ms >= 0.0f) times.emplace_back(ms, i);
  }
  if (times.empty()) {
    destroy(plan);
    return BlasStatus{3, 0, "no algorithm serves this shape"};
  }
  std::sort(times.begin(), times.end());
  std::vector<Algo> keep;
  for (size_t i = 0; i < times.size() && static_cast<int>(keep.size()) < kBlasPreferred; ++i) {
    Algo cand;
    cand.algo = all[times[i].second].algo;
    keep.push_back(cand);
  }
  // y holds a product of the last algorithm run; leave it the fastest one's
  (void)matmul(handle, plan, keep[0], call);
  destroy(plan);
  g_preferred[PlanKey{dev, dtype, 0, n, k}] = keep;
  // choices already made for this (n, k) are made again, with these candidates
  for (auto it = g_algos.begin(); it != g_algos.end();) {
    it = (it->first.dev == dev && it->first.dtype == dtype && it->first.n == n && it->first.k == k)
             ? g_algos.erase(it)
             : std::next(it);
  }
  for (auto it = g_plans.begin(); it != g_plans.end();) {
    if (it->first.dev == dev && it->first.dtype == dtype && it->first.n == n && it->first.k == k) {
      destroy(it->second);
      it = g_plans.erase(it);
    } else {
      ++it;
    }
  }
  timed_out = static_cast<int>(times.size());
  return BlasStatus{0, 0, nullptr};
}

int blas_plans_cached() {
  std::lock_guard<std::mutex> lock(g_blas_mutex);
  return static_cast<int>(g_plans.size());
}

}  // namespace mvllm
