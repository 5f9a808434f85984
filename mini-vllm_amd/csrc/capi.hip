// The C ABI (include/minivllm_hip.h): argument validation, planning and launch.
//
// Validation mirrors the refusals of the reference's host entry points
// (csrc/paged_attention.cu:608-676, rmsnorm.cu:122-144, rope.cu:119-176,
// swiglu.cu:88-102) for everything expressible without torch tensors; the Python
// seam checks devices, dtypes and contiguity of the tensors before calling in.

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <cstdarg>
#include <mutex>

#include "../../include/minivllm_hip.h"
#include "blas.hpp"
#include "common.hpp"
#include "dense.hpp"
#include "elementwise.hpp"
#include "kv_write.hpp"
#include "linear.hpp"
#include "sampler.hpp"
#include "paged_attention.hpp"
#include "probe.hpp"

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return MVLLM_OK;
  return fail(MVLLM_ERR_HIP, "%s: HIP error %d (%s)", what, static_cast<int>(err),
              hipGetErrorString(err));
}

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// Compute units of the current device, cached per device id.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cached = cache[dev].load(std::memory_order_relaxed);
  if (cached > 0) return cached;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0) {
    cus = 256;
  }
  cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// The planner's options with the defaults filled in (mvllm_plan_options: 0 = default).
struct Options {
  int decode_schedule = 0;
  int decode_wgs_per_cu = 1;
  int decode_waves_per_cu = 16;
  int decode_split_tokens = 0;
  int prefill_schedule = 0;
  int prefill_wgs_per_cu = 1;
  int prefill_share_tiles = mvllm::kPrefillShareTiles;
  int prefill_staging = 0;
  int prefill_pieces = mvllm::kSplitDefaultPieces;
  int prefill_piece_pct = mvllm::kSplitDefaultPct;
};

int read_options(const mvllm_plan_options* o, Options& out) {
  out = Options{};
  if (o == nullptr) return MVLLM_OK;
  if (o->decode_schedule < 0 || o->decode_schedule > MVLLM_DECODE_GRID ||
      o->prefill_schedule < 0 || o->prefill_schedule > 2 || o->prefill_staging < 0 ||
      o->prefill_staging > 1 || o->decode_wgs_per_cu < 0 || o->decode_waves_per_cu < 0 ||
      o->decode_split_tokens < 0 || o->prefill_wgs_per_cu < 0 || o->prefill_share_tiles < 0 ||
      o->prefill_pieces < 0 || o->prefill_pieces > 64 || o->prefill_piece_pct < 0 ||
      (o->prefill_piece_pct > 0 && o->prefill_piece_pct < 50) || o->prefill_piece_pct > 10000) {
    return fail(MVLLM_ERR_INVALID, "paged_attention: plan options out of range");
  }
  out.decode_schedule = o->decode_schedule;
  if (o->decode_wgs_per_cu > 0) out.decode_wgs_per_cu = o->decode_wgs_per_cu;
  if (o->decode_waves_per_cu > 0) out.decode_waves_per_cu = o->decode_waves_per_cu;
  out.decode_split_tokens = o->decode_split_tokens;
  out.prefill_schedule = o->prefill_schedule;
  if (o->prefill_wgs_per_cu > 0) out.prefill_wgs_per_cu = o->prefill_wgs_per_cu;
  if (o->prefill_share_tiles > 0) out.prefill_share_tiles = o->prefill_share_tiles;
  out.prefill_staging = o->prefill_staging;
  if (o->prefill_pieces > 0) out.prefill_pieces = o->prefill_pieces;
  if (o->prefill_piece_pct > 0) out.prefill_piece_pct = o->prefill_piece_pct;
  return MVLLM_OK;
}

int check_paged_shape(int32_t num_tokens, int32_t num_seqs, int32_t hq, int32_t hk, int32_t d,
                      int32_t block_size, int32_t max_q, int32_t max_ctx, int32_t q_dtype,
                      int32_t kv_dtype) {
  if (num_tokens < 0 || num_seqs < 0) {
    return fail(MVLLM_ERR_INVALID, "paged_attention: negative token or sequence count");
  }
  if (q_dtype != mvllm::kF32 && q_dtype != mvllm::kF16 && q_dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "paged_attention: q dtype code %d is not supported (float32, float16 and "
                "bfloat16 are; float64 is not supported, the accumulators here are fp32)",
                q_dtype);
  }
  if (kv_dtype != q_dtype && kv_dtype != mvllm::kFP8E4M3) {
    return fail(MVLLM_ERR_INVALID,
                "paged_attention: q and the pools must share a dtype (or the pools be "
                "float8_e4m3fn), got codes %d and %d",
                q_dtype, kv_dtype);
  }
  if (d != 32 && d != 64 && d != 128 && d != 256) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "paged_attention: head dim %d is not supported; this build serves 32, 64, "
                "128 and 256",
                d);
  }
  if (hk <= 0 || hq <= 0 || hq % hk != 0) {
    return fail(MVLLM_ERR_INVALID, "paged_attention: H_q (%d) must be a multiple of H_k (%d)",
                hq, hk);
  }
  if (!is_pow2(block_size)) {
    return fail(MVLLM_ERR_INVALID,
                "paged_attention: the block size must be a power of two, got %d", block_size);
  }
  if (max_q < 1) {
    return fail(MVLLM_ERR_INVALID, "paged_attention: max_query_len must be >= 1, got %d", max_q);
  }
  if (max_ctx < max_q) {
    return fail(MVLLM_ERR_INVALID,
                "paged_attention: max_context_len (%d) must be at least max_query_len (%d); a "
                "pass cannot compute more tokens than it may attend over",
                max_ctx, max_q);
  }
  return MVLLM_OK;
}

// A plan plus the workspace layout it implies.
struct Plan {
  mvllm_paged_plan pub;
  int max_splits = 1;
  int register_staging = 0;  // prefill: the register-staged kernel even where direct-to-LDS serves
  int prefill_share_tiles = mvllm::kPrefillShareTiles;  // stream prefill: fewest tiles a share
  uint64_t off_o = 0;       // byte offsets into the workspace
  uint64_t off_ml = 0;
  uint64_t off_pf = 0;      // stream prefill: [prefix][O partials][(m, l) partials]
  uint64_t off_pf_o = 0;
  uint64_t off_pf_ml = 0;
  int split_ranks = 0;      // split prefill grid: rank extent, partial slots per column,
  int split_slots = 0;      // piece length (percent of the mean tiles per CU)
  int split_pct = 0;
  uint64_t off_split = 0;   // split prefill grid: the partial slots
};

uint64_t align256(uint64_t v) { return (v + 255) / 256 * 256; }

void plan_decode(Plan& plan, int32_t num_tokens, int32_t num_seqs, int32_t hq, int32_t hk,
                 int32_t d, int32_t block_size, int32_t max_q, int32_t max_ctx, int32_t q_dtype,
                 int32_t kv_dtype, const Options& o);

// The MFMA prefill's schedule. The grid (one workgroup per 128-query item) is chosen
// when there are at least half as many items as CUs: the hardware dispatcher then
// balances them, with no partials to merge (four 512-query chunks beside 28 decodes,
// 136 items: grid 102 us, stream 110 us). With fewer items (one chunk of a long
// prompt, 40 items: stream 104 us, grid 109 us) the grid would leave CUs idle behind a
// few long items, so
// the stream schedule is used: one persistent workgroup per CU (times the
// prefill_wgs_per_cu option) with balanced shares of all key tiles, cut items merged
// after (measured at 8K-16K contexts: 2.5-3x the grid). The item count is estimated
// from host sizes: ceil(num_tokens / 128) query tiles per kv column. The
// prefill_schedule option 1 / 2 forces stream / grid. The stream's workspace follows
// the decode part's.
// The grid's split (pieces of long items, merged in the same launch) where the
// pipelined kernel runs it: D = 128, GQA pairs, pages of >= 16 keys, 16-bit or fp8
// pools, and at most kSplitMaxItems items (bounded from host sizes: a sequence of L
// queries has ceil(L / 128) items, so there are at most min(num_seqs * ceil(max_q /
// 128), ceil(num_tokens / 128) + num_seqs)) over at most kSplitMaxCols columns.
void plan_split(Plan& plan, int32_t num_tokens, int32_t num_seqs, int32_t hq, int32_t hk,
                int32_t d, int32_t block_size, int32_t max_q, int32_t q_dtype, int32_t kv_dtype,
                const Options& o) {
  if (o.prefill_pieces < 2 || o.prefill_staging != 0 || d != 128 ||
      mvllm::prefill_item_heads(hq / hk) != 2 || block_size < 16) {
    return;
  }
  if (q_dtype != mvllm::kF16 && q_dtype != mvllm::kBF16) return;
  if (kv_dtype != q_dtype && kv_dtype != mvllm::kFP8E4M3) return;
  const int64_t q_tiles = (max_q + mvllm::kPrefillQueryTile - 1) / mvllm::kPrefillQueryTile;
  const int64_t by_seqs = static_cast<int64_t>(num_seqs) * q_tiles;
  const int64_t by_tokens =
      (static_cast<int64_t>(num_tokens) + mvllm::kPrefillQueryTile - 1) / mvllm::kPrefillQueryTile +
      num_seqs;
  const int64_t items = by_seqs < by_tokens ? by_seqs : by_tokens;
  const int cols = hq / 2;
  if (items > mvllm::kSplitMaxItems || cols > mvllm::kSplitMaxCols) return;
  const int cus = device_cus();
  plan.pub.prefill_pieces = o.prefill_pieces;
  plan.split_pct = o.prefill_piece_pct;
  plan.split_ranks = static_cast<int>(items) + mvllm::split_extra_ranks(cus, cols, plan.split_pct);
  plan.split_slots = mvllm::split_slots(cus, cols, plan.split_pct);
  plan.off_split = align256(plan.pub.workspace_bytes);
  plan.pub.workspace_bytes =
      plan.off_split + static_cast<uint64_t>(plan.split_slots) * cols * mvllm::kSplitSlotFloats *
                           sizeof(float);
}

void plan_prefill(Plan& plan, int32_t num_tokens, int32_t num_seqs, int32_t hq, int32_t hk,
                  int32_t d, int32_t block_size, int32_t max_q, int32_t q_dtype,
                  int32_t kv_dtype, const Options& o) {
  if (!plan.pub.prefill_mfma) return;
  plan.register_staging = o.prefill_staging;
  plan.prefill_share_tiles = o.prefill_share_tiles;
  const int forced = o.prefill_schedule;
  const int64_t items = static_cast<int64_t>((num_tokens + mvllm::kPrefillQueryTile - 1) /
                                             mvllm::kPrefillQueryTile) *
                        (hq / mvllm::prefill_item_heads(hq / hk));
  if (num_seqs > mvllm::kMaxStreamSeqs || forced == 2 ||
      (forced != 1 && 2 * items >= device_cus())) {
    plan_split(plan, num_tokens, num_seqs, hq, hk, d, block_size, max_q, q_dtype, kv_dtype, o);
    return;
  }
  int64_t wgs = static_cast<int64_t>(o.prefill_wgs_per_cu) * device_cus();
  if (wgs > mvllm::kMaxPrefillWgs) wgs = mvllm::kMaxPrefillWgs;
  const uint64_t rows = static_cast<uint64_t>(2 * wgs) * mvllm::prefill_item_heads(hq / hk) *
                        mvllm::kPrefillQueryTile;
  plan.pub.prefill_workgroups = static_cast<int32_t>(wgs);
  plan.off_pf = align256(plan.pub.workspace_bytes);
  plan.off_pf_o = plan.off_pf + align256(static_cast<uint64_t>(num_seqs + 1) * sizeof(int));
  plan.off_pf_ml = plan.off_pf_o + align256(rows * d * sizeof(float));
  plan.pub.workspace_bytes = plan.off_pf_ml + align256(rows * 2 * sizeof(float));
}

Plan make_plan(int32_t num_tokens, int32_t num_seqs, int32_t hq, int32_t hk, int32_t d,
               int32_t block_size, int32_t max_q, int32_t max_ctx, int32_t q_dtype,
               int32_t kv_dtype, const Options& o = Options{}) {
  Plan plan{};
  plan_decode(plan, num_tokens, num_seqs, hq, hk, d, block_size, max_q, max_ctx, q_dtype,
              kv_dtype, o);
  plan_prefill(plan, num_tokens, num_seqs, hq, hk, d, block_size, max_q, q_dtype, kv_dtype, o);
  return plan;
}

void plan_decode(Plan& plan, int32_t num_tokens, int32_t num_seqs, int32_t hq, int32_t hk,
                 int32_t d, int32_t block_size, int32_t max_q, int32_t max_ctx, int32_t q_dtype,
                 int32_t kv_dtype, const Options& o) {
  const bool has_prefill = max_q > 1;
  const bool mfma =
      has_prefill && mvllm::paged_prefill_supported(q_dtype, kv_dtype, d, hq, hk, block_size);
  // Query lengths are at most max_q and sum to num_tokens, so num_tokens ==
  // num_seqs * max_q (with max_q > 1) means every sequence is a prefill chunk.
  const bool all_prefill =
      has_prefill && static_cast<int64_t>(num_seqs) * max_q == static_cast<int64_t>(num_tokens);
  const int64_t units = static_cast<int64_t>(hk) * (hq / hk / mvllm::decode_group_chunk(hq / hk));
  plan.pub.prefill_mfma = mfma ? 1 : 0;

  if (has_prefill && !mfma) {
    plan.pub.decode_mode = MVLLM_DECODE_BY_ROW;
  } else if (all_prefill || num_seqs == 0) {
    plan.pub.decode_mode = MVLLM_DECODE_NONE;
  } else if (num_seqs <= mvllm::kMaxStreamSeqs && units <= 8 &&
             static_cast<int64_t>(num_seqs) * max_ctx < (int64_t{1} << 31) &&
             o.decode_schedule != MVLLM_DECODE_GRID) {
    plan.pub.decode_mode = MVLLM_DECODE_STREAM;
  } else {
    plan.pub.decode_mode = MVLLM_DECODE_GRID;
  }

  if (plan.pub.decode_mode == MVLLM_DECODE_STREAM) {
    // A few workgroups per CU, each streaming an equal share of all decode keys; no
    // more workgroups than there are ~64-key shares in the largest possible batch.
    int64_t wgs = static_cast<int64_t>(o.decode_wgs_per_cu) * device_cus();
    const int64_t by_size = (static_cast<int64_t>(num_seqs) * max_ctx + 63) / 64;
    if (wgs > by_size) wgs = by_size;
    if (wgs < 1) wgs = 1;
    plan.pub.decode_workgroups = static_cast<int32_t>(wgs);
    // [prefix: num_seqs + 1 int32][O partials][(m, l) partials]
    const uint64_t entries = static_cast<uint64_t>(wgs + num_seqs) * hq;
    const uint64_t head = align256(static_cast<uint64_t>(num_seqs + 1) * sizeof(int));
    plan.off_o = head;
    plan.off_ml = plan.off_o + align256(entries * d * sizeof(float));
    plan.pub.workspace_bytes = plan.off_ml + align256(entries * 2 * sizeof(float));
    return;
  }
  if (plan.pub.decode_mode == MVLLM_DECODE_NONE) return;

  // Grid schedules: split each row's context until the grid holds ~16 waves per CU,
  // in splits of 64..1024 keys.
  const int64_t rows = plan.pub.decode_mode == MVLLM_DECODE_BY_ROW ? num_tokens : num_seqs;
  const int64_t target = static_cast<int64_t>(o.decode_waves_per_cu) * device_cus();
  const int64_t single = rows * units > 0 ? rows * units : 1;
  const int64_t wanted = (target + single - 1) / single;
  int64_t split = (max_ctx + wanted - 1) / wanted;
  split = (split + 63) / 64 * 64;
  const int override_split = o.decode_split_tokens;
  if (override_split > 0) split = (override_split + 15) / 16 * 16;
  if (split < 64) split = 64;
  if (split > mvllm::kMaxSplitTokens) split = mvllm::kMaxSplitTokens;
  const int64_t max_splits = (max_ctx + split - 1) / split;
  plan.pub.split_tokens = static_cast<int32_t>(split);
  plan.max_splits = static_cast<int>(max_splits < 1 ? 1 : max_splits);
  plan.pub.decode_workgroups = plan.max_splits;
  if (plan.max_splits > 1 && rows > 0) {
    const uint64_t entries = static_cast<uint64_t>(rows) * hq * plan.max_splits;
    plan.off_ml = align256(entries * d * sizeof(float));
    plan.pub.workspace_bytes = plan.off_ml + align256(entries * 2 * sizeof(float));
  }
}

// Arrival counters of the split prefill grid, in a static device array (each GPU holds
// its own from the library's load until the process ends; it starts at zero and every
// launch leaves its counters at zero). A stream takes one region of it on its first
// split launch and keeps it, so launches that may overlap in time (other streams)
// never share counters, while one stream's launches run in order. A stream beyond the
// regions runs its prefill with every item whole, and so does a launch made while its
// stream is being captured into a graph: the graph would carry the capture stream's
// region in its kernel arguments, and a replay on another stream could then overlap a
// launch still running on the capture stream over the same counters. Both cases are
// counted (mvllm_split_stats). Host code never names the array itself: each device's
// address comes from hipGetSymbolAddress, kept here.
constexpr int kCounterRegions = 32;
constexpr int kCounterInts = mvllm::kSplitMaxItems * mvllm::kSplitMaxCols;
static __device__ __align__(256) int split_counters[kCounterRegions * kCounterInts];

constexpr int kCounterDevices = 64;
std::mutex g_counter_mutex;
int* g_counter_base[kCounterDevices] = {};
hipStream_t g_counter_owner[kCounterDevices][kCounterRegions] = {};
bool g_counter_used[kCounterDevices][kCounterRegions] = {};
std::atomic<int64_t> g_split_whole_no_region{0};   // split launches run whole: no region left
std::atomic<int64_t> g_split_whole_capturing{0};   // split launches run whole: stream capturing

// The counter region of (current device, stream), or nullptr when there is none to give.
int* split_counters_for(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kCounterDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_counter_mutex);
  if (g_counter_base[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(split_counters)) != hipSuccess || ptr == nullptr) {
      return nullptr;
    }
    g_counter_base[dev] = static_cast<int*>(ptr);
  }
  int free_region = -1;
  for (int r = 0; r < kCounterRegions; ++r) {
    if (g_counter_used[dev][r] && g_counter_owner[dev][r] == stream) {
      return g_counter_base[dev] + r * kCounterInts;
    }
    if (!g_counter_used[dev][r] && free_region < 0) free_region = r;
  }
  if (free_region < 0) {
    g_split_whole_no_region.fetch_add(1, std::memory_order_relaxed);
    return nullptr;
  }
  g_counter_used[dev][free_region] = true;
  g_counter_owner[dev][free_region] = stream;
  return g_counter_base[dev] + free_region * kCounterInts;
}

// Fills the plan's schedule fields and workspace pointers into `p` and launches the
// decode and prefill kernels the plan names (shared by the paged and dense entries).
int launch_planned(const Plan& plan, mvllm::PagedParams& p, void* workspace, int32_t q_dtype,
                   int32_t kv_dtype, int32_t head_dim, int32_t max_query_len, hipStream_t s,
                   const char* name) {
  p.stream_wgs = plan.pub.decode_mode == MVLLM_DECODE_STREAM ? plan.pub.decode_workgroups : 0;
  p.split_tokens = plan.pub.split_tokens > 0 ? plan.pub.split_tokens : mvllm::kMaxSplitTokens;
  p.max_splits = plan.max_splits;
  p.by_row = plan.pub.decode_mode == MVLLM_DECODE_BY_ROW ? 1 : 0;
  p.pf_register_staging = plan.register_staging;
  p.pf_share_tiles = plan.prefill_share_tiles;
  if (plan.pub.workspace_bytes > 0) {
    char* ws = static_cast<char*>(workspace);
    if (plan.pub.decode_mode == MVLLM_DECODE_STREAM) p.seq_prefix = reinterpret_cast<int*>(ws);
    p.part_o = reinterpret_cast<float*>(ws + plan.off_o);
    p.part_ml = reinterpret_cast<float*>(ws + plan.off_ml);
    if (plan.pub.prefill_workgroups > 0) {
      p.pf_wgs = plan.pub.prefill_workgroups;
      p.pf_prefix = reinterpret_cast<int*>(ws + plan.off_pf);
      p.pf_o = reinterpret_cast<float*>(ws + plan.off_pf_o);
      p.pf_ml = reinterpret_cast<float*>(ws + plan.off_pf_ml);
    }
    if (plan.pub.prefill_pieces > 1) {
      hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(s, &capture) != hipSuccess ||
          capture != hipStreamCaptureStatusNone) {
        g_split_whole_capturing.fetch_add(1, std::memory_order_relaxed);
        p.pf_count = nullptr;  // items whole: a graph must not name a stream's counters
      } else {
        p.pf_count = split_counters_for(s);
      }
      if (p.pf_count != nullptr) {
        p.pf_pieces = plan.pub.prefill_pieces;
        p.pf_ranks = plan.split_ranks;
        p.pf_slots = plan.split_slots;
        p.pf_cus = device_cus();
        p.pf_piece_pct = plan.split_pct;
        p.pf_part = reinterpret_cast<float*>(ws + plan.off_split);
      }
    }
  }
  if (plan.pub.decode_mode != MVLLM_DECODE_NONE) {
    const int rc = hip_status(mvllm::launch_paged_decode(p, q_dtype, kv_dtype, head_dim, s),
                              name);
    if (rc != MVLLM_OK) return rc;
  }
  if (plan.pub.prefill_mfma) {
    const int rc = hip_status(
        mvllm::launch_paged_prefill(p, q_dtype, kv_dtype, head_dim, max_query_len, s), name);
    if (rc != MVLLM_OK) return rc;
  }
  return MVLLM_OK;
}

// The dense entries' checks, their virtual-page geometry and their workspace layout:
// the metadata first, then the paged plan's workspace.
struct DensePlan {
  Plan plan;
  int max_blocks = 0;
  int64_t slots_per_batch = 0;
  uint64_t off_tables = 0, off_cu = 0, off_ctx = 0, off_len = 0, off_paged = 0;
  uint64_t bytes = 0;
};

int dense_plan(const mvllm_dense_args* a, DensePlan& d) {
  if (a == nullptr) return fail(MVLLM_ERR_INVALID, "dense_attention: args is NULL");
  const char* name = a->query_len == 1 ? "decode_attention" : "flash_prefill";
  if (a->dtype != mvllm::kF32 && a->dtype != mvllm::kF16 && a->dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "%s: dtype code %d is not supported (float32, float16, bfloat16); float64 is not "
                "supported, the accumulators here are fp32",
                name, a->dtype);
  }
  if (a->batch < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 ||
      a->num_q_heads % a->num_kv_heads != 0) {
    return fail(MVLLM_ERR_INVALID, "%s: H_q (%d) must be a multiple of H_k (%d)", name,
                a->num_q_heads, a->num_kv_heads);
  }
  if (a->kv_len <= 0) {
    return fail(MVLLM_ERR_INVALID,
                "%s: the cache is empty, so there is nothing to attend to; softmax over zero "
                "keys is undefined",
                name);
  }
  if (a->query_len <= 0 || a->kv_len < a->query_len) {
    return fail(MVLLM_ERR_INVALID,
                "%s: %d queries against %d keys; this kernel masks causally, which needs S >= L "
                "> 0",
                name, a->query_len, a->kv_len);
  }
  const int esize = a->dtype == mvllm::kF32 ? 4 : 2;
  const int64_t sp = a->k_stride_pos, sh = a->k_stride_head, sb = a->k_stride_batch;
  if (sp != a->v_stride_pos || sh != a->v_stride_head || (a->batch > 1 && sb != a->v_stride_batch)) {
    return fail(MVLLM_ERR_UNSUPPORTED, "%s: k and v must share their strides", name);
  }
  if (sp <= 0 || sh < 0 || sb < 0 || (sp * esize) % 16 != 0 || (sh * esize) % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(a->k) | reinterpret_cast<uintptr_t>(a->v) |
       reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->out)) % 16 != 0) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: the position and head strides of k and v must be positive multiples of 16 "
                "bytes and every pointer 16-byte aligned",
                name);
  }
  if (a->batch > 1 && sb % sp != 0) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: the batch stride of k and v (%lld) must be a multiple of the position "
                "stride (%lld)",
                name, static_cast<long long>(sb), static_cast<long long>(sp));
  }
  d.max_blocks = (a->kv_len + 15) / 16;
  d.slots_per_batch = a->batch > 1 ? sb / sp : 0;
  if ((a->batch - 1) * d.slots_per_batch + 16 * static_cast<int64_t>(d.max_blocks) >=
          (int64_t{1} << 31) ||
      sh * esize * a->num_kv_heads >= (int64_t{1} << 32) || sp * esize * 16 >= (int64_t{1} << 32)) {
    return fail(MVLLM_ERR_UNSUPPORTED, "%s: the cache is too large for 32-bit page ids", name);
  }
  const int64_t tokens = static_cast<int64_t>(a->batch) * a->query_len;
  if (tokens >= (int64_t{1} << 31)) return fail(MVLLM_ERR_UNSUPPORTED, "%s: too many queries", name);
  const int rc = check_paged_shape(static_cast<int32_t>(tokens), a->batch, a->num_q_heads,
                                   a->num_kv_heads, a->head_dim, 16, a->query_len, a->kv_len,
                                   a->dtype, a->dtype);
  if (rc != MVLLM_OK) return rc;
  d.plan = make_plan(static_cast<int32_t>(tokens), a->batch, a->num_q_heads, a->num_kv_heads,
                     a->head_dim, 16, a->query_len, a->kv_len, a->dtype, a->dtype);
  const uint64_t b = static_cast<uint64_t>(a->batch);
  d.off_tables = 0;
  d.off_cu = align256(b * d.max_blocks * 4);
  d.off_ctx = d.off_cu + align256((b + 1) * 4);
  d.off_len = d.off_ctx + align256(b * 4);
  d.off_paged = d.off_len + align256(b * 4);
  d.bytes = d.off_paged + d.plan.pub.workspace_bytes;
  return MVLLM_OK;
}

// Checks and launch of the fused QK-norm + RoPE, optionally writing the KV pools.
int qk_norm_rope_entry(void* q_out, void* k_out, const void* q, const void* k,
                       const void* q_weight, const void* k_weight, const void* positions,
                       int32_t positions_bytes, const float* cos_table, const float* sin_table,
                       int64_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, int64_t num_positions, int64_t max_positions, float eps,
                       int32_t dtype, void* stream, const void* v, void* k_pool, void* v_pool,
                       const int32_t* slots, int64_t num_slots = 0, int64_t q_token_stride = 0,
                       int64_t kv_token_stride = 0) {
  if (dtype != mvllm::kF32 && dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "qk_norm_rope: dtype code %d is not supported; float64 is not supported", dtype);
  }
  if (!mvllm::qk_norm_rope_supported(dtype, head_dim)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "qk_norm_rope: head dim %d is not supported (16-byte chunks per head must be "
                "a power of two from 2 to 64); call rmsnorm and rope",
                head_dim);
  }
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0) {
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: bad shape");
  }
  if (positions_bytes != 4 && positions_bytes != 8) {
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: positions must be int32 or int64");
  }
  if (num_tokens == 0) return MVLLM_OK;
  if (num_positions <= 0 || num_tokens % num_positions != 0) {
    return fail(MVLLM_ERR_INVALID,
                "qk_norm_rope: %lld tokens is not a multiple of the %lld positions given, so the "
                "positions cannot broadcast over them",
                static_cast<long long>(num_tokens), static_cast<long long>(num_positions));
  }
  if (max_positions <= 0) return fail(MVLLM_ERR_INVALID, "qk_norm_rope: empty cos/sin tables");
  if (q_out == nullptr || (k_out == nullptr && k_pool == nullptr) || q == nullptr || k == nullptr ||
      q_weight == nullptr || k_weight == nullptr || positions == nullptr ||
      cos_table == nullptr || sin_table == nullptr) {
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: a required pointer is NULL");
  }
  const uintptr_t bits = reinterpret_cast<uintptr_t>(q_out) | reinterpret_cast<uintptr_t>(k_out) |
                         reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(q_weight) |
                         reinterpret_cast<uintptr_t>(k_weight) |
                         reinterpret_cast<uintptr_t>(cos_table) |
                         reinterpret_cast<uintptr_t>(sin_table);
  if (bits % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: every tensor must be 16-byte aligned");
  }
  // Token strides: whole head vectors per token, each token's rows 16-byte aligned.
  const int64_t elem = dtype == mvllm::kF32 ? 4 : 2;
  const int64_t q_row = static_cast<int64_t>(num_q_heads) * head_dim;
  const int64_t kv_row = static_cast<int64_t>(num_kv_heads) * head_dim;
  const int64_t qs = q_token_stride > 0 ? q_token_stride : q_row;
  const int64_t kvs = kv_token_stride > 0 ? kv_token_stride : kv_row;
  if (qs < q_row || kvs < kv_row || (qs * elem) % 16 != 0 || (kvs * elem) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "qk_norm_rope: token strides %lld (q) and %lld (k, v) must cover the token's "
                "heads (%lld, %lld elements) and keep every token 16-byte aligned",
                static_cast<long long>(qs), static_cast<long long>(kvs),
                static_cast<long long>(q_row), static_cast<long long>(kv_row));
  }
  return hip_status(
      mvllm::launch_qk_norm_rope(q, k, q_weight, k_weight, positions, positions_bytes, cos_table,
                                 sin_table, q_out, k_out, num_tokens, num_q_heads, num_kv_heads,
                                 head_dim, num_positions, max_positions, eps, dtype,
                                 static_cast<hipStream_t>(stream), v, k_pool, v_pool, slots,
                                 num_slots, qs, kvs),
      "qk_norm_rope: launch");
}

}  // namespace

extern "C" {

const char* mvllm_last_error(void) { return g_error; }

int mvllm_abi_version(void) { return 15; }

#ifndef MVLLM_SOURCE_HASH
#define MVLLM_SOURCE_HASH "unstamped"
#endif
const char* mvllm_build_id(void) { return MVLLM_SOURCE_HASH; }

void mvllm_split_stats(int32_t* regions_used, int64_t* whole_no_region,
                       int64_t* whole_capturing) {
  int dev = 0;
  int used = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kCounterDevices) {
    std::lock_guard<std::mutex> lock(g_counter_mutex);
    for (int r = 0; r < kCounterRegions; ++r) used += g_counter_used[dev][r] ? 1 : 0;
  }
  if (regions_used != nullptr) *regions_used = used;
  if (whole_no_region != nullptr) *whole_no_region = g_split_whole_no_region.load();
  if (whole_capturing != nullptr) *whole_capturing = g_split_whole_capturing.load();
}

int mvllm_paged_attention_plan(int32_t num_tokens, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t max_query_len, int32_t max_context_len, int32_t q_dtype,
                               int32_t kv_dtype, const mvllm_plan_options* options,
                               mvllm_paged_plan* plan) {
  g_error[0] = '\0';
  if (plan == nullptr) return fail(MVLLM_ERR_INVALID, "paged_attention_plan: plan is NULL");
  int rc = check_paged_shape(num_tokens, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             block_size, max_query_len, max_context_len, q_dtype, kv_dtype);
  if (rc != MVLLM_OK) return rc;
  Options o;
  rc = read_options(options, o);
  if (rc != MVLLM_OK) return rc;
  *plan = make_plan(num_tokens, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                    max_query_len, max_context_len, q_dtype, kv_dtype, o)
              .pub;
  return MVLLM_OK;
}

}  // extern "C"

namespace {

// The paged entry behind mvllm_paged_attention and mvllm_paged_attention_noalloc: the
// scratch pointer is the caller's workspace for the first and this library's static
// device array for the second (`name` prefixes the errors).
int paged_attention_entry(const char* name, void* out, const void* q, const void* key_pool,
                          const void* value_pool, const float* k_scales, const float* v_scales,
                          const int32_t* block_tables, const int32_t* cu_seqlens_q,
                          const int32_t* context_lens, const int32_t* seq_lens,
                          int32_t num_tokens, int32_t num_seqs, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int64_t num_blocks, int32_t max_blocks_per_seq, int32_t max_query_len,
                          int32_t max_context_len, float scale, int32_t q_dtype,
                          int32_t kv_dtype, const mvllm_plan_options* options, void* workspace,
                          uint64_t workspace_bytes, void* stream, bool static_scratch) {
  int rc = check_paged_shape(num_tokens, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             block_size, max_query_len, max_context_len, q_dtype, kv_dtype);
  if (rc != MVLLM_OK) return rc;
  Options o;
  rc = read_options(options, o);
  if (rc != MVLLM_OK) return rc;
  if (num_tokens == 0 || num_seqs == 0) return MVLLM_OK;
  if (out == nullptr || q == nullptr || key_pool == nullptr ||
      value_pool == nullptr || block_tables == nullptr || cu_seqlens_q == nullptr ||
      context_lens == nullptr || seq_lens == nullptr) {
    return fail(MVLLM_ERR_INVALID, "%s: a required pointer is NULL", name);
  }
  if (num_blocks <= 0 || max_blocks_per_seq <= 0) {
    return fail(MVLLM_ERR_INVALID, "paged_attention: empty pool or block table");
  }
  const bool fp8 = kv_dtype == mvllm::kFP8E4M3;
  if (fp8 != (k_scales != nullptr && v_scales != nullptr) || (!fp8 && (k_scales || v_scales))) {
    return fail(MVLLM_ERR_INVALID,
                "paged_attention: k_scales and v_scales are required for a float8 pool and "
                "only for one");
  }
  Plan plan = make_plan(num_tokens, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                        max_query_len, max_context_len, q_dtype, kv_dtype, o);
  if (static_scratch && plan.pub.workspace_bytes > workspace_bytes && plan.pub.prefill_pieces > 1) {
    // The split grid's partial slots do not fit the static scratch: items stay whole.
    o.prefill_pieces = 1;
    plan = make_plan(num_tokens, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                     max_query_len, max_context_len, q_dtype, kv_dtype, o);
  }
  const uint64_t need = plan.pub.workspace_bytes;
  if (static_scratch && need > workspace_bytes) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: this call needs %llu bytes of scratch, more than the library's static "
                "%llu (a prefill on the stream schedule is the usual cause: plan options "
                "prefill_schedule = 2 run it on the grid, which needs none)",
                name, static_cast<unsigned long long>(need),
                static_cast<unsigned long long>(workspace_bytes));
  }
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(MVLLM_ERR_WORKSPACE,
                "paged_attention: workspace of %llu bytes is smaller than the %llu the plan "
                "needs (call mvllm_paged_attention_plan)",
                static_cast<unsigned long long>(workspace_bytes),
                static_cast<unsigned long long>(need));
  }
  if (need > 0 && reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    return fail(MVLLM_ERR_INVALID, "paged_attention: the workspace must be 256-byte aligned");
  }

  int shift = 0;
  while ((1 << shift) < block_size) ++shift;

  mvllm::PagedParams p{};
  p.q = q;
  p.k_pool = key_pool;
  p.v_pool = value_pool;
  p.k_scales = k_scales;
  p.v_scales = v_scales;
  p.out = out;
  p.block_tables = block_tables;
  p.cu_seqlens_q = cu_seqlens_q;
  p.context_lens = context_lens;
  p.seq_lens = seq_lens;
  p.num_seqs = num_seqs;
  p.num_tokens = num_tokens;
  p.hq = num_q_heads;
  p.hk = num_kv_heads;
  p.max_blocks = max_blocks_per_seq;
  p.block_shift = shift;
  p.block_mask = block_size - 1;
  p.table_shift = shift;
  const int64_t kv_elem = kv_dtype == mvllm::kF32 ? 4 : (kv_dtype == mvllm::kFP8E4M3 ? 1 : 2);
  p.kv_head_bytes = static_cast<int64_t>(head_dim) * kv_elem;
  p.kv_row_bytes = p.kv_head_bytes * num_kv_heads;
  p.scale = scale;
  return launch_planned(plan, p, workspace, q_dtype, kv_dtype, head_dim, max_query_len,
                        static_cast<hipStream_t>(stream), name);
}

// The allocation-free entry's scratch: one array per device, held from the library's
// load until the process ends. Host code never names it directly (its host-side name
// is a stand-in, not a device address); each device's address comes from
// hipGetSymbolAddress once, with that device current, and is kept here.
constexpr uint64_t kNoallocScratchBytes = MVLLM_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address (resolved on the device's first call).
int scratch_for_current_device(void** ptr) {
  int dev = 0;
  int rc = hip_status(hipGetDevice(&dev), "paged_attention_noalloc: hipGetDevice");
  if (rc != MVLLM_OK) return rc;
  if (dev < 0 || dev >= kMaxDevices) {
    return fail(MVLLM_ERR_UNSUPPORTED, "paged_attention_noalloc: device %d out of range", dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                    "paged_attention_noalloc: hipGetSymbolAddress");
    if (rc != MVLLM_OK) return rc;
    if (p == nullptr || reinterpret_cast<uintptr_t>(p) % 256 != 0) {
      return fail(MVLLM_ERR_HIP, "paged_attention_noalloc: bad scratch address");
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MVLLM_OK;
}

}  // namespace

extern "C" {

int mvllm_paged_attention(void* out, const void* q, const void* key_pool,
                          const void* value_pool, const float* k_scales, const float* v_scales,
                          const int32_t* block_tables, const int32_t* cu_seqlens_q,
                          const int32_t* context_lens, const int32_t* seq_lens,
                          int32_t num_tokens, int32_t num_seqs, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int64_t num_blocks, int32_t max_blocks_per_seq, int32_t max_query_len,
                          int32_t max_context_len, float scale, int32_t q_dtype,
                          int32_t kv_dtype, const mvllm_plan_options* options, void* workspace,
                          uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  return paged_attention_entry("paged_attention", out, q, key_pool, value_pool, k_scales,
                               v_scales, block_tables, cu_seqlens_q, context_lens, seq_lens,
                               num_tokens, num_seqs, num_q_heads, num_kv_heads, head_dim,
                               block_size, num_blocks, max_blocks_per_seq, max_query_len,
                               max_context_len, scale, q_dtype, kv_dtype, options, workspace,
                               workspace_bytes, stream, false);
}

int mvllm_paged_attention_noalloc(void* out, const void* q, const void* key_pool,
                                  const void* value_pool, const float* k_scales,
                                  const float* v_scales, const int32_t* block_tables,
                                  const int32_t* cu_seqlens_q, const int32_t* context_lens,
                                  const int32_t* seq_lens, int32_t num_tokens, int32_t num_seqs,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int64_t num_blocks,
                                  int32_t max_blocks_per_seq, int32_t max_query_len,
                                  int32_t max_context_len, float scale, int32_t q_dtype,
                                  int32_t kv_dtype, const mvllm_plan_options* options,
                                  void* stream) {
  g_error[0] = '\0';
  void* ws = nullptr;
  if (num_tokens > 0 && num_seqs > 0) {
    const int rc = scratch_for_current_device(&ws);
    if (rc != MVLLM_OK) return rc;
  }
  return paged_attention_entry("paged_attention_noalloc", out, q, key_pool, value_pool,
                               k_scales, v_scales, block_tables, cu_seqlens_q, context_lens,
                               seq_lens, num_tokens, num_seqs, num_q_heads, num_kv_heads,
                               head_dim, block_size, num_blocks, max_blocks_per_seq,
                               max_query_len, max_context_len, scale, q_dtype, kv_dtype,
                               options, ws, kNoallocScratchBytes, stream, true);
}

int mvllm_paged_decode_qk_norm_rope(
    void* out, const void* q, const void* k, const void* v, int64_t q_token_stride,
    int64_t kv_token_stride, const void* q_weight, const void* k_weight, const float* cos_table,
    const float* sin_table, int64_t max_positions, float eps, void* key_pool, void* value_pool,
    const int32_t* block_tables, const int32_t* cu_seqlens_q, const int32_t* context_lens,
    const int32_t* seq_lens, int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_blocks_per_seq,
    int32_t max_context_len, float scale, int32_t dtype, const mvllm_plan_options* options,
    void* workspace, uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  const char* name = "paged_decode_qk_norm_rope";
  int rc = check_paged_shape(num_seqs, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                             1, max_context_len, dtype, dtype);
  if (rc != MVLLM_OK) return rc;
  Options o;
  rc = read_options(options, o);
  if (rc != MVLLM_OK) return rc;
  if (dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: dtype code %d is not served (float16 and bfloat16 pools are; call "
                "mvllm_qk_norm_rope_kv_write then mvllm_paged_attention)",
                name, dtype);
  }
  if (head_dim != 128) {
    return fail(MVLLM_ERR_UNSUPPORTED, "%s: head dim %d is not served (128 is)", name, head_dim);
  }
  if (num_seqs == 0) return MVLLM_OK;
  if (out == nullptr || q == nullptr || k == nullptr || v == nullptr || q_weight == nullptr ||
      k_weight == nullptr || cos_table == nullptr || sin_table == nullptr ||
      key_pool == nullptr || value_pool == nullptr || block_tables == nullptr ||
      cu_seqlens_q == nullptr || context_lens == nullptr || seq_lens == nullptr) {
    return fail(MVLLM_ERR_INVALID, "%s: a required pointer is NULL", name);
  }
  if (num_blocks <= 0 || max_blocks_per_seq <= 0 || max_positions <= 0) {
    return fail(MVLLM_ERR_INVALID, "%s: empty pool, block table or cos/sin tables", name);
  }
  const uintptr_t bits = reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(q) |
                         reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                         reinterpret_cast<uintptr_t>(q_weight) |
                         reinterpret_cast<uintptr_t>(k_weight) |
                         reinterpret_cast<uintptr_t>(cos_table) |
                         reinterpret_cast<uintptr_t>(sin_table) |
                         reinterpret_cast<uintptr_t>(key_pool) |
                         reinterpret_cast<uintptr_t>(value_pool);
  if (bits % 16 != 0) return fail(MVLLM_ERR_INVALID, "%s: every tensor must be 16-byte aligned", name);
  const int64_t q_row = static_cast<int64_t>(num_q_heads) * head_dim;
  const int64_t kv_row = static_cast<int64_t>(num_kv_heads) * head_dim;
  const int64_t qs = q_token_stride > 0 ? q_token_stride : q_row;
  const int64_t kvs = kv_token_stride > 0 ? kv_token_stride : kv_row;
  if (qs < q_row || kvs < kv_row || qs % 8 != 0 || kvs % 8 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "%s: token strides %lld (q) and %lld (k, v) must cover the token's heads (%lld, "
                "%lld elements) and keep every token 16-byte aligned",
                name, static_cast<long long>(qs), static_cast<long long>(kvs),
                static_cast<long long>(q_row), static_cast<long long>(kv_row));
  }
  const Plan plan = make_plan(num_seqs, num_seqs, num_q_heads, num_kv_heads, head_dim,
                              block_size, 1, max_context_len, dtype, dtype, o);
  if (plan.pub.decode_mode != MVLLM_DECODE_STREAM) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: the plan puts this batch on the grid schedule, which the fused entry does "
                "not serve (call mvllm_qk_norm_rope_kv_write then mvllm_paged_attention)",
                name);
  }
  const uint64_t need = plan.pub.workspace_bytes;
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(MVLLM_ERR_WORKSPACE,
                "%s: workspace of %llu bytes is smaller than the %llu the plan needs (call "
                "mvllm_paged_attention_plan with num_tokens = num_seqs, max_query_len = 1)",
                name, static_cast<unsigned long long>(workspace_bytes),
                static_cast<unsigned long long>(need));
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    return fail(MVLLM_ERR_INVALID, "%s: the workspace must be 256-byte aligned", name);
  }
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  mvllm::PagedParams p{};
  p.out = out;
  p.k_pool = key_pool;
  p.v_pool = value_pool;
  p.block_tables = block_tables;
  p.cu_seqlens_q = cu_seqlens_q;
  p.context_lens = context_lens;
  p.seq_lens = seq_lens;
  p.num_seqs = num_seqs;
  p.num_tokens = num_seqs;
  p.hq = num_q_heads;
  p.hk = num_kv_heads;
  p.max_blocks = max_blocks_per_seq;
  p.block_shift = shift;
  p.block_mask = block_size - 1;
  p.table_shift = shift;
  p.kv_head_bytes = static_cast<int64_t>(head_dim) * 2;
  p.kv_row_bytes = p.kv_head_bytes * num_kv_heads;
  p.scale = scale;
  p.stream_wgs = plan.pub.decode_workgroups;
  char* ws = static_cast<char*>(workspace);
  p.seq_prefix = reinterpret_cast<int*>(ws);
  p.part_o = reinterpret_cast<float*>(ws + plan.off_o);
  p.part_ml = reinterpret_cast<float*>(ws + plan.off_ml);
  mvllm::FreshParams f{};
  f.q = q;
  f.k = k;
  f.v = v;
  f.q_stride = qs;
  f.kv_stride = kvs;
  f.q_weight = q_weight;
  f.k_weight = k_weight;
  f.cos_t = cos_table;
  f.sin_t = sin_table;
  f.max_positions = max_positions;
  f.num_blocks = num_blocks;
  f.eps = eps;
  return hip_status(mvllm::launch_paged_decode_fresh(p, f, dtype, head_dim,
                                                     static_cast<hipStream_t>(stream)),
                    name);
}

int mvllm_dense_attention_plan(const mvllm_dense_args* args, uint64_t* workspace_bytes) {
  g_error[0] = '\0';
  if (workspace_bytes == nullptr) {
    return fail(MVLLM_ERR_INVALID, "dense_attention_plan: workspace_bytes is NULL");
  }
  DensePlan d;
  const int rc = dense_plan(args, d);
  if (rc != MVLLM_OK) return rc;
  *workspace_bytes = d.bytes;
  return MVLLM_OK;
}

int mvllm_dense_attention(const mvllm_dense_args* args, void* workspace, uint64_t workspace_bytes,
                          void* stream) {
  g_error[0] = '\0';
  DensePlan d;
  int rc = dense_plan(args, d);
  if (rc != MVLLM_OK) return rc;
  const char* name = args->query_len == 1 ? "decode_attention" : "flash_prefill";
  if (args->batch == 0) return MVLLM_OK;
  if (args->out == nullptr || args->q == nullptr || args->k == nullptr || args->v == nullptr) {
    return fail(MVLLM_ERR_INVALID, "%s: a required pointer is NULL", name);
  }
  if (workspace == nullptr || workspace_bytes < d.bytes) {
    return fail(MVLLM_ERR_WORKSPACE,
                "%s: workspace of %llu bytes is smaller than the %llu the call needs (call "
                "mvllm_dense_attention_plan)",
                name, static_cast<unsigned long long>(workspace_bytes),
                static_cast<unsigned long long>(d.bytes));
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    return fail(MVLLM_ERR_INVALID, "%s: the workspace must be 256-byte aligned", name);
  }
  char* ws = static_cast<char*>(workspace);
  mvllm::DenseMeta meta{};
  meta.block_tables = reinterpret_cast<int32_t*>(ws + d.off_tables);
  meta.cu_seqlens_q = reinterpret_cast<int32_t*>(ws + d.off_cu);
  meta.context_lens = reinterpret_cast<int32_t*>(ws + d.off_ctx);
  meta.seq_lens = reinterpret_cast<int32_t*>(ws + d.off_len);
  meta.batch = args->batch;
  meta.max_blocks = d.max_blocks;
  meta.slots_per_batch = d.slots_per_batch;
  meta.query_len = args->query_len;
  meta.kv_len = args->kv_len;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  rc = hip_status(mvllm::launch_dense_meta(meta, s), name);
  if (rc != MVLLM_OK) return rc;

  const int esize = args->dtype == mvllm::kF32 ? 4 : 2;
  mvllm::PagedParams p{};
  p.q = args->q;
  p.k_pool = args->k;
  p.v_pool = args->v;
  p.out = args->out;
  p.block_tables = meta.block_tables;
  p.cu_seqlens_q = meta.cu_seqlens_q;
  p.context_lens = meta.context_lens;
  p.seq_lens = meta.seq_lens;
  p.num_seqs = args->batch;
  p.num_tokens = args->batch * args->query_len;
  p.hq = args->num_q_heads;
  p.hk = args->num_kv_heads;
  p.max_blocks = d.max_blocks;
  p.block_shift = 4;
  p.block_mask = 15;
  p.table_shift = 0;
  p.kv_row_bytes = args->k_stride_pos * esize;
  p.kv_head_bytes = args->k_stride_head * esize;
  p.scale = args->scale;
  return launch_planned(d.plan, p, ws + d.off_paged, args->dtype, args->dtype, args->head_dim,
                        args->query_len, s, name);
}

uint64_t mvllm_argmax_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows < 1 || vocab < 1) return 0;
  return mvllm::argmax_workspace_bytes(rows, vocab);
}

int mvllm_argmax(int64_t* out, const void* logits, int64_t rows, int64_t vocab,
                 int64_t row_stride, int32_t dtype, void* workspace, uint64_t workspace_bytes,
                 void* stream) {
  g_error[0] = '\0';
  if (dtype != mvllm::kF32 && dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_UNSUPPORTED, "argmax: dtype code %d is not served (f32, f16, bf16)", dtype);
  }
  if (rows < 0 || rows >= (int64_t{1} << 31) || vocab <= 0 || vocab > mvllm::argmax_max_vocab() ||
      row_stride < vocab) {
    return fail(MVLLM_ERR_INVALID,
                "argmax: %lld rows of %lld logits, %lld apart: rows must be < 2^31, the row "
                "non-empty and at most %lld long, the stride at least the row",
                static_cast<long long>(rows), static_cast<long long>(vocab),
                static_cast<long long>(row_stride),
                static_cast<long long>(mvllm::argmax_max_vocab()));
  }
  if (rows == 0) return MVLLM_OK;
  if (out == nullptr || logits == nullptr) {
    return fail(MVLLM_ERR_INVALID, "argmax: a required pointer is NULL");
  }
  const uint64_t need = mvllm::argmax_workspace_bytes(rows, vocab);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need ||
                   reinterpret_cast<uintptr_t>(workspace) % 8 != 0)) {
    return fail(MVLLM_ERR_WORKSPACE,
                "argmax: needs %llu bytes of 8-byte aligned workspace "
                "(mvllm_argmax_workspace_bytes), got %llu",
                static_cast<unsigned long long>(need), static_cast<unsigned long long>(workspace_bytes));
  }
  return hip_status(mvllm::launch_argmax(out, logits, rows, vocab, row_stride, dtype, workspace,
                                         static_cast<hipStream_t>(stream)),
                    "argmax: launch");
}

int mvllm_rmsnorm(void* out, const void* x, const void* weight, int64_t rows, int64_t dim,
                  float eps, int32_t dtype, void* stream) {
  g_error[0] = '\0';
  if (dtype != mvllm::kF32 && dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "rmsnorm: dtype code %d is not supported; float64 is not supported, this kernel "
                "accumulates in fp32",
                dtype);
  }
  if (rows < 0 || dim < 0 || dim > (1 << 30)) return fail(MVLLM_ERR_INVALID, "rmsnorm: bad shape");
  if (rows == 0 || dim == 0) return MVLLM_OK;
  if (out == nullptr || x == nullptr || weight == nullptr) {
    return fail(MVLLM_ERR_INVALID, "rmsnorm: a required pointer is NULL");
  }
  return hip_status(mvllm::launch_rmsnorm(x, weight, out, rows, static_cast<int>(dim), eps, dtype,
                                          static_cast<hipStream_t>(stream)),
                    "rmsnorm: launch");
}

int mvllm_rope(void* out, const void* x, const void* positions, int32_t positions_bytes,
               const float* cos_table, const float* sin_table, int64_t rows, int64_t heads,
               int64_t head_dim, int64_t num_positions, int64_t max_positions, int32_t dtype,
               void* stream) {
  g_error[0] = '\0';
  if (dtype != mvllm::kF32 && dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "rope: dtype code %d is not supported; float64 is not supported, this kernel "
                "computes the rotation in fp32",
                dtype);
  }
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > (1 << 20)) {
    return fail(MVLLM_ERR_INVALID, "rope: the head dimension must be even, got %lld",
                static_cast<long long>(head_dim));
  }
  if (positions_bytes != 4 && positions_bytes != 8) {
    return fail(MVLLM_ERR_INVALID, "rope: positions must be int32 or int64");
  }
  if (rows < 0 || heads <= 0 || rows % heads != 0) {
    return fail(MVLLM_ERR_INVALID, "rope: rows (%lld) must be tokens x heads (%lld)",
                static_cast<long long>(rows), static_cast<long long>(heads));
  }
  if (rows == 0) return MVLLM_OK;
  if (num_positions <= 0) return fail(MVLLM_ERR_INVALID, "rope: positions is empty");
  if ((rows / heads) % num_positions != 0) {
    return fail(MVLLM_ERR_INVALID,
                "rope: x holds %lld tokens, which is not a multiple of the %lld positions given, "
                "so the positions cannot broadcast over it",
                static_cast<long long>(rows / heads), static_cast<long long>(num_positions));
  }
  if (max_positions <= 0) return fail(MVLLM_ERR_INVALID, "rope: empty cos/sin tables");
  if (out == nullptr || x == nullptr || positions == nullptr || cos_table == nullptr ||
      sin_table == nullptr) {
    return fail(MVLLM_ERR_INVALID, "rope: a required pointer is NULL");
  }
  return hip_status(mvllm::launch_rope(x, positions, positions_bytes, cos_table, sin_table, out,
                                       rows, heads, static_cast<int>(head_dim), num_positions,
                                       max_positions, dtype, static_cast<hipStream_t>(stream)),
                    "rope: launch");
}

int mvllm_qk_norm_rope(void* q_out, void* k_out, const void* q, const void* k,
                       const void* q_weight, const void* k_weight, const void* positions,
                       int32_t positions_bytes, const float* cos_table, const float* sin_table,
                       int64_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, int64_t num_positions, int64_t max_positions, float eps,
                       int32_t dtype, void* stream) {
  g_error[0] = '\0';
  return qk_norm_rope_entry(q_out, k_out, q, k, q_weight, k_weight, positions, positions_bytes,
                            cos_table, sin_table, num_tokens, num_q_heads, num_kv_heads, head_dim,
                            num_positions, max_positions, eps, dtype, stream, nullptr, nullptr,
                            nullptr, nullptr, 0);
}

int mvllm_qk_norm_rope_kv_write(void* q_out, void* key_pool, void* value_pool, const void* q,
                                const void* k, const void* v, const void* q_weight,
                                const void* k_weight, const void* positions,
                                int32_t positions_bytes, const float* cos_table,
                                const float* sin_table, const int32_t* slot_mapping,
                                int64_t num_slots, int64_t num_tokens, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int64_t num_positions,
                                int64_t max_positions, float eps, int64_t q_token_stride,
                                int64_t kv_token_stride, int32_t dtype, void* stream) {
  g_error[0] = '\0';
  if (num_slots < 0) return fail(MVLLM_ERR_INVALID, "qk_norm_rope_kv_write: negative num_slots");
  if (num_tokens > 0 && (key_pool == nullptr || value_pool == nullptr || v == nullptr ||
                         slot_mapping == nullptr)) {
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope_kv_write: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(key_pool) | reinterpret_cast<uintptr_t>(value_pool) |
       reinterpret_cast<uintptr_t>(v)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope_kv_write: every tensor must be 16-byte aligned");
  }
  return qk_norm_rope_entry(q_out, nullptr, q, k, q_weight, k_weight, positions, positions_bytes,
                            cos_table, sin_table, num_tokens, num_q_heads, num_kv_heads, head_dim,
                            num_positions, max_positions, eps, dtype, stream, v, key_pool,
                            value_pool, slot_mapping, num_slots, q_token_stride, kv_token_stride);
}

int mvllm_swiglu(void* out, const void* gate, const void* up, int64_t n, int32_t dtype,
                 void* stream) {
  g_error[0] = '\0';
  if (dtype != mvllm::kF32 && dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "swiglu: dtype code %d is not supported; float64 is not supported, this kernel "
                "evaluates the sigmoid in fp32",
                dtype);
  }
  if (n < 0) return fail(MVLLM_ERR_INVALID, "swiglu: negative size");
  if (n == 0) return MVLLM_OK;
  if (out == nullptr || gate == nullptr || up == nullptr) {
    return fail(MVLLM_ERR_INVALID, "swiglu: a required pointer is NULL");
  }
  return hip_status(
      mvllm::launch_swiglu(gate, up, out, n, dtype, static_cast<hipStream_t>(stream)),
      "swiglu: launch");
}

int mvllm_add_rmsnorm(void* h_out, void* out, const void* x, const void* residual,
                      const void* weight, int64_t rows, int32_t dim, float eps, int32_t dtype,
                      void* stream) {
  g_error[0] = '\0';
  if (!mvllm::add_rmsnorm_supported(dtype, dim)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "add_rmsnorm: dtype code %d with dim %d is not served (f32/f16/bf16, dim a "
                "multiple of one 16-byte chunk, at most 512 chunks); add then call rmsnorm",
                dtype, dim);
  }
  if (rows < 0) return fail(MVLLM_ERR_INVALID, "add_rmsnorm: negative row count");
  if (rows == 0) return MVLLM_OK;
  if (h_out == nullptr || out == nullptr || x == nullptr || residual == nullptr ||
      weight == nullptr) {
    return fail(MVLLM_ERR_INVALID, "add_rmsnorm: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(h_out) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) |
       reinterpret_cast<uintptr_t>(weight)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "add_rmsnorm: every tensor must be 16-byte aligned");
  }
  return hip_status(mvllm::launch_add_rmsnorm(x, residual, weight, h_out, out, rows, dim, eps,
                                              dtype, static_cast<hipStream_t>(stream)),
                    "add_rmsnorm: launch");
}

int mvllm_embed_rmsnorm(void* h_out, void* out, const void* table, int64_t vocab,
                        const int64_t* ids, const int64_t* index, const int64_t* prev,
                        int64_t rows, int32_t dim, const void* weight, float eps, int32_t dtype,
                        void* stream) {
  g_error[0] = '\0';
  if (!mvllm::add_rmsnorm_supported(dtype, dim)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "embed_rmsnorm: dtype code %d with dim %d is not served (f32/f16/bf16, dim a "
                "multiple of one 16-byte chunk, at most 512 chunks); look the rows up, then "
                "call rmsnorm",
                dtype, dim);
  }
  if (rows < 0 || vocab <= 0) return fail(MVLLM_ERR_INVALID, "embed_rmsnorm: bad row or vocab count");
  if (rows == 0) return MVLLM_OK;
  if (h_out == nullptr || out == nullptr || table == nullptr || ids == nullptr ||
      weight == nullptr || (index != nullptr && prev == nullptr)) {
    return fail(MVLLM_ERR_INVALID, "embed_rmsnorm: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(h_out) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(weight)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "embed_rmsnorm: the table, weight and outputs must be 16-byte aligned");
  }
  return hip_status(mvllm::launch_embed_rmsnorm(table, vocab, ids, index, prev, weight, h_out, out,
                                                rows, dim, eps, dtype,
                                                static_cast<hipStream_t>(stream)),
                    "embed_rmsnorm: launch");
}

int mvllm_swiglu_interleaved(void* out, const void* gate_up, int64_t rows, int64_t cols,
                             int32_t dtype, void* stream) {
  g_error[0] = '\0';
  if (dtype != mvllm::kF32 && dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "swiglu_interleaved: dtype code %d is not supported; float64 is not supported",
                dtype);
  }
  if (rows < 0 || cols < 0 || cols % 16 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "swiglu_interleaved: cols (%lld) must be a multiple of 16 (the interleave's "
                "group) and rows non-negative",
                static_cast<long long>(cols));
  }
  if (rows == 0 || cols == 0) return MVLLM_OK;
  if (out == nullptr || gate_up == nullptr) {
    return fail(MVLLM_ERR_INVALID, "swiglu_interleaved: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gate_up)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "swiglu_interleaved: every tensor must be 16-byte aligned");
  }
  return hip_status(mvllm::launch_swiglu_interleaved(gate_up, out, rows, cols, dtype,
                                                     static_cast<hipStream_t>(stream)),
                    "swiglu_interleaved: launch");
}

// Shared checks of the skinny projection entries: dtype, sizes, pointers, alignment.
int check_linear(const char* name, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                 int32_t dtype) {
  if (dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: dtype code %d is not served; the skinny kernel takes fp16 or bf16", name,
                dtype);
  }
  if (m < 0 || n < 0 || k < 0) return fail(MVLLM_ERR_INVALID, "%s: negative size", name);
  if (x == nullptr || w == nullptr) return fail(MVLLM_ERR_INVALID, "%s: a required pointer is NULL", name);
  if (!mvllm::skinny_linear_supported(dtype, m, n, k)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "%s: shape M=%lld N=%lld K=%lld is not served; the skinny kernel takes at most "
                "%lld rows and K a multiple of 64 up to %lld",
                name, static_cast<long long>(m), static_cast<long long>(n), static_cast<long long>(k),
                static_cast<long long>(mvllm::kSkinnyMaxRows),
                static_cast<long long>(mvllm::kSkinnyMaxK));
  }
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "%s: x and w must be 16-byte aligned", name);
  }
  return MVLLM_OK;
}

// The partial-sum workspace a skinny projection with K > 1024 needs, checked against
// what the caller gave.
int check_linear_workspace(const char* name, int64_t m, int64_t n, int64_t k, const void* workspace,
                           uint64_t workspace_bytes) {
  const uint64_t need = mvllm::skinny_linear_workspace_bytes(m, n, k);
  if (need == 0) return MVLLM_OK;
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(MVLLM_ERR_WORKSPACE,
                "%s: workspace of %llu bytes is smaller than the %llu this shape needs "
                "(mvllm_linear_workspace_bytes)",
                name, static_cast<unsigned long long>(workspace_bytes),
                static_cast<unsigned long long>(need));
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    return fail(MVLLM_ERR_INVALID, "%s: the workspace must be 256-byte aligned", name);
  }
  return MVLLM_OK;
}

uint64_t mvllm_linear_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m < 1 || n < 1 || k < 64) return 0;
  return mvllm::skinny_linear_workspace_bytes(m, n, k);
}

int mvllm_linear_pack(void* w_packed, const void* w, int64_t n, int64_t k, int32_t dtype,
                      void* stream) {
  g_error[0] = '\0';
  if (dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_UNSUPPORTED, "linear_pack: dtype code %d is not served (fp16 or bf16)",
                dtype);
  }
  if (n < 0 || k < 0) return fail(MVLLM_ERR_INVALID, "linear_pack: negative size");
  if (n == 0) return MVLLM_OK;
  if (!mvllm::skinny_linear_supported(dtype, 1, n, k)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "linear_pack: N=%lld K=%lld is not served; K must be a multiple of 64 up to %lld",
                static_cast<long long>(n), static_cast<long long>(k),
                static_cast<long long>(mvllm::kSkinnyMaxK));
  }
  if (w_packed == nullptr || w == nullptr) {
    return fail(MVLLM_ERR_INVALID, "linear_pack: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(w_packed) | reinterpret_cast<uintptr_t>(w)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "linear_pack: both buffers must be 16-byte aligned");
  }
  return hip_status(mvllm::launch_skinny_linear_pack(w_packed, w, n, k, static_cast<hipStream_t>(stream)),
                    "linear_pack: launch");
}

int mvllm_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                 int32_t dtype, void* workspace, uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  if (m == 0 || n == 0) return MVLLM_OK;
  int rc = check_linear("linear", x, w, m, n, k, dtype);
  if (rc != MVLLM_OK) return rc;
  if (y == nullptr) return fail(MVLLM_ERR_INVALID, "linear: a required pointer is NULL");
  rc = check_linear_workspace("linear", m, n, k, workspace, workspace_bytes);
  if (rc != MVLLM_OK) return rc;
  return hip_status(
      mvllm::launch_skinny_linear(y, x, w, m, n, k, dtype, workspace, static_cast<hipStream_t>(stream)),
                    "linear: launch");
}

int mvllm_linear_split(void* y0, void* y1, void* y2, const void* x, const void* w, int64_t m,
                       int64_t n0, int64_t n1, int64_t n2, int64_t k, int32_t dtype,
                       void* workspace, uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  if (n0 < 0 || n1 < 0 || n2 < 0) return fail(MVLLM_ERR_INVALID, "linear_split: negative size");
  if (n0 % 32 != 0 || n1 % 32 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "linear_split: the first two column groups (%lld, %lld) must be multiples of 32",
                static_cast<long long>(n0), static_cast<long long>(n1));
  }
  const int64_t n = n0 + n1 + n2;
  if (m == 0 || n == 0) return MVLLM_OK;
  int rc = check_linear("linear_split", x, w, m, n, k, dtype);
  if (rc != MVLLM_OK) return rc;
  if ((n0 > 0 && y0 == nullptr) || (n1 > 0 && y1 == nullptr) || (n2 > 0 && y2 == nullptr)) {
    return fail(MVLLM_ERR_INVALID, "linear_split: an output of a non-empty column group is NULL");
  }
  rc = check_linear_workspace("linear_split", m, n, k, workspace, workspace_bytes);
  if (rc != MVLLM_OK) return rc;
  return hip_status(mvllm::launch_skinny_linear_split(y0, y1, y2, x, w, m, n0, n1, n2, k, dtype,
                                                      workspace, static_cast<hipStream_t>(stream)),
                    "linear_split: launch");
}

int mvllm_linear_residual(void* y, const void* x, const void* w, const void* residual, int64_t m,
                          int64_t n, int64_t k, int32_t dtype, void* workspace,
                          uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  if (m == 0 || n == 0) return MVLLM_OK;
  int rc = check_linear("linear_residual", x, w, m, n, k, dtype);
  if (rc != MVLLM_OK) return rc;
  if (y == nullptr || residual == nullptr) {
    return fail(MVLLM_ERR_INVALID, "linear_residual: a required pointer is NULL");
  }
  rc = check_linear_workspace("linear_residual", m, n, k, workspace, workspace_bytes);
  if (rc != MVLLM_OK) return rc;
  return hip_status(mvllm::launch_skinny_linear_residual(y, x, w, residual, m, n, k, dtype, workspace,
                                                         static_cast<hipStream_t>(stream)),
                    "linear_residual: launch");
}

int mvllm_linear_swiglu(void* y, const void* x, const void* w_gate_up, int64_t m, int64_t n_out,
                        int64_t k, int32_t dtype, void* workspace, uint64_t workspace_bytes,
                        void* stream) {
  g_error[0] = '\0';
  if (n_out < 0) return fail(MVLLM_ERR_INVALID, "linear_swiglu: negative size");
  if (n_out % 16 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "linear_swiglu: %lld output columns; the gate/up interleave needs a multiple of 16",
                static_cast<long long>(n_out));
  }
  if (m == 0 || n_out == 0) return MVLLM_OK;
  int rc = check_linear("linear_swiglu", x, w_gate_up, m, 2 * n_out, k, dtype);
  if (rc != MVLLM_OK) return rc;
  if (y == nullptr) return fail(MVLLM_ERR_INVALID, "linear_swiglu: a required pointer is NULL");
  rc = check_linear_workspace("linear_swiglu", m, 2 * n_out, k, workspace, workspace_bytes);
  if (rc != MVLLM_OK) return rc;
  return hip_status(mvllm::launch_skinny_linear_swiglu(y, x, w_gate_up, m, n_out, k, dtype, workspace,
                                                       static_cast<hipStream_t>(stream)),
                    "linear_swiglu: launch");
}

int mvllm_linear_residual_rmsnorm(void* h_out, void* normed, const void* x, const void* w,
                                  const void* residual, const void* norm_weight, int64_t m,
                                  int64_t n, int64_t k, float eps, int32_t dtype, void* workspace,
                                  uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  if (m == 0 || n == 0) return MVLLM_OK;
  int rc = check_linear("linear_residual_rmsnorm", x, w, m, n, k, dtype);
  if (rc != MVLLM_OK) return rc;
  if (!mvllm::skinny_residual_rmsnorm_supported(dtype, m, n, k)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "linear_residual_rmsnorm: N=%lld K=%lld is not served; the fused norm takes K > "
                "1024 and N a multiple of 512 up to 4096",
                static_cast<long long>(n), static_cast<long long>(k));
  }
  if (h_out == nullptr || normed == nullptr || residual == nullptr || norm_weight == nullptr) {
    return fail(MVLLM_ERR_INVALID, "linear_residual_rmsnorm: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(h_out) | reinterpret_cast<uintptr_t>(normed) |
       reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(norm_weight)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "linear_residual_rmsnorm: every buffer must be 16-byte aligned");
  }
  rc = check_linear_workspace("linear_residual_rmsnorm", m, n, k, workspace, workspace_bytes);
  if (rc != MVLLM_OK) return rc;
  return hip_status(mvllm::launch_skinny_linear_residual_rmsnorm(
                        h_out, normed, x, w, residual, norm_weight, m, n, k, eps, dtype, workspace,
                        static_cast<hipStream_t>(stream)),
                    "linear_residual_rmsnorm: launch");
}

uint64_t mvllm_blas_workspace_bytes(void) { return mvllm::kBlasWorkspaceBytes; }

int mvllm_blas_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                      int32_t dtype, void* workspace, uint64_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  if (m < 0 || n < 0 || k < 0) return fail(MVLLM_ERR_INVALID, "blas_linear: negative size");
  if (m == 0 || n == 0) return MVLLM_OK;
  if (k == 0) return fail(MVLLM_ERR_UNSUPPORTED, "blas_linear: k = 0 is not served");
  if (dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_UNSUPPORTED, "blas_linear: dtype code %d is not served; fp16 or bf16",
                dtype);
  }
  if (x == nullptr || w == nullptr || y == nullptr) {
    return fail(MVLLM_ERR_INVALID, "blas_linear: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
       reinterpret_cast<uintptr_t>(y)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "blas_linear: x, w and y must be 16-byte aligned");
  }
  if (workspace == nullptr || workspace_bytes < mvllm::kBlasWorkspaceBytes ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "blas_linear: the workspace must be 256-byte aligned and hold %llu bytes "
                "(mvllm_blas_workspace_bytes), got %llu",
                static_cast<unsigned long long>(mvllm::kBlasWorkspaceBytes),
                static_cast<unsigned long long>(workspace_bytes));
  }
  const mvllm::BlasStatus st = mvllm::blas_linear(y, x, w, m, n, k, dtype, workspace,
                                                  static_cast<hipStream_t>(stream));
  switch (st.kind) {
    case 0:
      return MVLLM_OK;
    case 1:
      return fail(MVLLM_ERR_HIP, "blas_linear: %s: HIP error %d (%s)", st.what, st.code,
                  hipGetErrorString(static_cast<hipError_t>(st.code)));
    case 3:
      return fail(MVLLM_ERR_UNSUPPORTED, "blas_linear: M=%lld N=%lld K=%lld: %s",
                  static_cast<long long>(m), static_cast<long long>(n),
                  static_cast<long long>(k), st.what);
    default:
      return fail(MVLLM_ERR_HIP, "blas_linear: hipBLASLt %s failed with status %d", st.what,
                  st.code);
  }
}

int mvllm_blas_plans_cached(void) { return mvllm::blas_plans_cached(); }

int mvllm_blas_tune(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    int32_t dtype, void* workspace, uint64_t workspace_bytes, void* stream,
                    int32_t* timed) {
  g_error[0] = '\0';
  if (timed != nullptr) *timed = 0;
  if (m <= 0 || n <= 0 || k <= 0) return fail(MVLLM_ERR_INVALID, "blas_tune: sizes must be positive");
  if (dtype != mvllm::kF16 && dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_UNSUPPORTED, "blas_tune: dtype code %d is not served; fp16 or bf16",
                dtype);
  }
  if (x == nullptr || w == nullptr || y == nullptr) {
    return fail(MVLLM_ERR_INVALID, "blas_tune: a required pointer is NULL");
  }
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
       reinterpret_cast<uintptr_t>(y)) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "blas_tune: x, w and y must be 16-byte aligned");
  }
  if (workspace == nullptr || workspace_bytes < mvllm::kBlasWorkspaceBytes ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0) {
    return fail(MVLLM_ERR_INVALID,
                "blas_tune: the workspace must be 256-byte aligned and hold %llu bytes "
                "(mvllm_blas_workspace_bytes), got %llu",
                static_cast<unsigned long long>(mvllm::kBlasWorkspaceBytes),
                static_cast<unsigned long long>(workspace_bytes));
  }
  int count = 0;
  const mvllm::BlasStatus st = mvllm::blas_tune(y, x, w, m, n, k, dtype, workspace,
                                                static_cast<hipStream_t>(stream), count);
  if (timed != nullptr) *timed = count;
  switch (st.kind) {
    case 0:
      return MVLLM_OK;
    case 1:
      return fail(MVLLM_ERR_HIP, "blas_tune: %s: HIP error %d (%s)", st.what, st.code,
                  hipGetErrorString(static_cast<hipError_t>(st.code)));
    case 3:
    case 4:
      return fail(MVLLM_ERR_UNSUPPORTED, "blas_tune: M=%lld N=%lld K=%lld: %s",
                  static_cast<long long>(m), static_cast<long long>(n),
                  static_cast<long long>(k), st.what);
    default:
      return fail(MVLLM_ERR_HIP, "blas_tune: hipBLASLt %s failed with status %d", st.what,
                  st.code);
  }
}

int mvllm_blas_tuning(int64_t m, int64_t n, int64_t k, int32_t dtype, mvllm_blas_choice* out) {
  g_error[0] = '\0';
  if (out == nullptr) return fail(MVLLM_ERR_INVALID, "blas_tuning: out is NULL");
  mvllm::BlasTuning t;
  if (!mvllm::blas_tuning(m, n, k, dtype, t)) {
    return fail(MVLLM_ERR_INVALID, "blas_tuning: M=%lld N=%lld K=%lld dtype %d was not called",
                static_cast<long long>(m), static_cast<long long>(n), static_cast<long long>(k),
                dtype);
  }
  out->candidates = t.candidates;
  out->timed = t.timed;
  out->chosen = t.chosen;
  out->first_us = t.first_us;
  out->chosen_us = t.chosen_us;
  return MVLLM_OK;
}

int mvllm_kv_write(void* key_pool, void* value_pool, float* k_scales, float* v_scales,
                   const void* key, const void* value, const int32_t* slot_mapping,
                   int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                   int32_t block_size, int64_t num_blocks, int32_t src_dtype,
                   int32_t pool_dtype, void* stream) {
  g_error[0] = '\0';
  if (src_dtype != mvllm::kF32 && src_dtype != mvllm::kF16 && src_dtype != mvllm::kBF16) {
    return fail(MVLLM_ERR_INVALID,
                "kv_write: key/value dtype code %d is not supported; float64 is not supported",
                src_dtype);
  }
  if (!mvllm::kv_write_supported(src_dtype, pool_dtype, head_dim)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "kv_write: a pool of dtype code %d cannot take keys of dtype code %d at head dim "
                "%d; the pool must share the keys' dtype or be float8_e4m3fn (head dim 32, 64, "
                "128 or 256)",
                pool_dtype, src_dtype, head_dim);
  }
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0) {
    return fail(MVLLM_ERR_INVALID, "kv_write: bad shape");
  }
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) {
    return fail(MVLLM_ERR_INVALID, "kv_write: block size %d is not a power of two", block_size);
  }
  if (num_blocks * block_size >= (int64_t{1} << 31)) {
    return fail(MVLLM_ERR_INVALID, "kv_write: more slots than int32 slot_mapping addresses");
  }
  if (num_tokens == 0) return MVLLM_OK;
  if (key_pool == nullptr || value_pool == nullptr || key == nullptr || value == nullptr ||
      slot_mapping == nullptr) {
    return fail(MVLLM_ERR_INVALID, "kv_write: a required pointer is NULL");
  }
  const bool fp8 = pool_dtype == mvllm::kFP8E4M3;
  if (fp8 != (k_scales != nullptr && v_scales != nullptr) || (!fp8 && (k_scales || v_scales))) {
    return fail(MVLLM_ERR_INVALID,
                "kv_write: k_scales and v_scales are required for a float8 pool and only for one");
  }
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  return hip_status(mvllm::launch_kv_write(key_pool, value_pool, k_scales, v_scales, key, value,
                                           slot_mapping, num_tokens, num_kv_heads, head_dim,
                                           shift, num_blocks, src_dtype, pool_dtype,
                                           static_cast<hipStream_t>(stream)),
                    "kv_write: launch");
}

int mvllm_read_probe(const void* base, int64_t base_bytes, const int32_t* page_ids,
                     int64_t num_pages, int64_t page_bytes, int32_t workgroups, uint32_t* sink,
                     int64_t sink_words, void* stream) {
  g_error[0] = '\0';
  if (base == nullptr || sink == nullptr) return fail(MVLLM_ERR_INVALID, "read_probe: NULL buffer");
  if (!mvllm::read_probe_supported(page_bytes)) {
    return fail(MVLLM_ERR_UNSUPPORTED,
                "read_probe: page_bytes %lld is not served (4, 8, 16, 32 or 64 KB)",
                static_cast<long long>(page_bytes));
  }
  if (num_pages < 0 || base_bytes < 0 || workgroups <= 0 || workgroups > 65536) {
    return fail(MVLLM_ERR_INVALID, "read_probe: bad page count or workgroups");
  }
  if (base_bytes / page_bytes < (page_ids == nullptr ? num_pages : 1)) {
    return fail(MVLLM_ERR_INVALID, "read_probe: the base buffer holds fewer pages than read");
  }
  if (sink_words < mvllm::read_probe_sink_words(workgroups)) {
    return fail(MVLLM_ERR_INVALID, "read_probe: the sink must hold %d words",
                mvllm::read_probe_sink_words(workgroups));
  }
  if (reinterpret_cast<uintptr_t>(base) % 16 != 0) {
    return fail(MVLLM_ERR_INVALID, "read_probe: base must be 16-byte aligned");
  }
  if (num_pages == 0) return MVLLM_OK;
  return hip_status(mvllm::launch_read_probe(base, page_ids, num_pages, page_bytes, workgroups,
                                             sink, static_cast<hipStream_t>(stream)),
                    "read_probe: launch");
}

int mvllm_axpby(float* y, const float* x, float a, float b, int64_t n, void* stream) {
  g_error[0] = '\0';
  if (n < 0) return fail(MVLLM_ERR_INVALID, "axpby: negative size");
  if (n == 0) return MVLLM_OK;
  if (x == nullptr || y == nullptr) return fail(MVLLM_ERR_INVALID, "axpby: NULL pointer");
  return hip_status(mvllm::launch_axpby(x, y, a, b, n, static_cast<hipStream_t>(stream)),
                    "axpby: launch");
}

}  // extern "C"
