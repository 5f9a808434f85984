// Paged KV write: scatter one iteration's keys and values into their pool slots.
//
// Replaces the two index_copy_ calls of the reference's PagedKvPool.write
// (block/kv_pool.py:116-155): key/value [T, H_k, D] rows go to pool slot
// slot_mapping[t] of the flat [num_blocks * P, H_k, D] view, for K and V in one launch.
// A negative slot skips its token (padding rows of a captured decode graph).
//
// Same storage type: a copy, one thread per 16-byte chunk of K or V.
//
// fp8-e4m3 pools (no counterpart in the reference) carry one fp32 scale per (block, kv
// head) for K and for V: stored code = e4m3(x / scale), read as code * scale. Writes
// arrive a few tokens at a time, so the scale of a page grows as it fills. Scales are
// powers of two, so re-encoding the rows already in a page under a grown scale only
// shifts their exponents (exact, except where a value drops into e4m3's subnormals):
//   * a run = consecutive tokens of this call that land on consecutive rows of one page
//     (a page belongs to one sequence, whose new tokens are consecutive on the token
//     axis and in the page, so a page gets one run per call: callers must keep it so);
//     one wave per run;
//   * a run that starts at offset 0 opens the page: the old scale and rows are dead;
//   * new scale s = max(old scale, pow2ceil(max|x| / 448)) over the run's rows (0 when
//     all are 0), pow2ceil = the least power of two >= its argument;
//   * if s grew, the rows already in the page are re-encoded: e4m3((code * old) / s);
//   * the run's rows are encoded as e4m3(clamp(x / s, -448, 448)), RNE (0 when s = 0).
// Every step is an fp32 multiply / divide with one rounding, so the CPU restatement
// (oracle/kv_write.py) reproduces the bytes exactly; since scales are powers of two the
// kernel divides by multiplying with the exact reciprocal, which gives the same results.

#include <algorithm>

#include "common.hpp"
#include "kv_write.hpp"
#include "paged_attention.hpp"

namespace mvllm {

namespace {

// --------------------------------------------------------------------- copy

__global__ __launch_bounds__(256) void kv_copy_kernel(void* __restrict__ k_pool,
                                                      void* __restrict__ v_pool,
                                                      const void* __restrict__ key,
                                                      const void* __restrict__ value,
                                                      const int32_t* __restrict__ slots,
                                                      int64_t chunks_per_token, int64_t total,
                                                      int64_t num_slots) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= 2 * total) return;
  const bool is_v = i >= total;
  const int64_t j = is_v ? i - total : i;
  const int64_t t = j / chunks_per_token;
  const int64_t c = j - t * chunks_per_token;
  const int32_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const char* src = static_cast<const char*>(is_v ? value : key) + j * 16;
  char* dst = static_cast<char*>(is_v ? v_pool : k_pool) +
              (static_cast<int64_t>(slot) * chunks_per_token + c) * 16;
  store16(dst, nt_load16(src));
}

// Scalar fallback for row sizes that are not a multiple of 16 bytes.
template <typename T>
__global__ __launch_bounds__(256) void kv_copy_scalar_kernel(void* __restrict__ k_pool,
                                                             void* __restrict__ v_pool,
                                                             const void* __restrict__ key,
                                                             const void* __restrict__ value,
                                                             const int32_t* __restrict__ slots,
                                                             int64_t row, int64_t total,
                                                             int64_t num_slots) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= 2 * total) return;
  const bool is_v = i >= total;
  const int64_t j = is_v ? i - total : i;
  const int64_t t = j / row;
  const int32_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  static_cast<T*>(is_v ? v_pool : k_pool)[static_cast<int64_t>(slot) * row + (j - t * row)] =
      static_cast<const T*>(is_v ? value : key)[j];
}

// ---------------------------------------------------------------------- fp8

// Least power of two >= t (t >= 0 finite; 0 stays 0): clear the mantissa and, if it
// was not already clear, step the exponent (a subnormal t gives 2^-126).
__device__ __forceinline__ float pow2_ceil(float t) {
  const uint32_t b = __float_as_uint(t);
  if ((b & 0x7fffffu) == 0) return t;
  return __uint_as_float((b & 0x7f800000u) + 0x800000u);
}

// Four values -> four e4m3 bytes (two packed conversions), each clamped to +-448.
__device__ __forceinline__ uint32_t encode_fp8x4(float a, float b, float c, float d) {
  auto cl = [](float v) { return fminf(fmaxf(v, -448.0f), 448.0f); };
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), lo, true));
}

// One workgroup per `tokens_per_wg` consecutive tokens (at most 64; one for small
// calls, so that decode steps spread over workgroups, up to 64 for large ones, so that
// no workgroup is launched only to find that its token continues a run): a ballot over
// those tokens finds the runs that start among them, and the workgroup writes them one
// after another, each whole. The run's length comes from a ballot over the following
// slots (every wave takes the same ballots). Thread task = (kv head, K or V, 8-element
// piece of a row), kPieces consecutive lanes per (head, K/V), a workgroup's worth of
// tasks at a time (all of them for 8 kv heads at D = 128). Each thread loads its piece
// of up to kRows run rows at once (one round trip), reduces max|x| over them, the
// kPieces lanes of a (head, K/V) combine theirs into the page's scale, rows already in
// the page are re-encoded if it grew, and the rows still in registers are encoded and
// stored. Longer runs (pages of more than kRows tokens) are read kRows rows at a time
// for the scale and read again to encode, except the last batch, still held.
template <typename TS, int D>
__device__ __forceinline__ void kv_write_fp8_run(uint8_t* __restrict__ k_pool,
                                                 uint8_t* __restrict__ v_pool,
                                                 float* __restrict__ k_scales,
                                                 float* __restrict__ v_scales,
                                                 const void* __restrict__ key,
                                                 const void* __restrict__ value,
                                                 const int32_t* __restrict__ slots, int num_tokens,
                                                 int hk, int block_shift, int t0) {
  constexpr int E = 8;            // elements per task piece
  constexpr int kPieces = D / E;  // tasks per (head, K/V)
  constexpr int kChunks = Elem<TS>::kBytes == 4 ? 2 : 1;  // 16-byte loads per row piece
  constexpr int kRows = 16 / kChunks;                     // rows held per task
  static_assert(D % E == 0 && kWave % kPieces == 0, "head dim");
  const int lane = threadIdx.x % kWave;
  const int slot0 = slots[t0];
  const int page = slot0 >> block_shift;
  const int rows_per_page = 1 << block_shift;
  const int off0 = slot0 & (rows_per_page - 1);
  // Run length: the longest stretch of slot0 + i for i < min(rows left in the page,
  // tokens left), 64 candidates per ballot.
  const int limit = min(rows_per_page - off0, num_tokens - t0);
  int len = limit;
  for (int base = 1; base < limit; base += kWave) {
    const int i = base + lane;
    const bool stop = i < limit && slots[t0 + i] != slot0 + i;
    const uint64_t mask = __builtin_amdgcn_ballot_w64(stop);
    if (mask != 0) {
      len = base + __builtin_ctzll(mask);
      break;
    }
  }

  const int ntasks = 2 * hk * kPieces;
  const int64_t src_stride = static_cast<int64_t>(hk) * D * Elem<TS>::kBytes;  // bytes per token
  const int64_t pool_stride = static_cast<int64_t>(hk) * D;                    // bytes per slot
  const int last = (len - 1) / kRows * kRows;  // first row of the last batch
  for (int base = 0; base < ntasks; base += blockDim.x) {
    // A thread past the last task mirrors a valid one (its group of kPieces lanes is
    // all past it): loads stay in bounds and no store is made.
    const int task = base + static_cast<int>(threadIdx.x);
    const bool valid = task < ntasks;
    const int tk = valid ? task : task % ntasks;
    const int pair = tk / kPieces;
    const int piece = (tk % kPieces) * E;
    const bool is_v = pair & 1;
    const int head = pair >> 1;
    const char* src = static_cast<const char*>(is_v ? value : key) +
                      (static_cast<int64_t>(t0) * hk * D + head * D + piece) * Elem<TS>::kBytes;
    uint8_t* pool = (is_v ? v_pool : k_pool) +
                    (static_cast<int64_t>(page) << block_shift) * pool_stride + head * D + piece;
    float* scale_p = (is_v ? v_scales : k_scales) + static_cast<int64_t>(page) * hk + head;
    const float old = off0 > 0 ? *scale_p : 0.0f;

    u32x4 raw[kRows][kChunks];
    auto load_rows = [&](int r0) {
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        const int row = min(r0 + i, len - 1);  // rows past the run repeat its last
#pragma unroll
        for (int c = 0; c < kChunks; ++c) raw[i][c] = load16(src + row * src_stride + 16 * c);
      }
    };
    float amax = 0.0f;
    for (int r0 = 0; r0 < len; r0 += kRows) {
      load_rows(r0);
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        float x[E];
#pragma unroll
        for (int c = 0; c < kChunks; ++c) Chunk<TS>::unpack(raw[i][c], x + c * (E / kChunks));
#pragma unroll
        for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(x[e]));
      }
    }
    const float sc = fmaxf(old, pow2_ceil(group_max<kPieces>(amax) / 448.0f));
    const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;  // exact: a power of two

    // rows already in the page, re-encoded under a grown scale
    if (valid && old > 0.0f && sc > old) {
      for (int row = 0; row < off0; ++row) {
        uint8_t* p = pool + row * pool_stride;
        const u32x2 w = *reinterpret_cast<const u32x2*>(p);
        u32x2 out;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float v[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            // (code * old) / s: every factor a power of two or a 4-bit significand, so
            // the products are exact and equal the correctly rounded quotient
            v[b] = __fmul_rn(__fmul_rn(fp8e4m3_to_f32((w[i] >> (8 * b)) & 0xffu), old), inv);
          }
          out[i] = encode_fp8x4(v[0], v[1], v[2], v[3]);
        }
        *reinterpret_cast<u32x2*>(p) = out;
      }
    }

    // the run's rows, the last batch first (it is still in registers)
    for (int r0 = last; r0 >= 0; r0 -= kRows) {
      if (r0 != last) load_rows(r0);
      if (valid) {
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
          float x[E];
#pragma unroll
          for (int c = 0; c < kChunks; ++c) Chunk<TS>::unpack(raw[i][c], x + c * (E / kChunks));
          u32x2 out;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            // x / s == x * (1 / s) exactly: s is a power of two
            out[h] = sc > 0.0f ? encode_fp8x4(__fmul_rn(x[4 * h], inv), __fmul_rn(x[4 * h + 1], inv),
                                              __fmul_rn(x[4 * h + 2], inv), __fmul_rn(x[4 * h + 3], inv))
                               : 0u;
          }
          if (r0 + i < len) *reinterpret_cast<u32x2*>(pool + (off0 + r0 + i) * pool_stride) = out;
        }
      }
    }
    if (valid && tk % kPieces == 0) *scale_p = sc;
  }
}

template <typename TS, int D>
__global__ __launch_bounds__(256) void kv_write_fp8_kernel(uint8_t* __restrict__ k_pool,
                                                           uint8_t* __restrict__ v_pool,
                                                           float* __restrict__ k_scales,
                                                           float* __restrict__ v_scales,
                                                           const void* __restrict__ key,
                                                           const void* __restrict__ value,
                                                           const int32_t* __restrict__ slots,
                                                           int num_tokens, int hk, int block_shift,
                                                           int64_t num_blocks, int tokens_per_wg) {
  // Token t starts a run when its slot is in the pool and does not continue the slot of
  // token t - 1 on the same page. Workgroups go to the XCDs round robin; with the grid a
  // multiple of 8, XCD x takes the x-th eighth of the token windows (window = (bid % 8)
  // * grid / 8 + bid / 8), so the slot lines one L2 serves are its own (measured, 2048
  // tokens of 16-token pages: 14.6 -> 9.7 us).
  const int lane = threadIdx.x % kWave;
  const int nwin = static_cast<int>(gridDim.x);
  const int bid = static_cast<int>(blockIdx.x);
  const int win = nwin % kXcds == 0 ? (bid % kXcds) * (nwin / kXcds) + bid / kXcds : bid;
  const int t = win * tokens_per_wg + lane;
  bool start = false;
  if (lane < tokens_per_wg && t < num_tokens) {
    const int slot = slots[t];
    if (slot >= 0 && (slot >> block_shift) < num_blocks) {
      start = true;
      if (t > 0) {
        const int prev = slots[t - 1];
        if (prev >= 0 && prev + 1 == slot && (prev >> block_shift) == (slot >> block_shift)) start = false;
      }
    }
  }
  uint64_t starts = __builtin_amdgcn_ballot_w64(start);
  while (starts != 0) {
    const int t0 = win * tokens_per_wg + __builtin_ctzll(starts);
    starts &= starts - 1;
    kv_write_fp8_run<TS, D>(k_pool, v_pool, k_scales, v_scales, key, value, slots, num_tokens,
                            hk, block_shift, t0);
  }
}

template <typename TS>
hipError_t launch_fp8_t(void* k_pool, void* v_pool, float* k_scales, float* v_scales,
                        const void* key, const void* value, const int32_t* slots, int num_tokens,
                        int hk, int head_dim, int block_shift, int64_t num_blocks,
                        hipStream_t stream) {
  if (num_tokens <= 0) return hipSuccess;
  // Tokens per workgroup: one below 2048 tokens (a decode step's rows are runs of one,
  // each workgroup writes one); from 2048 (prefill chunks: runs of a page each) about
  // 256 workgroups of up to 16 tokens, so that few workgroups are launched only to find
  // no run start. Launched workgroups cost time even when idle (measured, 2048 tokens
  // of 16-token pages: 1024 workgroups 9.7 us, 256 of 8 tokens 6.1 us; 8192 tokens 12.2
  // -> 10.5 us; 65536 tokens 86.8 -> 82.7 us); runs of one then cost a workgroup up to
  // 16 in turn (2048 decode rows: 16.6 -> 29.3 us).
  const int tpw = num_tokens >= 2048 ? std::min(16, num_tokens / 256) : 1;
  const unsigned grid = static_cast<unsigned>((num_tokens + tpw - 1) / tpw);
  // threads per workgroup: the 2 * hk * D / 8 tasks, in whole waves, at most 256
  auto threads = [hk](int dim) {
    const int tasks = 2 * hk * dim / 8;
    return tasks >= 256 ? 256 : (tasks + kWave - 1) / kWave * kWave;
  };
#define MVLLM_KV_FP8(DIM)                                                                     \
  kv_write_fp8_kernel<TS, DIM><<<grid, threads(DIM), 0, stream>>>(                             \
      static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), k_scales, v_scales, key, \
      value, slots, num_tokens, hk, block_shift, num_blocks, tpw)
  switch (head_dim) {
    case 32: MVLLM_KV_FP8(32); break;
    case 64: MVLLM_KV_FP8(64); break;
    case 128: MVLLM_KV_FP8(128); break;
    case 256: MVLLM_KV_FP8(256); break;
    default: return hipErrorInvalidValue;
  }
#undef MVLLM_KV_FP8
  return hipGetLastError();
}

}  // namespace

bool kv_write_supported(int src_dtype, int pool_dtype, int head_dim) {
  if (src_dtype != kF32 && src_dtype != kF16 && src_dtype != kBF16) return false;
  if (pool_dtype == src_dtype) return true;
  return pool_dtype == kFP8E4M3 &&
         (head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256);
}

hipError_t launch_kv_write(void* k_pool, void* v_pool, float* k_scales, float* v_scales,
                           const void* key, const void* value, const int32_t* slots,
                           int num_tokens, int hk, int head_dim, int block_shift,
                           int64_t num_blocks, int src_dtype, int pool_dtype, hipStream_t stream) {
  if (pool_dtype == kFP8E4M3) {
    switch (src_dtype) {
      case kF32: return launch_fp8_t<float>(k_pool, v_pool, k_scales, v_scales, key, value, slots, num_tokens, hk, head_dim, block_shift, num_blocks, stream);
      case kF16: return launch_fp8_t<f16_t>(k_pool, v_pool, k_scales, v_scales, key, value, slots, num_tokens, hk, head_dim, block_shift, num_blocks, stream);
      case kBF16: return launch_fp8_t<bf16_t>(k_pool, v_pool, k_scales, v_scales, key, value, slots, num_tokens, hk, head_dim, block_shift, num_blocks, stream);
      default: return hipErrorInvalidValue;
    }
  }
  const int elt = src_dtype == kF32 ? 4 : 2;
  const int64_t num_slots = num_blocks << block_shift;
  const int64_t row_bytes = static_cast<int64_t>(hk) * head_dim * elt;
  const bool aligned = (reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool) |
                        reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value)) % 16 == 0;
  if (aligned && row_bytes % 16 == 0) {
    const int64_t per_token = row_bytes / 16;
    const int64_t total = per_token * num_tokens;
    kv_copy_kernel<<<static_cast<unsigned>((2 * total + 255) / 256), 256, 0, stream>>>(
        k_pool, v_pool, key, value, slots, per_token, total, num_slots);
  } else {
    const int64_t row = static_cast<int64_t>(hk) * head_dim;
    const int64_t total = row * num_tokens;
    const unsigned grid = static_cast<unsigned>((2 * total + 255) / 256);
    if (elt == 4) {
      kv_copy_scalar_kernel<float><<<grid, 256, 0, stream>>>(k_pool, v_pool, key, value, slots, row, total, num_slots);
    } else {
      kv_copy_scalar_kernel<uint16_t><<<grid, 256, 0, stream>>>(k_pool, v_pool, key, value, slots, row, total, num_slots);
    }
  }
  return hipGetLastError();
}

}  // namespace mvllm
