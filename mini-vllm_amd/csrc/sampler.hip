// Greedy sampling: the index of each logits row's maximum (torch.argmax(dim=-1)).
//
// The reference engine samples through mini_vllm/sampler.py: greedy rows take
// logits.argmax(dim=-1) (sampler.py:135-141), the decode loop's last device op before
// the one host read per iteration. Over a Qwen3 vocabulary (151936 entries) torch's
// generic reduction took ~50 us for 32 rows on this GPU, more than a whole layer's
// attention; the row is a 300 KB read, a few microseconds of HBM time.
//
// Design (this library's own): each row is cut into segments of 16384 logits, one
// workgroup of 256 threads each (a row on one CU streamed at well under the chip's
// share: ~19 us for 32 rows), every thread issuing its 16-byte loads up front and
// keeping the best (key, index) of its elements; a wave reduction and an LDS pass
// finish the segment, and a second launch the row (none for a one-segment row). Ordering follows torch exactly: values compare as floats with -0
// equal to +0, NaN greater than any number, and among equal maxima the first index
// wins. That order is one 64-bit unsigned max over
//     key   = monotone map of the float's bits (NaN -> all ones, -0 -> +0)
//     index = stored as 0xFFFFFFFF - index
// so the reduction is order-independent and the result deterministic.

#include <algorithm>

#include "common.hpp"
#include "sampler.hpp"

namespace mvllm {

namespace {

constexpr int kArgmaxThreads = 256;
constexpr int64_t kSegment = 16384;  // elements per workgroup
constexpr int kMaxSegments = 64;

__device__ __forceinline__ uint64_t argmax_key(float f, uint32_t index) {
  uint32_t bits = __float_as_uint(f);
  if (f == 0.0f) bits = 0;  // -0 compares equal to +0
  uint32_t key = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  if (f != f) key = 0xFFFFFFFFu;  // NaN beats every number
  return (static_cast<uint64_t>(key) << 32) | (0xFFFFFFFFu - index);
}

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
  const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
  return (static_cast<uint64_t>(static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi), mask, 64)))
          << 32) |
         static_cast<uint32_t>(__shfl_xor(static_cast<int>(lo), mask, 64));
}

__device__ __forceinline__ uint64_t wave_max64(uint64_t v) {
#pragma unroll
  for (int mask = 1; mask < kWave; mask <<= 1) v = max64(v, shfl_xor64(v, mask));
  return v;
}

// The best key of segment blockIdx.y (kSegment elements) of row blockIdx.x: to
// keys[row * gridDim.y + segment], or, with one segment, the index to out[row].
template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(int64_t* __restrict__ out,
                                                               uint64_t* __restrict__ keys,
                                                               const T* __restrict__ logits,
                                                               int64_t v, int64_t row_stride,
                                                               bool vec) {
  __shared__ uint64_t wave_best[kArgmaxThreads / kWave];
  const T* row = logits + static_cast<int64_t>(blockIdx.x) * row_stride;
  const int64_t lo = static_cast<int64_t>(blockIdx.y) * kSegment;
  const int64_t hi = min(v, lo + kSegment);
  uint64_t best = 0;
  if (vec && hi / (16 / static_cast<int64_t>(sizeof(T))) > lo / (16 / static_cast<int64_t>(sizeof(T)))) {
    // 16-byte chunks: 16 / sizeof(T) elements each (kSegment is a multiple), every load
    // of the thread issued first; the segment holds at least one whole chunk.
    constexpr int kPer = 16 / sizeof(T);
    constexpr int kAhead = kSegment / kPer / kArgmaxThreads;
    const int64_t c_lo = lo / kPer, c_hi = hi / kPer;  // whole chunks of the segment
    u32x4 w[kAhead];
#pragma unroll
    for (int a = 0; a < kAhead; ++a) {
      const int64_t c = min(c_lo + threadIdx.x + a * kArgmaxThreads, c_hi - 1);
      w[a] = load16(static_cast<const char*>(static_cast<const void*>(row)) + c * 16);
    }
#pragma unroll
    for (int a = 0; a < kAhead; ++a) {
      const int64_t c = c_lo + threadIdx.x + a * kArgmaxThreads;
      if (c < c_hi) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          best = max64(best, argmax_key(Elem<T>::load(&w[a], i), static_cast<uint32_t>(c * kPer + i)));
        }
      }
    }
    for (int64_t i = c_hi * kPer + threadIdx.x; i < hi; i += kArgmaxThreads) {
      best = max64(best, argmax_key(Elem<T>::load(row, i), static_cast<uint32_t>(i)));
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kArgmaxThreads) {
      best = max64(best, argmax_key(Elem<T>::load(row, i), static_cast<uint32_t>(i)));
    }
  }
  best = wave_max64(best);
  if (threadIdx.x % kWave == 0) wave_best[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x < kWave) {
    best = threadIdx.x < kArgmaxThreads / kWave ? wave_best[threadIdx.x] : 0;
    best = wave_max64(best);
    if (threadIdx.x == 0) {
      if (gridDim.y == 1) {
        out[blockIdx.x] = 0xFFFFFFFFu - static_cast<uint32_t>(best);
      } else {
        keys[static_cast<int64_t>(blockIdx.x) * gridDim.y + blockIdx.y] = best;
      }
    }
  }
}

// One wave per row: the best of its segments' keys, as an index.
__global__ __launch_bounds__(kWave) void argmax_finish_kernel(int64_t* __restrict__ out,
                                                             const uint64_t* __restrict__ keys,
                                                             int segments) {
  const uint64_t* k = keys + static_cast<int64_t>(blockIdx.x) * segments;
  uint64_t best = threadIdx.x < segments ? k[threadIdx.x] : 0;
  best = wave_max64(best);
  if (threadIdx.x == 0) out[blockIdx.x] = 0xFFFFFFFFu - static_cast<uint32_t>(best);
}

int segments_of(int64_t v) { return static_cast<int>((v + kSegment - 1) / kSegment); }

template <typename T>
hipError_t launch_argmax_t(int64_t* out, const void* logits, int64_t rows, int64_t v,
                           int64_t row_stride, void* workspace, hipStream_t stream) {
  const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) &&
                   (row_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0;
  const int segments = segments_of(v);
  argmax_kernel<T><<<dim3(static_cast<unsigned>(rows), segments), kArgmaxThreads, 0, stream>>>(
      out, static_cast<uint64_t*>(workspace), static_cast<const T*>(logits), v, row_stride, vec);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || segments == 1) return e;
  argmax_finish_kernel<<<static_cast<unsigned>(rows), kWave, 0, stream>>>(
      out, static_cast<const uint64_t*>(workspace), segments);
  return hipGetLastError();
}

}  // namespace

uint64_t argmax_workspace_bytes(int64_t rows, int64_t v) {
  const int segments = segments_of(v);
  return segments > 1 ? static_cast<uint64_t>(rows) * segments * sizeof(uint64_t) : 0;
}

int64_t argmax_max_vocab() { return kSegment * kMaxSegments; }

hipError_t launch_argmax(int64_t* out, const void* logits, int64_t rows, int64_t v,
                         int64_t row_stride, int dtype, void* workspace, hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_argmax_t<float>(out, logits, rows, v, row_stride, workspace, stream);
    case kF16: return launch_argmax_t<f16_t>(out, logits, rows, v, row_stride, workspace, stream);
    case kBF16: return launch_argmax_t<bf16_t>(out, logits, rows, v, row_stride, workspace, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mvllm
