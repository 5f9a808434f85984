// Greedy sampling: the index of each logits row's maximum (torch.argmax(dim=-1)).
//
// The reference engine samples through mini_vllm/sampler.py: greedy rows take
// logits.argmax(dim=-1) (sampler.py:135-141), the decode loop's last device op before
// the one host read per iteration. Over a Qwen3 vocabulary (151936 entries) torch's
// generic reduction took ~50 us for 32 rows on this GPU, more than a whole layer's
// attention; the row is a 300 KB read, a few microseconds of HBM time.
//
// Design (this library's own): one workgroup of 1024 threads per row, every thread
// issuing its 16-byte loads of the row up front (V / 8 / 1024 ~ 19 for bf16) and
// keeping the best (key, index) of its elements; a wave reduction and an LDS pass
// finish the row. Ordering follows torch exactly: values compare as floats with -0
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

constexpr int kArgmaxThreads = 1024;

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

template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(int64_t* __restrict__ out,
                                                               const T* __restrict__ logits,
                                                               int64_t v, int64_t row_stride,
                                                               bool vec) {
  __shared__ uint64_t wave_best[kArgmaxThreads / kWave];
  const T* row = logits + static_cast<int64_t>(blockIdx.x) * row_stride;
  uint64_t best = 0;
  if (vec) {
    // 16-byte chunks: 16 / sizeof(T) elements each, all loads of the thread first.
    constexpr int kPer = 16 / sizeof(T);
    constexpr int kAhead = 24;  // a 196608-element bf16 row in one batch
    const int64_t chunks = v / kPer;
    for (int64_t c0 = threadIdx.x; c0 < chunks; c0 += kAhead * kArgmaxThreads) {
      u32x4 w[kAhead];
#pragma unroll
      for (int a = 0; a < kAhead; ++a) {
        const int64_t c = min(c0 + a * kArgmaxThreads, chunks - 1);
        w[a] = load16(static_cast<const char*>(static_cast<const void*>(row)) + c * 16);
      }
#pragma unroll
      for (int a = 0; a < kAhead; ++a) {
        const int64_t c = c0 + a * kArgmaxThreads;
        if (c < chunks) {
#pragma unroll
          for (int i = 0; i < kPer; ++i) {
            best = max64(best, argmax_key(Elem<T>::load(&w[a], i), static_cast<uint32_t>(c * kPer + i)));
          }
        }
      }
    }
    for (int64_t i = chunks * kPer + threadIdx.x; i < v; i += kArgmaxThreads) {
      best = max64(best, argmax_key(Elem<T>::load(row, i), static_cast<uint32_t>(i)));
    }
  } else {
    for (int64_t i = threadIdx.x; i < v; i += kArgmaxThreads) {
      best = max64(best, argmax_key(Elem<T>::load(row, i), static_cast<uint32_t>(i)));
    }
  }
#pragma unroll
  for (int mask = 1; mask < kWave; mask <<= 1) best = max64(best, shfl_xor64(best, mask));
  if (threadIdx.x % kWave == 0) wave_best[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x < kWave) {
    best = threadIdx.x < kArgmaxThreads / kWave ? wave_best[threadIdx.x] : 0;
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) best = max64(best, shfl_xor64(best, mask));
    if (threadIdx.x == 0) out[blockIdx.x] = 0xFFFFFFFFu - static_cast<uint32_t>(best);
  }
}

template <typename T>
hipError_t launch_argmax_t(int64_t* out, const void* logits, int64_t rows, int64_t v,
                           int64_t row_stride, hipStream_t stream) {
  const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) &&
                   (row_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0;
  argmax_kernel<T><<<static_cast<unsigned>(rows), kArgmaxThreads, 0, stream>>>(
      out, static_cast<const T*>(logits), v, row_stride, vec);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_argmax(int64_t* out, const void* logits, int64_t rows, int64_t v,
                         int64_t row_stride, int dtype, hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_argmax_t<float>(out, logits, rows, v, row_stride, stream);
    case kF16: return launch_argmax_t<f16_t>(out, logits, rows, v, row_stride, stream);
    case kBF16: return launch_argmax_t<bf16_t>(out, logits, rows, v, row_stride, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mvllm
