// The memory-bound elementwise kernels between the attention calls: RMSNorm (also
// used as Qwen3's per-head QK-norm), rotate-halves RoPE and SwiGLU.
//
// Each one is one read and one write of its tensors. Rounding points follow the
// reference's PyTorch expressions exactly, because those are what parity is judged
// against:
//   rmsnorm  out = T(w * T(x * rsqrt(mean(x^2) + eps)))   (layer_norm.py:40-46,
//            csrc/rmsnorm.cu:80-87): fp32 reduction, round before the weight multiply.
//   rope     out = T(x*cos[pos] + rotate_half(x)*sin[pos]) in fp32 with the two
//            products rounded separately (positional_encoding.py:58-62); products are
//            rounded on their own: this file is compiled with -ffp-contract=off (the
//            build sets it), since HIP's default contraction fuses x*cos - y*sin into one
//            FMA that rounds once where the reference rounds three times. A pragma is not
//            enough: the products come from inlined header functions.
//   swiglu   out = T(T(g * T(sigmoid(g))) * u) (basics.py:39-41, csrc/swiglu.cu:48-51),
//            sigmoid = 1 / (1 + expf(-g)).

#include "common.hpp"
#include "elementwise.hpp"

namespace mvllm {

// ------------------------------------------------------------------- rmsnorm

// kR lanes per row (a power of two <= 64), each holding up to kMaxCh 16-byte chunks of
// the row in registers between the reduction and the scale pass; 64 / kR rows per wave.
// x and out are streamed nontemporally, the weight row (shared by every row) is cached.
template <typename T, int kR, int kMaxCh>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(const void* __restrict__ x,
                                                          const void* __restrict__ w,
                                                          void* __restrict__ out, int64_t rows,
                                                          int dim, float eps) {
  constexpr int E = Chunk<T>::kN;
  const int lane = threadIdx.x % kWave;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kR;
  const int r = lane % kR;
  const bool live = row < rows;
  const int chunks = dim / E;

  const char* xr = static_cast<const char*>(x) + (live ? row : 0) * static_cast<int64_t>(dim) * Elem<T>::kBytes;
  u32x4 held[kMaxCh];
  float sumsq = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    const int chunk = r + c * kR;
    if (chunk < chunks) {
      held[c] = nt_load16(xr + chunk * 16);
      float f[E];
      Chunk<T>::unpack(held[c], f);
#pragma unroll
      for (int e = 0; e < E; ++e) sumsq = fmaf(f[e], f[e], sumsq);
    }
  }
  sumsq = group_sum<kR>(sumsq);
  const float inv = rsqrtf(sumsq / static_cast<float>(dim) + eps);
  if (!live) return;

  char* orow = static_cast<char*>(out) + row * static_cast<int64_t>(dim) * Elem<T>::kBytes;
  const char* wr = static_cast<const char*>(w);
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    const int chunk = r + c * kR;
    if (chunk < chunks) {
      float f[E], wf[E];
      Chunk<T>::unpack(held[c], f);
      Chunk<T>::unpack(load16(wr + chunk * 16), wf);
      u32x4 res;
      if constexpr (E == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) res[e] = __float_as_uint(__fmul_rn(__fmul_rn(f[e], inv), wf[e]));
      } else {
#pragma unroll
        for (int e = 0; e < E; e += 2) {
          float o2[2];
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const float normalized = Elem<T>::round(__fmul_rn(f[e + k], inv));
            o2[k] = __fmul_rn(normalized, wf[e + k]);
          }
          if constexpr (__is_same(T, bf16_t)) {
            res[e / 2] = f32_to_bf16_bits(o2[0]) | (f32_to_bf16_bits(o2[1]) << 16);
          } else {
            res[e / 2] = f32_to_f16_bits(o2[0]) | (f32_to_f16_bits(o2[1]) << 16);
          }
        }
      }
      nt_store16(orow + chunk * 16, res);
    }
  }
}

// Any shape, any alignment: one wave per row, element at a time.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_scalar_kernel(const void* __restrict__ x,
                                                             const void* __restrict__ w,
                                                             void* __restrict__ out, int64_t rows,
                                                             int dim, float eps) {
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;  // whole wave leaves together
  const int64_t base = row * dim;
  float sumsq = 0.0f;
  for (int i = lane; i < dim; i += kWave) {
    const float v = Elem<T>::load(x, base + i);
    sumsq = fmaf(v, v, sumsq);
  }
  sumsq = wave_sum(sumsq);
  const float inv = rsqrtf(sumsq / static_cast<float>(dim) + eps);
  for (int i = lane; i < dim; i += kWave) {
    const float normalized = Elem<T>::round(__fmul_rn(Elem<T>::load(x, base + i), inv));
    Elem<T>::store(out, base + i, __fmul_rn(normalized, Elem<T>::load(w, i)));
  }
}

namespace {

template <typename T, int kR>
hipError_t launch_rmsnorm_r(const void* x, const void* w, void* out, int64_t rows, int dim,
                            float eps, hipStream_t stream) {
  constexpr int E = Chunk<T>::kN;
  const int chunks = dim / E;
  const int per_lane = (chunks + kR - 1) / kR;
  const int64_t threads = rows * kR;
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (per_lane <= 1) {
    rmsnorm_vec_kernel<T, kR, 1><<<grid, 256, 0, stream>>>(x, w, out, rows, dim, eps);
  } else if (per_lane <= 2) {
    rmsnorm_vec_kernel<T, kR, 2><<<grid, 256, 0, stream>>>(x, w, out, rows, dim, eps);
  } else if (per_lane <= 4) {
    rmsnorm_vec_kernel<T, kR, 4><<<grid, 256, 0, stream>>>(x, w, out, rows, dim, eps);
  } else {
    rmsnorm_vec_kernel<T, kR, 8><<<grid, 256, 0, stream>>>(x, w, out, rows, dim, eps);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_rmsnorm_t(const void* x, const void* w, void* out, int64_t rows, int dim,
                            float eps, hipStream_t stream) {
  constexpr int E = Chunk<T>::kN;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                        reinterpret_cast<uintptr_t>(out)) % 16 == 0;
  const int chunks = dim / E;
  if (!aligned || dim % E != 0 || chunks > 64 * 8) {
    const dim3 grid(static_cast<unsigned>((rows * kWave + 255) / 256));
    rmsnorm_scalar_kernel<T><<<grid, 256, 0, stream>>>(x, w, out, rows, dim, eps);
    return hipGetLastError();
  }
  if (chunks <= 1) return launch_rmsnorm_r<T, 1>(x, w, out, rows, dim, eps, stream);
  if (chunks <= 2) return launch_rmsnorm_r<T, 2>(x, w, out, rows, dim, eps, stream);
  if (chunks <= 4) return launch_rmsnorm_r<T, 4>(x, w, out, rows, dim, eps, stream);
  if (chunks <= 8) return launch_rmsnorm_r<T, 8>(x, w, out, rows, dim, eps, stream);
  if (chunks <= 16) return launch_rmsnorm_r<T, 16>(x, w, out, rows, dim, eps, stream);
  if (chunks <= 32) return launch_rmsnorm_r<T, 32>(x, w, out, rows, dim, eps, stream);
  return launch_rmsnorm_r<T, 64>(x, w, out, rows, dim, eps, stream);
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int dim,
                          float eps, int dtype, hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_rmsnorm_t<float>(x, w, out, rows, dim, eps, stream);
    case kF16: return launch_rmsnorm_t<f16_t>(x, w, out, rows, dim, eps, stream);
    case kBF16: return launch_rmsnorm_t<bf16_t>(x, w, out, rows, dim, eps, stream);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------- rope

// One thread per rotated pair (element i and i + D/2 of one head vector).
// positions[token % num_positions] broadcasts a short position tensor over a batch,
// as the reference's kernel does (csrc/rope.cu:58-62). A position outside the tables
// produces NaN for that pair rather than an out-of-bounds read.
template <typename T, typename TPos>
__global__ __launch_bounds__(256) void rope_kernel(const void* __restrict__ x,
                                                   const TPos* __restrict__ positions,
                                                   const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t,
                                                   void* __restrict__ out, int64_t pairs, int half,
                                                   int64_t heads, int64_t num_positions,
                                                   int64_t max_positions) {
  const int64_t index = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= pairs) return;
  const int64_t row = index / half;
  const int i = static_cast<int>(index % half);
  const int64_t token = row / heads;
  const int64_t pos = static_cast<int64_t>(positions[token % num_positions]);
  const int64_t dim = 2 * half;
  const int64_t lo = row * dim + i;
  const int64_t hi = lo + half;
  if (pos < 0 || pos >= max_positions) {
    Elem<T>::store(out, lo, __int_as_float(0x7fc00000));
    Elem<T>::store(out, hi, __int_as_float(0x7fc00000));
    return;
  }
  const float xl = Elem<T>::load(x, lo);
  const float xh = Elem<T>::load(x, hi);
  const int64_t tl = pos * dim + i;
  const int64_t th = tl + half;
  Elem<T>::store(out, lo, __fsub_rn(__fmul_rn(xl, cos_t[tl]), __fmul_rn(xh, sin_t[tl])));
  Elem<T>::store(out, hi, __fadd_rn(__fmul_rn(xh, cos_t[th]), __fmul_rn(xl, sin_t[th])));
}

// Pack N floats (N = 16 / sizeof(T)) back into one 16-byte chunk of T.
template <typename T>
__device__ __forceinline__ u32x4 pack_chunk(const float* v) {
  u32x4 r;
  if constexpr (__is_same(T, float)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = __float_as_uint(v[e]);
  } else if constexpr (__is_same(T, bf16_t)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = f32_to_f16_bits(v[2 * e]) | (f32_to_f16_bits(v[2 * e + 1]) << 16);
  }
  return r;
}

// Vectorised RoPE: one thread per 16-byte chunk of the lower half of a head vector and
// the matching chunk of the upper half, so every access to x and out is a 16-byte
// vector access and the cos/sin rows are read as 16-byte pieces. x and out are streamed
// nontemporally; the cos/sin rows, which every head of a token reads again, are
// ordinary cached loads. `tpr` = threads per
// head vector = (D/2) / N. Same rounding points as rope_kernel. Indices are 32-bit:
// the host takes this path only when rows * tpr < 2^31.
template <typename T, typename TPos>
__global__ __launch_bounds__(256) void rope_vec_kernel(const void* __restrict__ x,
                                                       const TPos* __restrict__ positions,
                                                       const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t,
                                                       void* __restrict__ out, uint32_t threads,
                                                       uint32_t tpr, uint32_t heads,
                                                       int64_t num_positions, int64_t max_positions) {
  constexpr int N = Chunk<T>::kN;
  const uint32_t index = blockIdx.x * blockDim.x + threadIdx.x;
  if (index >= threads) return;
  const uint32_t row = index / tpr;
  const uint32_t c = index - row * tpr;
  const uint32_t token = row / heads;
  const int64_t pos = static_cast<int64_t>(positions[static_cast<int64_t>(token) % num_positions]);
  const int64_t half_bytes = static_cast<int64_t>(tpr) * 16;
  const int64_t lo_off = static_cast<int64_t>(row) * 2 * half_bytes + c * 16;
  char* o = static_cast<char*>(out) + lo_off;
  if (pos < 0 || pos >= max_positions) {
    float nan[N];
#pragma unroll
    for (int e = 0; e < N; ++e) nan[e] = __int_as_float(0x7fc00000);
    store16(o, pack_chunk<T>(nan));
    store16(o + half_bytes, pack_chunk<T>(nan));
    return;
  }
  const char* xp = static_cast<const char*>(x) + lo_off;
  float xl[N], xh[N];
  Chunk<T>::unpack(nt_load16(xp), xl);
  Chunk<T>::unpack(nt_load16(xp + half_bytes), xh);
  const int64_t half = static_cast<int64_t>(tpr) * N;
  const int64_t tl = pos * 2 * half + static_cast<int64_t>(c) * N;
  float cl[N], sl[N], ch[N], sh[N];
#pragma unroll
  for (int e = 0; e < N; e += 4) {
    Chunk<float>::unpack(load16(cos_t + tl + e), cl + e);
    Chunk<float>::unpack(load16(sin_t + tl + e), sl + e);
    Chunk<float>::unpack(load16(cos_t + tl + half + e), ch + e);
    Chunk<float>::unpack(load16(sin_t + tl + half + e), sh + e);
  }
  float lo[N], hi[N];
#pragma unroll
  for (int e = 0; e < N; ++e) {
    lo[e] = __fsub_rn(__fmul_rn(xl[e], cl[e]), __fmul_rn(xh[e], sl[e]));
    hi[e] = __fadd_rn(__fmul_rn(xh[e], ch[e]), __fmul_rn(xl[e], sh[e]));
  }
  nt_store16(o, pack_chunk<T>(lo));
  nt_store16(o + half_bytes, pack_chunk<T>(hi));
}

namespace {
template <typename T>
hipError_t launch_rope_t(const void* x, const void* positions, int pos_bytes, const float* cos_t,
                         const float* sin_t, void* out, int64_t rows, int64_t heads, int dim,
                         int64_t num_positions, int64_t max_positions, hipStream_t stream) {
  constexpr int N = Chunk<T>::kN;
  const int half = dim / 2;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                        reinterpret_cast<uintptr_t>(cos_t) | reinterpret_cast<uintptr_t>(sin_t)) % 16 == 0;
  const int64_t tpr = half / N;
  if (aligned && half % N == 0 && rows * tpr < (int64_t{1} << 31) && heads < (int64_t{1} << 31)) {
    const uint32_t threads = static_cast<uint32_t>(rows * tpr);
    const dim3 grid((threads + 255) / 256);
    if (pos_bytes == 8) {
      rope_vec_kernel<T, int64_t><<<grid, 256, 0, stream>>>(
          x, static_cast<const int64_t*>(positions), cos_t, sin_t, out, threads,
          static_cast<uint32_t>(tpr), static_cast<uint32_t>(heads), num_positions, max_positions);
    } else {
      rope_vec_kernel<T, int32_t><<<grid, 256, 0, stream>>>(
          x, static_cast<const int32_t*>(positions), cos_t, sin_t, out, threads,
          static_cast<uint32_t>(tpr), static_cast<uint32_t>(heads), num_positions, max_positions);
    }
    return hipGetLastError();
  }
  const int64_t pairs = rows * half;
  const dim3 grid(static_cast<unsigned>((pairs + 255) / 256));
  if (pos_bytes == 8) {
    rope_kernel<T, int64_t><<<grid, 256, 0, stream>>>(x, static_cast<const int64_t*>(positions),
                                                       cos_t, sin_t, out, pairs, half, heads,
                                                       num_positions, max_positions);
  } else {
    rope_kernel<T, int32_t><<<grid, 256, 0, stream>>>(x, static_cast<const int32_t*>(positions),
                                                       cos_t, sin_t, out, pairs, half, heads,
                                                       num_positions, max_positions);
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_rope(const void* x, const void* positions, int pos_bytes, const float* cos_t,
                       const float* sin_t, void* out, int64_t rows, int64_t heads, int dim,
                       int64_t num_positions, int64_t max_positions, int dtype,
                       hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_rope_t<float>(x, positions, pos_bytes, cos_t, sin_t, out, rows, heads, dim, num_positions, max_positions, stream);
    case kF16: return launch_rope_t<f16_t>(x, positions, pos_bytes, cos_t, sin_t, out, rows, heads, dim, num_positions, max_positions, stream);
    case kBF16: return launch_rope_t<bf16_t>(x, positions, pos_bytes, cos_t, sin_t, out, rows, heads, dim, num_positions, max_positions, stream);
    default: return hipErrorInvalidValue;
  }
}

// -------------------------------------------------------------------- swiglu

template <typename T>
__device__ __forceinline__ float swiglu_one(float g, float u) {
  const float sig = Elem<T>::round(1.0f / (1.0f + expf(-g)));
  const float act = Elem<T>::round(__fmul_rn(g, sig));
  return __fmul_rn(act, u);
}

template <typename T>
__device__ __forceinline__ u32x4 swiglu_chunk(const u32x4& gw, const u32x4& uw) {
  constexpr int E = Chunk<T>::kN;
  float g[E], u[E], r[E];
  Chunk<T>::unpack(gw, g);
  Chunk<T>::unpack(uw, u);
#pragma unroll
  for (int e = 0; e < E; ++e) r[e] = swiglu_one<T>(g[e], u[e]);
  return pack_chunk<T>(r);
}

// One thread per 16-byte chunk of the flat buffers, streamed nontemporally (measured on
// MI355X at I=3072 bf16: faster than ordinary loads, and than two chunks per thread).
template <typename T>
__global__ __launch_bounds__(256) void swiglu_vec_kernel(const void* __restrict__ gate,
                                                         const void* __restrict__ up,
                                                         void* __restrict__ out, int64_t chunks) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= chunks) return;
  const u32x4 g = nt_load16(static_cast<const char*>(gate) + i * 16);
  const u32x4 u = nt_load16(static_cast<const char*>(up) + i * 16);
  nt_store16(static_cast<char*>(out) + i * 16, swiglu_chunk<T>(g, u));
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_scalar_kernel(const void* __restrict__ gate,
                                                            const void* __restrict__ up,
                                                            void* __restrict__ out, int64_t n) {
  const int64_t index = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= n) return;
  Elem<T>::store(out, index, swiglu_one<T>(Elem<T>::load(gate, index), Elem<T>::load(up, index)));
}

namespace {
template <typename T>
hipError_t launch_swiglu_t(const void* gate, const void* up, void* out, int64_t n,
                           hipStream_t stream) {
  constexpr int E = Chunk<T>::kN;
  const bool aligned = (reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) |
                        reinterpret_cast<uintptr_t>(out)) % 16 == 0;
  if (aligned && n % E == 0) {
    const int64_t chunks = n / E;
    swiglu_vec_kernel<T><<<static_cast<unsigned>((chunks + 255) / 256), 256, 0, stream>>>(gate, up, out, chunks);
  } else {
    swiglu_scalar_kernel<T><<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(gate, up, out, n);
  }
  return hipGetLastError();
}
}  // namespace

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
                         hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_swiglu_t<float>(gate, up, out, n, stream);
    case kF16: return launch_swiglu_t<f16_t>(gate, up, out, n, stream);
    case kBF16: return launch_swiglu_t<bf16_t>(gate, up, out, n, stream);
    default: return hipErrorInvalidValue;
  }
}

// --------------------------------------------------------------------- axpby

// y = a * x + b: the toolchain smoke kernel (reference csrc/hello.cu:11-21).
__global__ void axpby_kernel(const float* __restrict__ x, float* __restrict__ y, float a, float b,
                             int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a * x[i] + b;
}

hipError_t launch_axpby(const float* x, float* y, float a, float b, int64_t n, hipStream_t stream) {
  axpby_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(x, y, a, b, n);
  return hipGetLastError();
}

}  // namespace mvllm
