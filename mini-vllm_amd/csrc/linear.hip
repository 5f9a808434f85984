// Skinny projections: y[M, N] = x[M, K] * W[N, K]^T for the few rows of a decode step
// (M <= 64: one row per running sequence), bf16 or fp16 in and out, fp32 accumulate.
//
// The reference computes every projection with a plain matmul (mini_vllm/model/
// basics.py linear -> torch, i.e. the vendor BLAS). At decode sizes that is a
// matrix-vector problem: the weight matrix is read once and each element feeds
// at most M multiply-adds, so the bound is HBM bandwidth on W (2 N K bytes), not
// MFMA throughput. The BLAS tiles such shapes as small GEMMs (32 x 32 tiles, N / 32
// workgroups with the whole K each) and reached ~11 us per projection where the
// weights take ~1-4 us to read.
//
// Design (this library's own):
//  * workgroup = 32 output columns (32 rows of W) x all M rows, 4 waves; wave w owns a
//    quarter of K. No LDS staging: the MFMA 32x32x16 operands are 16-byte row pieces
//    in global memory - A = W (lane: row n0 + l32, k 8h .. 8h+7), B = x^T (lane: row
//    l32 of x, same k) - so each lane loads its fragments directly, kUnroll k-steps
//    ahead (all loads of a batch issued before its MFMAs).
//  * M > 32: a second 32-row block of x shares each W fragment.
//  * the 4 waves' partial 32 x 32 sums meet in LDS; all 256 threads add them and run
//    the epilogue:
//      plain     y = T(x w^T)
//      split     columns [0, n0) to y0, [n0, n0 + n1) to y1, the rest to y2 (the q, k
//                and v projections as one launch over their concatenated weights)
//      residual  y = T(r + T(x w^T)) (the projection, then the residual add, each
//                rounded as the two torch ops round them)
//      swiglu    w holds gate and up rows interleaved in groups of 16 (rows
//                32j .. 32j+15 = gate rows 16j .. 16j+15, the next 16 = the same up
//                rows): y[:, 16j + i] = swiglu(T(gate), T(up)), rounded as the
//                elementwise SwiGLU kernel rounds it.
//    At decode sizes every launch costs a few microseconds whatever it does, so these
//    fusions, not the GEMM's inner loop, are what the projections gain.
//  * rows of x past M read row M - 1 (discarded); columns past N read row N - 1 of W
//    (not stored).

#include "common.hpp"
#include "linear.hpp"

namespace mvllm {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct LinMma;
template <> struct LinMma<bf16_t> {
  __device__ static f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static uint16_t bits(float v) { return static_cast<uint16_t>(pack_bf16x2(v, 0.0f)); }
};
template <> struct LinMma<f16_t> {
  __device__ static f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static uint16_t bits(float v) { return static_cast<uint16_t>(f32_to_f16_bits(v)); }
};

constexpr int kColTile = 32;   // output columns per workgroup (W rows)
constexpr int kWaves = 4;      // K quarters
constexpr int kUnroll = 8;     // k-steps (16 elements each) loaded ahead of their MFMAs

struct Out {
  void* y0;
  void* y1;
  void* y2;
  const void* residual;
  int n0, n1;  // split: columns of y0 and y1
};

template <typename T, int MB, int EPI>
__global__ __launch_bounds__(kWaves * kWave) void skinny_linear_kernel(
    Out out, const void* __restrict__ x, const void* __restrict__ w, int m, int n, int k) {
  __shared__ f32x16 part[kWaves][MB][kWave];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int n0 = blockIdx.x * kColTile;

  // This lane's W row and x rows (clamped), as byte pointers at k = 8 * hsel.
  const int wrow = min(n0 + l32, n - 1);
  const char* wp = static_cast<const char*>(w) + (static_cast<int64_t>(wrow) * k + 8 * hsel) * 2;
  const char* xp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int xrow = min(mb * 32 + l32, m - 1);
    xp[mb] = static_cast<const char*>(x) + (static_cast<int64_t>(xrow) * k + 8 * hsel) * 2;
  }

  f32x16 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};

  const int kq = k / kWaves;  // a multiple of 16 (k % 64 == 0)
  const int kbeg = wave * kq;
  const int kend = kbeg + kq;
  int k0 = kbeg;
  for (; k0 + 16 * kUnroll <= kend; k0 += 16 * kUnroll) {
    u32x4 a[kUnroll], b[MB][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = load16(wp + (k0 + 16 * u) * 2);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) b[mb][u] = load16(xp[mb] + (k0 + 16 * u) * 2);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = LinMma<T>::run(a[u], b[mb][u], acc[mb]);
    }
  }
  for (; k0 < kend; k0 += 16) {
    const u32x4 a = load16(wp + k0 * 2);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = LinMma<T>::run(a, load16(xp[mb] + k0 * 2), acc[mb]);
  }

#pragma unroll
  for (int mb = 0; mb < MB; ++mb) part[wave][mb][lane] = acc[mb];
  __syncthreads();

  // Accumulator element r of lane (l32, hsel) is C[W row 8(r/4) + 4 hsel + r%4][x row
  // l32]; the sum over the waves of C[col][row] of this tile:
  auto total = [&](int row, int col) __attribute__((always_inline)) {
    const int mb = row / 32, r32 = row % 32;
    const int src = ((col >> 2) & 1) * 32 + r32;
    const int reg = (col >> 3) * 4 + (col & 3);
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) sum += part[wv][mb][src][reg];
    return sum;
  };
  if constexpr (EPI == kLinearSwiglu) {
    // 16 output columns per tile: gate col j pairs with up col 16 + j.
    const int nout = n / 2;
    uint16_t* yo = static_cast<uint16_t*>(out.y0);
    for (int e = threadIdx.x; e < MB * 32 * 16; e += kWaves * kWave) {
      const int j = e % 16, row = e / 16;
      const float g = Elem<T>::round(total(row, j));
      const float u = Elem<T>::round(total(row, 16 + j));
      const int gcol = blockIdx.x * 16 + j;
      if (row < m && gcol < nout) yo[static_cast<int64_t>(row) * nout + gcol] = LinMma<T>::bits(swiglu_one<T>(g, u));
    }
  } else {
    for (int e = threadIdx.x; e < MB * 32 * kColTile; e += kWaves * kWave) {
      const int col = e % kColTile, row = e / kColTile;
      const int gcol = n0 + col;
      if (row >= m || gcol >= n) continue;
      const float sum = total(row, col);
      if constexpr (EPI == kLinearPlain) {
        static_cast<uint16_t*>(out.y0)[static_cast<int64_t>(row) * n + gcol] = LinMma<T>::bits(sum);
      } else if constexpr (EPI == kLinearResidual) {
        const int64_t i = static_cast<int64_t>(row) * n + gcol;
        const float r = Elem<T>::load(out.residual, i);
        static_cast<uint16_t*>(out.y0)[i] = LinMma<T>::bits(r + Elem<T>::round(sum));
      } else {  // split: a 32-column tile lies in one destination (n0, n1 multiples of 32)
        void* dst = out.y0;
        int c = gcol, width = out.n0;
        if (gcol >= out.n0 + out.n1) {
          dst = out.y2; c = gcol - out.n0 - out.n1; width = n - out.n0 - out.n1;
        } else if (gcol >= out.n0) {
          dst = out.y1; c = gcol - out.n0; width = out.n1;
        }
        static_cast<uint16_t*>(dst)[static_cast<int64_t>(row) * width + c] = LinMma<T>::bits(sum);
      }
    }
  }
}

template <typename T, int EPI>
hipError_t launch_t(const Out& out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((n + kColTile - 1) / kColTile));
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  if (m <= 32) {
    skinny_linear_kernel<T, 1, EPI><<<grid, kWaves * kWave, 0, stream>>>(out, x, w, mi, ni, ki);
  } else {
    skinny_linear_kernel<T, 2, EPI><<<grid, kWaves * kWave, 0, stream>>>(out, x, w, mi, ni, ki);
  }
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_e(const Out& out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    int dtype, hipStream_t stream) {
  if (dtype == kBF16) return launch_t<bf16_t, EPI>(out, x, w, m, n, k, stream);
  if (dtype == kF16) return launch_t<f16_t, EPI>(out, x, w, m, n, k, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool skinny_linear_supported(int dtype, int64_t m, int64_t n, int64_t k) {
  if (dtype != kBF16 && dtype != kF16) return false;
  return m >= 1 && m <= kSkinnyMaxRows && n >= 1 && n < (int64_t{1} << 31) / 64 && k >= 64 &&
         k % 64 == 0 && k < (int64_t{1} << 24);
}

hipError_t launch_skinny_linear(void* y, const void* x, const void* w, int64_t m, int64_t n,
                                int64_t k, int dtype, hipStream_t stream) {
  return launch_e<kLinearPlain>(Out{y, nullptr, nullptr, nullptr, 0, 0}, x, w, m, n, k, dtype, stream);
}

hipError_t launch_skinny_linear_split(void* y0, void* y1, void* y2, const void* x, const void* w,
                                      int64_t m, int64_t n0, int64_t n1, int64_t n2, int64_t k,
                                      int dtype, hipStream_t stream) {
  return launch_e<kLinearSplit>(Out{y0, y1, y2, nullptr, static_cast<int>(n0), static_cast<int>(n1)},
                                x, w, m, n0 + n1 + n2, k, dtype, stream);
}

hipError_t launch_skinny_linear_residual(void* y, const void* x, const void* w, const void* residual,
                                         int64_t m, int64_t n, int64_t k, int dtype,
                                         hipStream_t stream) {
  return launch_e<kLinearResidual>(Out{y, nullptr, nullptr, residual, 0, 0}, x, w, m, n, k, dtype,
                                   stream);
}

hipError_t launch_skinny_linear_swiglu(void* y, const void* x, const void* w_gate_up, int64_t m,
                                       int64_t n_out, int64_t k, int dtype, hipStream_t stream) {
  return launch_e<kLinearSwiglu>(Out{y, nullptr, nullptr, nullptr, 0, 0}, x, w_gate_up, m, 2 * n_out,
                                 k, dtype, stream);
}

}  // namespace mvllm
