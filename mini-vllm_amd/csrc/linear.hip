// Skinny projections: y[M, N] = x[M, K] * W[N, K]^T for the few rows of a decode step
// (M <= 64: one row per running sequence), bf16 or fp16 in and out, fp32 accumulate.
//
// The reference computes every projection with a plain matmul (mini_vllm/model/
// basics.py linear -> torch, i.e. the vendor BLAS). At decode sizes that is a
// matrix-vector problem: the weight matrix is read once and each element feeds
// at most M multiply-adds, so the bound is HBM bandwidth on W (2 N K bytes), not
// MFMA throughput. In a decode step the weights are cold (a model's layers together
// exceed the last-level cache), so the time is set by how well the reads of W stream:
// how many bytes are in flight at once, and how many cache lines each load touches.
//
// Design (this library's own):
//  * W is stored pre-shuffled into MFMA fragment order ("packed", done once when the
//    weights are loaded): for each tile of 32 rows and each k-step of 16 elements, the
//    1 KB that the 64 lanes of a wave need for one v_mfma_f32_32x32x16 A operand lie
//    contiguously, lane l = 32 h + r holding W[32 t + r][16 s + 8 h .. 16 s + 8 h + 7]:
//        byte offset ((t * K/16 + s) * 64 + l) * 16.
//    A wave's load of a k-step is then one fully used 1 KB run (8 cache lines), where
//    the row-major layout touches 32 lines for 32 bytes each (measured: ~2.5 us more per
//    8 MB of cold weights). Rows past N are zero padding to the 32-row tile.
//  * a workgroup is one tile of 32 output columns with all M rows, and 4 (K <= 1024) or
//    8 waves that split K between them, in batches of at most 16 k-steps per wave; each
//    wave issues every load of a batch before its first MFMA, so a projection's weights
//    are requested up front. The waves' partial 32 x 32 sums meet in LDS. K is not split
//    over workgroups: a cross-workgroup reduction needs device-scope release/acquire
//    fences, which write back and invalidate L2 on this part (measured 2-3x slower).
//    The split depends on K alone, so a column's sum is formed the same way whatever N,
//    M or epilogue: the fused launches below equal the plain one bit for bit.
//  * B = x^T fragments (lane: row l32 of x, the same k): each wave copies its batch of
//    x (32 or 64 rows x its k-steps) from global memory into LDS with the direct-to-LDS
//    load (fully used 1 KB runs; x stays in L2), swizzled, and reads the fragments back
//    from there - the same line-count argument as for W, measured ~2.5 us per projection
//    against fragment loads straight from x. M > 32: a second 32-row block of x shares
//    each W fragment.
//  * epilogues, run by all threads over the LDS sums:
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
//    fusions save as much as the GEMM's inner loop.
//  * rows of x past M read row M - 1 (discarded); k-steps past a wave's range re-read
//    its last step (not summed). M0 is set only by the LDS copies.

#include <algorithm>

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

constexpr int kColTile = 32;    // output columns per workgroup (W rows)
constexpr int kBatch = 16;      // k-steps (16 elements) a wave loads before its MFMAs

struct Out {
  void* y0;
  void* y1;
  void* y2;
  const void* residual;
  int n0, n1;  // split: columns of y0 and y1
};

// Waves per workgroup for a K: 4 up to K = 1024 (one batch of 16 k-steps each), 8
// above (two waves per SIMD still leave each 256 registers for a batch's 32 fragments).
int waves_of(int64_t k) { return k <= 1024 ? 4 : 8; }

// A wave's partial 32 x 32 tile in LDS: [x row][W row], rows padded to 33 floats so
// that both its writes (a lane's 16 values: one W row each, x row = lane) and its reads
// (32 consecutive W rows of one x row) fall in distinct banks.
constexpr int kPartRow = 33;

// k-steps per batch: 16, or 8 where 8 waves of two 32-row blocks of x would outgrow LDS.
template <int MB, int WAVES> constexpr int batch_of() { return MB == 2 && WAVES == 8 ? 8 : 16; }

template <typename T, int MB, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES * kWave) void skinny_linear_kernel(
    Out out, const void* __restrict__ x, const void* __restrict__ w, int m, int n, int k) {
  constexpr int kB = batch_of<MB, WAVES>();
  constexpr int kRow = kB * 32;               // bytes of one x row in a batch
  constexpr int kSlice = MB * 32 * kRow;      // one wave's x batch
  constexpr int kPart = MB * 32 * kPartRow * 4;  // one wave's partial tile
  constexpr int kLds = WAVES * (kSlice > kPart ? kSlice : kPart);
  // Per wave: its batch of x rows (swizzled), then, after the K loop, its partial sums.
  __shared__ __attribute__((aligned(1024))) char lds[kLds];

  constexpr int waves = WAVES;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int tile = blockIdx.x;
  const int n0 = tile * kColTile;

  // This wave's k-steps [beg, beg + cnt): an even partition of the K / 16 over the waves.
  const int steps = k / 16;
  const int beg = wave * steps / waves;
  const int cnt = (wave + 1) * steps / waves - beg;

  // The packed tile's k-step s is the 1 KB at (tile * steps + s) * 1024; this lane's
  // 16 bytes of it at lane * 16.
  const char* wp = static_cast<const char*>(w) +
                   (static_cast<int64_t>(tile) * steps + beg) * 1024 + lane * 16;

  // x batches go to LDS with fully used 1 KB copies (lane i of copy j: x row
  // j * 32/kB + i / (2 kB), 16-byte chunk c = (i % 2kB) ^ (row % 2kB), so the fragment
  // reads below - 32 rows at one chunk each - spread over the banks) and are read back
  // as MFMA fragments; x rows past M read row M - 1.
  char* slice = lds + wave * kSlice;
  const uint32_t slice_lds = lds_address(slice);
  constexpr int kRowsPerCopy = 1024 / kRow;
  constexpr int kCopies = MB * 32 / kRowsPerCopy;
  const int copy_row = lane / (2 * kB);
  const int copy_slot = lane % (2 * kB);

  f32x16 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};
  for (int b0 = 0; b0 < cnt; b0 += kB) {
    const int nb = min(kB, cnt - b0);
    const int st0 = beg + b0;
    const char* xbase = static_cast<const char*>(x) + static_cast<int64_t>(st0) * 32;
    u32x4 a[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) a[u] = load16(wp + static_cast<int64_t>(b0 + min(u, nb - 1)) * 1024);
    // The previous batch's fragment reads are done before its slice is overwritten.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      const int row = j * kRowsPerCopy + copy_row;
      const int chunk = min(copy_slot ^ (row & (2 * kB - 1)), 2 * nb - 1);
      const uint32_t voff = static_cast<uint32_t>((min(row, m - 1) * k + 8 * chunk) * 2);
      copy_to_lds(xbase, voff, slice_lds + j * 1024);
    }
    // Everything of the batch has landed (the weights from HBM arrive last anyway); the
    // explicit wait covers the LDS copies, which the compiler does not count.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // All fragment reads go out before the MFMAs, which then wait only for the weights.
    u32x4 b[MB][kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int c = (2 * u + hsel) ^ (l32 & (2 * kB - 1));
        b[mb][u] = *reinterpret_cast<const u32x4*>(slice + (mb * 32 + l32) * kRow + c * 16);
      }
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      if (u < nb) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] = LinMma<T>::run(a[u], b[mb][u], acc[mb]);
      }
    }
  }

  // Every wave is past its last read of its x slice before the partial sums reuse LDS.
  __syncthreads();
  // Accumulator element r of lane (l32, hsel) is C[W row 8(r/4) + 4 hsel + r%4][x row
  // l32]; it goes to part[wave][mb][x row][W row].
  float* part = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float* dst = part + ((wave * MB + mb) * 32 + l32) * kPartRow + 4 * hsel;
#pragma unroll
    for (int r = 0; r < 16; ++r) dst[8 * (r / 4) + r % 4] = acc[mb][r];
  }
  __syncthreads();

  // The sum over the waves (in order) of C[col][row] of this tile.
  auto total = [&](int row, int col) __attribute__((always_inline)) {
    const float* src = part + ((row / 32) * 32 + row % 32) * kPartRow + col;
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < waves; ++wv) sum += src[wv * MB * 32 * kPartRow];
    return sum;
  };

  if constexpr (EPI == kLinearSwiglu) {
    // 16 output columns per tile: gate col j pairs with up col 16 + j.
    const int nout = n / 2;
    uint16_t* yo = static_cast<uint16_t*>(out.y0);
    for (int e = threadIdx.x; e < MB * 32 * 16; e += WAVES * kWave) {
      const int j = e % 16, row = e / 16;
      const int gcol = tile * 16 + j;
      if (row >= m || gcol >= nout) continue;
      const float g = Elem<T>::round(total(row, j));
      const float u = Elem<T>::round(total(row, 16 + j));
      yo[static_cast<int64_t>(row) * nout + gcol] = LinMma<T>::bits(swiglu_one<T>(g, u));
    }
  } else {
    for (int e = threadIdx.x; e < MB * 32 * kColTile; e += WAVES * kWave) {
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

template <typename T, int MB, int EPI>
hipError_t launch_m(const Out& out, const void* x, const void* w, int m, int n, int k,
                    hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((n + kColTile - 1) / kColTile));
  if (waves_of(k) == 4) {
    skinny_linear_kernel<T, MB, 4, EPI><<<grid, 4 * kWave, 0, stream>>>(out, x, w, m, n, k);
  } else {
    skinny_linear_kernel<T, MB, 8, EPI><<<grid, 8 * kWave, 0, stream>>>(out, x, w, m, n, k);
  }
  return hipGetLastError();
}

template <typename T, int EPI>
hipError_t launch_t(const Out& out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream) {
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  if (m <= 32) return launch_m<T, 1, EPI>(out, x, w, mi, ni, ki, stream);
  return launch_m<T, 2, EPI>(out, x, w, mi, ni, ki, stream);
}

template <int EPI>
hipError_t launch_e(const Out& out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    int dtype, hipStream_t stream) {
  if (dtype == kBF16) return launch_t<bf16_t, EPI>(out, x, w, m, n, k, stream);
  if (dtype == kF16) return launch_t<f16_t, EPI>(out, x, w, m, n, k, stream);
  return hipErrorInvalidValue;
}

// Packs W [n, k] (row-major) into the fragment order: one thread per 16 bytes.
__global__ void pack_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, int64_t n,
                            int64_t k) {
  const int64_t chunks = k / 8;  // 16-byte pieces per row
  const int64_t steps = k / 16;
  const int64_t total = (n + kColTile - 1) / kColTile * kColTile * chunks;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    // i = ((t * steps + s) * 64 + 32 h + r): W row 32 t + r, piece 2 s + h.
    const int64_t l = i % 64, ts = i / 64;
    const int64_t t = ts / steps, s = ts % steps;
    const int64_t row = t * kColTile + (l & 31);
    const int64_t piece = 2 * s + (l >> 5);
    dst[i] = row < n ? src[row * chunks + piece] : uint4{0, 0, 0, 0};
  }
}

}  // namespace

bool skinny_linear_supported(int dtype, int64_t m, int64_t n, int64_t k) {
  if (dtype != kBF16 && dtype != kF16) return false;
  return m >= 1 && m <= kSkinnyMaxRows && n >= 1 && n < (int64_t{1} << 31) / 64 && k >= 64 &&
         k % 64 == 0 && k <= kSkinnyMaxK;
}

int64_t skinny_linear_packed_elements(int64_t n, int64_t k) {
  return (n + kColTile - 1) / kColTile * kColTile * k;
}

hipError_t launch_skinny_linear_pack(void* w_packed, const void* w, int64_t n, int64_t k,
                                     hipStream_t stream) {
  const int64_t total = skinny_linear_packed_elements(n, k) / 8;
  const int blocks = static_cast<int>(std::min<int64_t>((total + 255) / 256, 4096));
  pack_kernel<<<blocks, 256, 0, stream>>>(static_cast<uint4*>(w_packed), static_cast<const uint4*>(w),
                                          n, k);
  return hipGetLastError();
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
