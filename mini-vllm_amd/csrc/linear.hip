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
//  * K is cut into T = 4 ceil(K / 1024) ranges of at most 16 k-steps (16 elements
//    each), one per wave; a wave issues every load of its range before its first MFMA,
//    so a projection's weights are requested up front. K <= 1024 (T = 4): one workgroup
//    of 4 waves per tile of 32 output columns, the waves' 32 x 32 partial sums meeting in
//    LDS, the epilogue in the same launch. K > 1024: T one-wave workgroups per tile (the
//    N = 1024 projections of a decode step would otherwise run on 32 CUs), each
//    writing its fp32 partial tile to a workspace, and a second launch adds the T
//    partials and runs the epilogue - a kernel boundary, because a reduction inside one
//    launch needs device-scope release/acquire fences, which write back and invalidate
//    L2 on this part (measured 2-3x slower). The row-wise second launch also runs the
//    RMSNorm that follows the o and down projections (`residual_rmsnorm`). Both add the
//    T partials in wave order from zero, as the LDS reduction does, and the partition
//    depends on K alone: a column's sum is formed the same way whatever N, M or
//    epilogue, so every fused launch equals the plain one bit for bit.
//  * B = x^T fragments (lane: row l32 of x, the same k): each wave copies its batch of
//    x (32 or 64 rows x its k-steps) from global memory into LDS with the direct-to-LDS
//    load (fully used 1 KB runs; x stays in L2), swizzled, and reads the fragments back
//    from there - the same line-count argument as for W, measured ~2.5 us per projection
//    against fragment loads straight from x. M > 32: a second 32-row block of x shares
//    each W fragment.
//  * epilogues, over the summed tile:
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
//  * residual_rmsnorm: h = T(r + T(x w^T)) and out = RMSNorm(h) (rounded as
//    `rmsnorm_vec_kernel` rounds, with the same lane map and sum order, so bit for bit
//    the unfused pair); one wave (workgroup) per row.

#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "linear.hpp"
#include "paged_attention.hpp"

namespace mvllm {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

constexpr int kColTile = 32;  // output columns per tile (W rows)
constexpr int kSteps = 16;    // most k-steps (16 elements) of one wave, all loaded at once
constexpr int kGroup = 4;     // waves per workgroup
constexpr int kRowBytes = kSteps * 32;  // one x row of a wave's range in LDS

// Waves over K (T): 4 per 1024 elements of K.
int waves_of(int64_t k) { return static_cast<int>(4 * ((k / 16 + 4 * kSteps - 1) / (4 * kSteps))); }

// A wave's partial 32 x 32 tile in LDS: [x row][W row], rows padded to 33 floats so
// that both its writes (a lane's 16 values: one W row each, x row = lane) and its reads
// (32 consecutive W rows of one x row) fall in distinct banks.
constexpr int kPartRow = 33;

struct Out {
  void* y0;
  void* y1;
  void* y2;
  const void* residual;
  int n0, n1;  // split: columns of y0 and y1
};

// One wave's sum over its k-steps of the tile: acc[mb] is the MFMA accumulator of x rows
// 32 mb .. 32 mb + 31. `slice` is the wave's LDS region (MB * 32 x rows of 512 bytes).
template <typename T, int MB>
__device__ __forceinline__ void wave_tile(f32x16 (&acc)[MB], const char* __restrict__ x,
                                          const char* __restrict__ w, char* slice, int m, int k,
                                          int tile, int g, int total_waves) {
  const int lane = threadIdx.x % kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  // This wave's k-steps [beg, beg + cnt) of the K / 16, an even partition over the
  // T waves (1 <= cnt <= 16).
  const int steps = k / 16;
  const int beg = g * steps / total_waves;
  const int cnt = (g + 1) * steps / total_waves - beg;

  // The packed tile's k-step s is the 1 KB at (tile * steps + s) * 1024; this lane's
  // 16 bytes of it at lane * 16.
  const char* wp = w + (static_cast<int64_t>(tile) * steps + beg) * 1024 + lane * 16;
  u32x4 a[kSteps];
#pragma unroll
  for (int u = 0; u < kSteps; ++u) a[u] = load16(wp + static_cast<int64_t>(min(u, cnt - 1)) * 1024);

  // x goes to LDS with fully used 1 KB copies (lane i of copy j: x row 2 j + i / 32,
  // 16-byte chunk c = (i % 32) ^ (row % 32), so the fragment reads below - 32 rows at
  // one chunk each - spread over the banks) and is read back as MFMA fragments; x rows
  // past M read row M - 1.
  const uint32_t slice_lds = lds_address(slice);
  const char* xbase = x + static_cast<int64_t>(beg) * 32;
#pragma unroll
  for (int j = 0; j < MB * 16; ++j) {
    const int row = 2 * j + (lane >> 5);
    const int chunk = min(l32 ^ (row & 31), 2 * cnt - 1);
    const uint32_t voff = static_cast<uint32_t>((min(row, m - 1) * k + 8 * chunk) * 2);
    copy_to_lds(xbase, voff, slice_lds + j * 1024);
  }
  // Everything has landed (the weights from HBM arrive last anyway); the explicit wait
  // covers the LDS copies, which the compiler does not count.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // All fragment reads go out before the MFMAs, which then wait only for the weights.
  u32x4 b[MB][kSteps];
#pragma unroll
  for (int u = 0; u < kSteps; ++u) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int c = (2 * u + hsel) ^ l32;
      b[mb][u] = *reinterpret_cast<const u32x4*>(slice + (mb * 32 + l32) * kRowBytes + c * 16);
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16{};
#pragma unroll
  for (int u = 0; u < kSteps; ++u) {
    if (u < cnt) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = LinMma<T>::run(a[u], b[mb][u], acc[mb]);
    }
  }
}

// The epilogue of one tile over `total(row, col)`, the summed x w^T (fp32).
template <typename T, int MB, int EPI, typename Total>
__device__ __forceinline__ void epilogue(const Out& out, int tile, int m, int n, Total total) {
  const int nthreads = kGroup * kWave;
  if constexpr (EPI == kLinearSwiglu) {
    // 16 output columns per tile: gate col j pairs with up col 16 + j.
    const int nout = n / 2;
    uint16_t* yo = static_cast<uint16_t*>(out.y0);
    for (int e = threadIdx.x; e < MB * 32 * 16; e += nthreads) {
      const int j = e % 16, row = e / 16;
      const int gcol = tile * 16 + j;
      if (row >= m || gcol >= nout) continue;
      const float g = Elem<T>::round(total(row, j));
      const float u = Elem<T>::round(total(row, 16 + j));
      yo[static_cast<int64_t>(row) * nout + gcol] = LinMma<T>::bits(swiglu_one<T>(g, u));
    }
  } else {
    const int n0 = tile * kColTile;
    for (int e = threadIdx.x; e < MB * 32 * kColTile; e += nthreads) {
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

// K <= 1024: one workgroup of 4 waves per tile, reduction in LDS, epilogue in place.
template <typename T, int MB, int EPI>
__global__ __launch_bounds__(kGroup * kWave) void skinny_linear_kernel(
    Out out, const void* __restrict__ x, const void* __restrict__ w, int m, int n, int k) {
  constexpr int kSlice = MB * 32 * kRowBytes;
  __shared__ __attribute__((aligned(1024))) char lds[kGroup * kSlice];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  f32x16 acc[MB];
  wave_tile<T, MB>(acc, static_cast<const char*>(x), static_cast<const char*>(w),
                   lds + wave * kSlice, m, k, blockIdx.x, wave, kGroup);

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
  // The sum over the waves (in order, from zero) of C[col][row] of this tile.
  auto total = [&](int row, int col) __attribute__((always_inline)) {
    const float* src = part + row * kPartRow + col;
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kGroup; ++wv) sum += src[wv * MB * 32 * kPartRow];
    return sum;
  };
  epilogue<T, MB, EPI>(out, blockIdx.x, m, n, total);
}

// K > 1024: wave g = blockIdx.y of the T writes its fp32 partial tile to
// partials[tile][g][x row][col] (MB * 32 x rows). The waves share nothing, so each is a
// workgroup of its own: the weights are then requested from as many CUs as there are
// waves (256 and 384 for the o and down projections of a decode step), and a CU pulls
// only so many bytes per microsecond (one-wave workgroups against four: 7.7 -> 7.0 us
// for the o projection with its reduction, 8.6 -> 8.2 for down).
template <typename T, int MB>
__global__ __launch_bounds__(kWave) void skinny_partial_kernel(
    float* __restrict__ partials, const void* __restrict__ x, const void* __restrict__ w, int m,
    int k, int total_waves) {
  constexpr int kSlice = MB * 32 * kRowBytes;
  __shared__ __attribute__((aligned(1024))) char lds[kSlice];
  const int lane = threadIdx.x % kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int g = blockIdx.y;
  f32x16 acc[MB];
  wave_tile<T, MB>(acc, static_cast<const char*>(x), static_cast<const char*>(w), lds, m, k,
                   blockIdx.x, g, total_waves);
  float* dst = partials + (static_cast<int64_t>(blockIdx.x) * total_waves + g) * (MB * 32 * kColTile);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    float* row = dst + (mb * 32 + l32) * kColTile + 4 * hsel;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      *reinterpret_cast<f32x4*>(row + 8 * q) =
          f32x4{acc[mb][4 * q], acc[mb][4 * q + 1], acc[mb][4 * q + 2], acc[mb][4 * q + 3]};
    }
  }
}

// Adds T partial float4s, `stride` floats apart, in order from zero: eight loads in
// flight at a time, the additions sequential (the LDS reduction's order).
__device__ __forceinline__ f32x4 sum_partials(const float* __restrict__ src, int64_t stride,
                                              int total_waves) {
  f32x4 sum = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  int g = 0;
  for (; g + 8 <= total_waves; g += 8) {
    f32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const f32x4*>(src + (g + i) * stride);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] = sum[e] + v[i][e];
    }
  }
  for (; g < total_waves; ++g) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + g * stride);
#pragma unroll
    for (int e = 0; e < 4; ++e) sum[e] = sum[e] + v[e];
  }
  return sum;
}

// K > 1024, tile epilogues: one workgroup per tile adds the T partials in wave order
// (four columns per thread) into LDS, then runs the epilogue.
template <typename T, int MB, int EPI>
__global__ __launch_bounds__(kGroup * kWave) void skinny_reduce_kernel(
    Out out, const float* __restrict__ partials, int m, int n, int total_waves) {
  constexpr int kTile = MB * 32 * kColTile;
  __shared__ float tot[kTile];
  const float* base = partials + static_cast<int64_t>(blockIdx.x) * total_waves * kTile;
  for (int e4 = threadIdx.x; e4 < kTile / 4; e4 += kGroup * kWave) {
    *reinterpret_cast<f32x4*>(tot + 4 * e4) = sum_partials(base + 4 * e4, kTile, total_waves);
  }
  __syncthreads();
  auto total = [&](int row, int col) __attribute__((always_inline)) {
    return tot[row * kColTile + col];
  };
  epilogue<T, MB, EPI>(out, blockIdx.x, m, n, total);
}

// K > 1024, residual + RMSNorm: one wave (workgroup) per x row, lane r holding 8-column
// chunks r, r + 64, ... (the lane map of rmsnorm_vec_kernel<T, 64, kCh>): h = T(r +
// T(sum)), then out = T(T(h * inv) * weight) with inv from the lane-ordered fma sum of
// squares reduced by group_sum<64>, as that kernel computes it. The residual and weight
// chunks, which do not depend on the partials, are requested first; then all of a
// lane's partial loads for kB waves at a time go out together (kCh x 2 x kB float4s; kB
// divides T), so the kernel waits on one memory round trip instead of three.
template <typename T, int MB, int kCh, int kB>
__global__ __launch_bounds__(kWave) void skinny_reduce_norm_kernel(
    void* __restrict__ h_out, void* __restrict__ normed, const float* __restrict__ partials,
    const void* __restrict__ residual, const void* __restrict__ norm_weight, int m, int n,
    int total_waves, float eps) {
  constexpr int64_t kTile = MB * 32 * kColTile;
  const int row = blockIdx.x;
  const int r = threadIdx.x;
  const int64_t tile_stride = static_cast<int64_t>(total_waves) * kTile;
  const int chunks = n / 8;
  const char* res = static_cast<const char*>(residual) + static_cast<int64_t>(row) * n * 2;
  char* hrow = static_cast<char*>(h_out) + static_cast<int64_t>(row) * n * 2;

  const char* wr = static_cast<const char*>(norm_weight);
  const float* src[kCh];
  u32x4 res_v[kCh], w_v[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int chunk = min(r + c * kWave, chunks - 1);
    const int col = chunk * 8;
    src[c] = partials + (col / kColTile) * tile_stride + row * kColTile + col % kColTile;
    res_v[c] = load16(res + col * 2);
    w_v[c] = load16(wr + chunk * 16);
  }
  f32x4 sum[kCh][2];
#pragma unroll
  for (int c = 0; c < kCh; ++c) sum[c][0] = sum[c][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int g0 = 0; g0 < total_waves; g0 += kB) {
    f32x4 v[kCh][2][kB];
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int64_t off = static_cast<int64_t>(g0 + i) * kTile;
#pragma unroll
      for (int c = 0; c < kCh; ++c) {
        v[c][0][i] = *reinterpret_cast<const f32x4*>(src[c] + off);
        v[c][1][i] = *reinterpret_cast<const f32x4*>(src[c] + off + 4);
      }
    }
    // Every load of the round is issued before the first addition (left to itself the
    // scheduler interleaves them, one round trip per wave's partial).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kB; ++i) {
#pragma unroll
      for (int c = 0; c < kCh; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum[c][0][e] = sum[c][0][e] + v[c][0][i][e];
          sum[c][1][e] = sum[c][1][e] + v[c][1][i][e];
        }
      }
    }
  }

  u32x4 held[kCh];
  float sumsq = 0.0f;
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int chunk = r + c * kWave;
    if (chunk < chunks) {
      const int col = chunk * 8;
      float rf[8];
      Chunk<T>::unpack(res_v[c], rf);
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = Elem<T>::round(rf[e] + Elem<T>::round(sum[c][e / 4][e % 4]));
      u32x4 hv;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        hv[e / 2] = static_cast<uint32_t>(LinMma<T>::bits(f[e])) |
                    (static_cast<uint32_t>(LinMma<T>::bits(f[e + 1])) << 16);
      }
      held[c] = hv;
      store16(hrow + col * 2, hv);
#pragma unroll
      for (int e = 0; e < 8; ++e) sumsq = fmaf(f[e], f[e], sumsq);
    }
  }
  sumsq = group_sum<kWave>(sumsq);
  const float inv = rsqrtf(sumsq / static_cast<float>(n) + eps);
  char* orow = static_cast<char*>(normed) + static_cast<int64_t>(row) * n * 2;
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const int chunk = r + c * kWave;
    if (chunk < chunks) {
      float f[8], wf[8];
      Chunk<T>::unpack(held[c], f);
      Chunk<T>::unpack(w_v[c], wf);
      u32x4 res_v;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float o2[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float normalized = Elem<T>::round(__fmul_rn(f[e + q], inv));
          o2[q] = __fmul_rn(normalized, wf[e + q]);
        }
        res_v[e / 2] = static_cast<uint32_t>(LinMma<T>::bits(o2[0])) |
                       (static_cast<uint32_t>(LinMma<T>::bits(o2[1])) << 16);
      }
      store16(orow + chunk * 16, res_v);
    }
  }
}

int row_blocks(int64_t m) { return m <= 32 ? 1 : 2; }

template <typename T, int MB, int EPI>
hipError_t launch_m(const Out& out, const void* x, const void* w, int m, int n, int k,
                    void* workspace, hipStream_t stream) {
  const unsigned tiles = static_cast<unsigned>((n + kColTile - 1) / kColTile);
  const int t_waves = waves_of(k);
  if (t_waves == kGroup) {
    skinny_linear_kernel<T, MB, EPI><<<tiles, kGroup * kWave, 0, stream>>>(out, x, w, m, n, k);
    return hipGetLastError();
  }
  float* partials = static_cast<float*>(workspace);
  skinny_partial_kernel<T, MB><<<dim3(tiles, t_waves), kWave, 0, stream>>>(
      partials, x, w, m, k, t_waves);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  skinny_reduce_kernel<T, MB, EPI><<<tiles, kGroup * kWave, 0, stream>>>(out, partials, m, n, t_waves);
  return hipGetLastError();
}

template <typename T, int EPI>
hipError_t launch_t(const Out& out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    void* workspace, hipStream_t stream) {
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  if (row_blocks(m) == 1) return launch_m<T, 1, EPI>(out, x, w, mi, ni, ki, workspace, stream);
  return launch_m<T, 2, EPI>(out, x, w, mi, ni, ki, workspace, stream);
}

template <int EPI>
hipError_t launch_e(const Out& out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    int dtype, void* workspace, hipStream_t stream) {
  if (dtype == kBF16) return launch_t<bf16_t, EPI>(out, x, w, m, n, k, workspace, stream);
  if (dtype == kF16) return launch_t<f16_t, EPI>(out, x, w, m, n, k, workspace, stream);
  return hipErrorInvalidValue;
}

template <typename T, int MB>
hipError_t launch_norm_m(void* h_out, void* normed, const void* x, const void* w, const void* residual,
                         const void* norm_weight, int m, int n, int k, float eps, void* workspace,
                         hipStream_t stream) {
  const unsigned tiles = static_cast<unsigned>((n + kColTile - 1) / kColTile);
  const int t_waves = waves_of(k);
  float* partials = static_cast<float*>(workspace);
  skinny_partial_kernel<T, MB><<<dim3(tiles, t_waves), kWave, 0, stream>>>(
      partials, x, w, m, k, t_waves);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const unsigned rows = static_cast<unsigned>(m);
  const int per_lane = n / 8 / kWave;
  // kB: the most waves' partials a lane loads at once that divides T (a multiple of
  // 4), at most 32 / kCh of them (kCh x 2 x kB float4s in registers).
  auto run = [&](auto ch, auto b) {
    skinny_reduce_norm_kernel<T, MB, decltype(ch)::value, decltype(b)::value><<<rows, kWave, 0, stream>>>(
        h_out, normed, partials, residual, norm_weight, m, n, t_waves, eps);
  };
  using C2 = std::integral_constant<int, 2>;
  using C4 = std::integral_constant<int, 4>;
  using C8 = std::integral_constant<int, 8>;
  using B4 = std::integral_constant<int, 4>;
  using B8 = std::integral_constant<int, 8>;
  using B12 = std::integral_constant<int, 12>;
  using B16 = std::integral_constant<int, 16>;
  if (per_lane <= 2) {
    if (t_waves % 16 == 0) run(C2{}, B16{});
    else if (t_waves % 12 == 0) run(C2{}, B12{});
    else if (t_waves % 8 == 0) run(C2{}, B8{});
    else run(C2{}, B4{});
  } else if (per_lane <= 4) {
    if (t_waves % 8 == 0) run(C4{}, B8{});
    else run(C4{}, B4{});
  } else {
    run(C8{}, B4{});
  }
  return hipGetLastError();
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

bool skinny_residual_rmsnorm_supported(int dtype, int64_t m, int64_t n, int64_t k) {
  return skinny_linear_supported(dtype, m, n, k) && waves_of(k) > kGroup && n % 512 == 0 &&
         n <= 4096;
}

uint64_t skinny_linear_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  const int t_waves = waves_of(k);
  if (t_waves == kGroup) return 0;
  const uint64_t tiles = static_cast<uint64_t>((n + kColTile - 1) / kColTile);
  return tiles * t_waves * row_blocks(m) * 32 * kColTile * sizeof(float);
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
                                int64_t k, int dtype, void* workspace, hipStream_t stream) {
  return launch_e<kLinearPlain>(Out{y, nullptr, nullptr, nullptr, 0, 0}, x, w, m, n, k, dtype,
                                workspace, stream);
}

hipError_t launch_skinny_linear_split(void* y0, void* y1, void* y2, const void* x, const void* w,
                                      int64_t m, int64_t n0, int64_t n1, int64_t n2, int64_t k,
                                      int dtype, void* workspace, hipStream_t stream) {
  return launch_e<kLinearSplit>(Out{y0, y1, y2, nullptr, static_cast<int>(n0), static_cast<int>(n1)},
                                x, w, m, n0 + n1 + n2, k, dtype, workspace, stream);
}

hipError_t launch_skinny_linear_residual(void* y, const void* x, const void* w, const void* residual,
                                         int64_t m, int64_t n, int64_t k, int dtype,
                                         void* workspace, hipStream_t stream) {
  return launch_e<kLinearResidual>(Out{y, nullptr, nullptr, residual, 0, 0}, x, w, m, n, k, dtype,
                                   workspace, stream);
}

hipError_t launch_skinny_linear_swiglu(void* y, const void* x, const void* w_gate_up, int64_t m,
                                       int64_t n_out, int64_t k, int dtype, void* workspace,
                                       hipStream_t stream) {
  return launch_e<kLinearSwiglu>(Out{y, nullptr, nullptr, nullptr, 0, 0}, x, w_gate_up, m, 2 * n_out,
                                 k, dtype, workspace, stream);
}

hipError_t launch_skinny_linear_residual_rmsnorm(void* h_out, void* normed, const void* x,
                                                 const void* w, const void* residual,
                                                 const void* norm_weight, int64_t m, int64_t n,
                                                 int64_t k, float eps, int dtype, void* workspace,
                                                 hipStream_t stream) {
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  if (dtype == kBF16) {
    return row_blocks(m) == 1
               ? launch_norm_m<bf16_t, 1>(h_out, normed, x, w, residual, norm_weight, mi, ni, ki, eps, workspace, stream)
               : launch_norm_m<bf16_t, 2>(h_out, normed, x, w, residual, norm_weight, mi, ni, ki, eps, workspace, stream);
  }
  if (dtype == kF16) {
    return row_blocks(m) == 1
               ? launch_norm_m<f16_t, 1>(h_out, normed, x, w, residual, norm_weight, mi, ni, ki, eps, workspace, stream)
               : launch_norm_m<f16_t, 2>(h_out, normed, x, w, residual, norm_weight, mi, ni, ki, eps, workspace, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mvllm
