// Prefill projections: y[M, N] = x[M, K] w[N, K]^T for prefill-sized x (hundreds to
// thousands of token rows), bf16 or fp16 in and out, fp32 accumulate, one rounding.
//
// The reference runs every projection through torch's matmul (model/basics.py linear);
// at a 2048-token prefill of Qwen3-0.6B the four projections per layer are M = 2048
// GEMMs with N x K of 4096 x 1024 (q/k/v), 1024 x 2048 (o), 6144 x 1024 (gate/up) and
// 1024 x 3072 (down). The vendor BLAS runs the N = 1024 ones at 17-24% of the bf16 MFMA
// peak on this GPU: with large macro tiles they make few tiles and most CUs sit idle.
// Here the tile is chosen from the shape so the grid fills the CUs.
//
// Design (this library's own):
//  * output tile BM x BN (256 x 128, 128 x 128 or 128 x 64, chosen from the shape so
//    that the grid fills the CUs in whole rounds: `pick_config`), K in steps of BK =
//    64; waves in a WM x 2 arrangement, each a block of v_mfma_f32_32x32x16 tiles:
//    C^T = W X^T, so the A operand is rows of W (output columns) and the B operand
//    rows of x (tokens), and each lane ends up holding four consecutive output columns
//    of one token row (8-byte stores);
//  * both operands staged by direct-to-LDS loads (global_load_lds_dwordx4, 1 KB per
//    wave instruction = 8 rows of 128 bytes), two or three stages in flight: the
//    copies of k-step t + STAGES - 1 are issued while t is computed, one barrier per
//    k-step;
//  * a 128-byte LDS row holds 8 chunks of 16 bytes; logical chunk c of row r sits at
//    chunk c ^ ((r >> 1) & 7), so the 16 lanes that one LDS cycle serves (16 rows, one
//    chunk each) fall in 16 distinct bank groups;
//  * the fragments of k-substep s + 1 are read while substep s's MFMAs run;
//  * workgroups are numbered so that each XCD takes a contiguous block of tiles
//    (round-robin dispatch puts workgroup b on XCD b % 8): tiles that share x rows
//    share that XCD's L2;
//  * token rows past M read row M - 1 and are not stored; N must be a multiple of 64
//    (128 for the wider tiles) and K of 64 (the host checks).
//
// Measured against the vendor BLAS at M = 2048 on random bf16 data (graph replays, us):
// q/k/v 26.4 against 21.4, o 17.5 against 15.5, gate/up 45.5 against 28.5, down 23.3
// against 20.8 (constant-valued inputs run ~20% faster and misled a first comparison).
// Slower everywhere, so the model keeps its prefill projections on the BLAS
// (ops.NOT_YET_FASTER); the kernel stays, tested, for the work that would close the
// gap (larger per-wave tiles need more of LDS bandwidth than this layout leaves).

#include "common.hpp"
#include "gemm.hpp"

namespace mvllm {

namespace {

typedef __bf16 gbf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 gf16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct GemmMma;
template <> struct GemmMma<bf16_t> {
  __device__ static f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gbf16x8_t, a),
                                                   __builtin_bit_cast(gbf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct GemmMma<f16_t> {
  __device__ static f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(gf16x8_t, a),
                                                  __builtin_bit_cast(gf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) {
    return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
  }
};

constexpr int kBK = 64;      // K per stage (128-byte rows)
constexpr int kRowBytes = kBK * 2;

// The XCD-contiguous tile order: workgroup b -> tile index.
__device__ __forceinline__ int tile_of(int b, int tiles) {
  constexpr int kXcds = 8;
  if (tiles % kXcds != 0) return b;
  return (b % kXcds) * (tiles / kXcds) + b / kXcds;
}

// BM token rows x BN output columns per workgroup, STAGES k-steps of LDS in flight;
// WM x 2 waves, wave (wm, wn) computing BM/WM x BN/2.
template <typename T, int BM, int BN, int STAGES, int WM>
__global__ __launch_bounds__(WM * 2 * kWave) void gemm_kernel(void* __restrict__ y,
                                                              const void* __restrict__ x,
                                                              const void* __restrict__ w, int m,
                                                              int n, int k) {
  constexpr int kWaves = WM * 2;
  constexpr int kThr = kWaves * kWave;
  constexpr int kWaveM = BM / WM;              // token rows per wave
  constexpr int kWaveN = BN / 2;               // output columns per wave
  constexpr int kMB = kWaveM / 32;             // 32-row MFMA blocks per wave
  constexpr int kNB = kWaveN / 32;             // 32-column MFMA blocks per wave
  constexpr int kXBytes = BM * kRowBytes;      // one stage of x
  constexpr int kWBytes = BN * kRowBytes;      // one stage of W
  constexpr int kXCopies = kXBytes / (kThr * 16);
  constexpr int kWCopies = kWBytes / (kThr * 16);
  constexpr int kCopies = kXCopies + kWCopies;  // vector-memory ops of one stage per lane
  constexpr int kSub = kBK / 16;                // MFMA k-substeps per stage
  static_assert(kMB >= 1 && kNB >= 1 && kXCopies >= 1 && kWCopies >= 1 && STAGES >= 2, "tile");
  __shared__ __align__(1024) char lds[STAGES * (kXBytes + kWBytes)];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform: LDS bases are scalar
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int wm = wave % WM;  // token block of the tile
  const int wn = wave / WM;  // column half

  const int n_tiles = n / BN;
  const int tiles = n_tiles * ((m + BM - 1) / BM);
  const int t = tile_of(static_cast<int>(blockIdx.x), tiles);
  const int m0 = (t / n_tiles) * BM;
  const int n0 = (t % n_tiles) * BN;
  const int ksteps = k / kBK;

  const char* xg = static_cast<const char*>(x);
  const char* wg = static_cast<const char*>(w);
  const int64_t x_row = static_cast<int64_t>(k) * 2;  // bytes per row of x and of W

  // Copy j of this wave fills 1 KB of a stage, rows 8 (j kWaves + wave) .. +7: lane ->
  // row 8 (j kWaves + wave) + lane / 8, chunk position lane % 8 holding logical chunk
  // (lane % 8) ^ ((row >> 1) & 7).
  uint32_t x_off[kXCopies], w_off[kWCopies];
#pragma unroll
  for (int j = 0; j < kXCopies; ++j) {
    const int row = 8 * (j * kWaves + wave) + lane / 8;
    const int chunk = (lane % 8) ^ ((row >> 1) & 7);
    const int grow = min(m0 + row, m - 1);
    x_off[j] = static_cast<uint32_t>(grow * x_row + chunk * 16);
  }
#pragma unroll
  for (int j = 0; j < kWCopies; ++j) {
    const int row = 8 * (j * kWaves + wave) + lane / 8;
    const int chunk = (lane % 8) ^ ((row >> 1) & 7);
    w_off[j] = static_cast<uint32_t>((n0 + row) * x_row + chunk * 16);
  }
  auto stage_x = [&](int s) __attribute__((always_inline)) -> char* { return lds + s * (kXBytes + kWBytes); };
  auto stage_w = [&](int s) __attribute__((always_inline)) -> char* { return stage_x(s) + kXBytes; };
  auto issue = [&](int kt, int s) __attribute__((always_inline)) {
    const char* xb = xg + static_cast<int64_t>(kt) * kRowBytes;
    const char* wb = wg + static_cast<int64_t>(kt) * kRowBytes;
    const uint32_t xd = lds_address(stage_x(s));
    const uint32_t wd = lds_address(stage_w(s));
#pragma unroll
    for (int j = 0; j < kXCopies; ++j) copy_to_lds(xb, x_off[j], xd + (j * kWaves + wave) * 8 * kRowBytes);
#pragma unroll
    for (int j = 0; j < kWCopies; ++j) copy_to_lds(wb, w_off[j], wd + (j * kWaves + wave) * 8 * kRowBytes);
  };

  // Fragment reads: operand row r (within the stage), k-substep ks: logical chunk
  // 2 ks + hsel at position (2 ks + hsel) ^ ((r >> 1) & 7). The swizzle term of
  // row 32 i + l32 is that of l32.
  const int swz = (l32 >> 1) & 7;
  auto frag = [&](const char* base, int r, int ks) __attribute__((always_inline)) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(base + r * kRowBytes + (((2 * ks + hsel) ^ swz) * 16));
  };

  f32x16 acc[kNB][kMB];
#pragma unroll
  for (int i = 0; i < kNB; ++i) {
#pragma unroll
    for (int j = 0; j < kMB; ++j) acc[i][j] = f32x16{};
  }

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(min(s, ksteps - 1), s);
  for (int kt = 0; kt < ksteps; ++kt) {
    const int s = kt % STAGES;
    // This wave's copies of k-step kt have landed (the next STAGES - 2 may be in
    // flight); the barrier publishes every wave's and retires k-step kt - 1's reads.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCopies * (STAGES - 2)) : "memory");
    asm volatile("s_barrier" ::: "memory");
    issue(min(kt + STAGES - 1, ksteps - 1), (kt + STAGES - 1) % STAGES);
    const char* xs = stage_x(s) + wm * kWaveM * kRowBytes;
    const char* ws = stage_w(s) + wn * kWaveN * kRowBytes;
    // Substep ks + 1's fragments are read while substep ks's MFMAs run.
    u32x4 a[2][kNB], b[2][kMB];
#pragma unroll
    for (int i = 0; i < kNB; ++i) a[0][i] = frag(ws, 32 * i + l32, 0);
#pragma unroll
    for (int j = 0; j < kMB; ++j) b[0][j] = frag(xs, 32 * j + l32, 0);
#pragma unroll
    for (int ks = 0; ks < kSub; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < kSub) {
#pragma unroll
        for (int i = 0; i < kNB; ++i) a[cur ^ 1][i] = frag(ws, 32 * i + l32, ks + 1);
#pragma unroll
        for (int j = 0; j < kMB; ++j) b[cur ^ 1][j] = frag(xs, 32 * j + l32, ks + 1);
      }
#pragma unroll
      for (int i = 0; i < kNB; ++i) {
#pragma unroll
        for (int j = 0; j < kMB; ++j) acc[i][j] = GemmMma<T>::run(a[cur][i], b[cur][j], acc[i][j]);
      }
    }
  }
  // No copy may still be writing LDS when the workgroup ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // acc[i][j] element r: output column n0 + wn kWaveN + 32 i + 8 (r / 4) + 4 hsel + r % 4
  // of token row m0 + wm kWaveM + 32 j + l32.
  char* yg = static_cast<char*>(y);
#pragma unroll
  for (int j = 0; j < kMB; ++j) {
    const int row = m0 + wm * kWaveM + 32 * j + l32;
    if (row >= m) continue;
#pragma unroll
    for (int i = 0; i < kNB; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + wn * kWaveN + 32 * i + 8 * q + 4 * hsel;
        const f32x16& c = acc[i][j];
        *reinterpret_cast<u32x2*>(yg + (static_cast<int64_t>(row) * n + col) * 2) =
            u32x2{GemmMma<T>::pack2(c[4 * q], c[4 * q + 1]), GemmMma<T>::pack2(c[4 * q + 2], c[4 * q + 3])};
      }
    }
  }
}

// Tile configurations: 0 = 256 x 128 (8 waves, each 64 x 64; three stages, 144 KB of
// LDS: one workgroup per CU), 1 = 128 x 128 (4 waves of 64 x 64; two stages, 64 KB: two
// workgroups per CU), 2 = 128 x 64 (4 waves of 64 x 32; three stages, 72 KB: two per
// CU). The largest is taken when its tiles fill whole rounds of the CUs, else 128 x 128
// when that gives two or more tiles per CU, else 128 x 64. Measured at M = 2048 on
// constant-valued bf16 inputs (us, the three configurations): N x K = 4096 x 1024:
// 21.7 / 22.0 / 28.7; 6144 x 1024: 36.5 / 35.0 / 41.5; 1024 x 2048: 28.6 / 22.2 / 16.1;
// 1024 x 3072: 39.5 / 31.9 / 22.3.
int pick_config(int64_t m, int64_t n, int cus) {
  const int64_t t0 = ((m + 255) / 256) * (n / 128);
  if (n % 128 == 0 && t0 >= cus && t0 % cus == 0) return 0;
  if (n % 128 == 0 && ((m + 127) / 128) * (n / 128) >= 2 * static_cast<int64_t>(cus)) return 1;
  return 2;
}

template <typename T>
hipError_t launch_gemm_t(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                         int cus, int forced, hipStream_t stream) {
  int pick = pick_config(m, n, cus);
  if (forced >= 0 && forced < 3 && (forced == 2 || n % 128 == 0)) pick = forced;
  const int bm = pick == 0 ? 256 : 128, bn = pick == 2 ? 64 : 128;
  const unsigned tiles = static_cast<unsigned>(((m + bm - 1) / bm) * (n / bn));
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  switch (pick) {
    case 0: gemm_kernel<T, 256, 128, 3, 4><<<tiles, 512, 0, stream>>>(y, x, w, mi, ni, ki); break;
    case 1: gemm_kernel<T, 128, 128, 2, 2><<<tiles, 256, 0, stream>>>(y, x, w, mi, ni, ki); break;
    default: gemm_kernel<T, 128, 64, 3, 2><<<tiles, 256, 0, stream>>>(y, x, w, mi, ni, ki); break;
  }
  return hipGetLastError();
}

}  // namespace

bool gemm_supported(int dtype, int64_t m, int64_t n, int64_t k) {
  if (dtype != kBF16 && dtype != kF16) return false;
  // int32 byte offsets inside the kernel: every operand under 2 GiB
  return m >= 1 && n >= 64 && n % 64 == 0 && k >= kBK && k % kBK == 0 &&
         m * k * 2 < (int64_t{1} << 31) && n * k * 2 < (int64_t{1} << 31) &&
         m * n < (int64_t{1} << 31);
}

hipError_t launch_gemm(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                       int dtype, int cus, int config, hipStream_t stream) {
  if (dtype == kBF16) return launch_gemm_t<bf16_t>(y, x, w, m, n, k, cus, config, stream);
  if (dtype == kF16) return launch_gemm_t<f16_t>(y, x, w, m, n, k, cus, config, stream);
  return hipErrorInvalidValue;
}

}  // namespace mvllm
