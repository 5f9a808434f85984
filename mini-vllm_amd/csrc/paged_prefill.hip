// Chunked paged prefill attention on CDNA4 matrix cores.
//
// Behaviour follows the reference's paged_prefill_kernel (csrc/paged_attention.cu:
// 306-472): for every sequence computing L > 1 query tokens, query r (0-based in the
// chunk) attends causally to keys [0, S - L + r] of its S = context_lens[s] keys, the
// keys being gathered through the sequence's block table. GQA: query head h reads kv
// head h / (H_q / H_k).
//
// Design (this library's own):
//
//  * workgroup = (128 query positions, kv head, HC = 2 (or 1) query heads of its GQA
//    group); wave w owns 32 positions for all HC heads, so every K or V fragment read
//    from LDS feeds HC MFMAs. The waves share the K/V tiles of their kv head,
//    page-gathered from HBM into LDS 64 keys at a time, double buffered; page ids are
//    fetched two tiles ahead and K/V one tile ahead, so the tile loop never waits on a
//    block-table read.
//  * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_{bf16,f16}:
//    a lane then owns one query column and 16 keys per 32-key block, so the softmax
//    row max is an in-lane max plus one xor-32 exchange.
//  * O^T = V^T P^T on the same MFMA. The P^T operand comes straight from the score
//    accumulators (converted to bf16/fp16); the MFMA's reduction axis is keys, so the
//    accumulator's key order is used as-is and V^T is read with the same key
//    permutation. V is transposed on its way into LDS.
//  * online softmax in fp32, log2 domain; causal masking only on tiles that cross the
//    diagonal; tiles past a wave's last visible key are skipped.
//  * fp8-e4m3 pools are dequantised (x * per-(page, kv head) scale) while staging
//    into LDS, and the MFMAs run in the query's 16-bit type.
//
// MFMA 32x32x16 operand layouts (lane l, l32 = l % 32, h = l / 32):
//   A[m][k]: lane holds m = l32, k = 8h .. 8h+7
//   B[k][n]: lane holds n = l32, k = 8h .. 8h+7
//   C[m][n]: lane holds n = l32, m = 8j + 4h + i for j, i in 0..3 (register 4j + i)

#include "common.hpp"
#include "paged_attention.hpp"

namespace mvllm {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTileKeys = 64;
constexpr int kThreadsMax = 256;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct Mma;
template <> struct Mma<bf16_t> {
  __device__ static f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Mma<f16_t> {
  __device__ static f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) {
    return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
  }
};

// Eight consecutive pool elements -> eight 16-bit elements of the compute type.
template <typename TQ, typename TKV> struct Stage;
template <typename TQ> struct Stage<TQ, TQ> {
  static constexpr int kSrcBytes = 16;
  __device__ static u32x4 load(const char* src, float) { return load16(src); }
};
template <typename TQ> struct Stage<TQ, fp8_t> {
  static constexpr int kSrcBytes = 8;
  __device__ static u32x4 load(const char* src, float scale) {
    const u32x2 w = *reinterpret_cast<const u32x2*>(src);
    u32x4 out;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
      out[2 * i] = Mma<TQ>::pack2(lo[0] * scale, lo[1] * scale);
      out[2 * i + 1] = Mma<TQ>::pack2(hi[0] * scale, hi[1] * scale);
    }
    return out;
  }
};

}  // namespace

template <typename TQ, typename TKV, int D, int HC>
__global__ __launch_bounds__(kThreadsMax) void paged_prefill_kernel(const PagedParams p) {
  constexpr int kKStride = D + 8;            // K tile row, 16-bit elements (16 B pad)
  constexpr int kVStride = kTileKeys + 4;    // V^T tile row, 16-bit elements (8 B pad)
  constexpr int kKSteps = D / 16;            // MFMA k-steps over the head dim
  constexpr int kDBlocks = D / 32;           // 32-row blocks of O^T
  constexpr int kKUnits = kTileKeys * D / 8 / kThreadsMax;  // 8-element K units per thread
  constexpr int kVPairs = 16 * (D / 8);                     // (key quad, dim octet) pairs
  constexpr int kVUnits = (kVPairs + kThreadsMax - 1) / kThreadsMax;
  constexpr int kElemBytes = Elem<TKV>::kBytes;
  constexpr bool kFp8 = kElemBytes == 1;
  constexpr int kWaves = kThreadsMax / kWave;  // 4 waves x 32 query positions
  static_assert(kKUnits >= 1, "head dim too small for the staging map");

  __shared__ __align__(16) uint16_t k_lds[2][kTileKeys * kKStride];
  __shared__ __align__(16) uint16_t v_lds[2][D * kVStride];

  // Grid (head chunks, sequences, query tiles), the query tile slowest and reversed:
  // workgroups are dispatched in index order, so the last (longest) query tiles of all
  // sequences start first and the short ones fill in behind them.
  const int seq = blockIdx.y;
  const int query_len = p.seq_lens[seq];
  if (query_len <= 1) return;  // a decode step: the decode kernel has it
  const int qtiles = (query_len + 32 * kWaves - 1) / (32 * kWaves);
  const int qt = static_cast<int>(gridDim.z) - 1 - static_cast<int>(blockIdx.z);
  if (qt < 0 || qt >= qtiles) return;
  const int qb = qt * 32 * kWaves;

  const int group = p.hq / p.hk;
  const int chunks = group / HC;
  const int kvh = blockIdx.x / chunks;
  const int head0 = kvh * group + (blockIdx.x % chunks) * HC;

  const int context = p.context_lens[seq];
  const int offset = context - query_len;  // causal offset S - L
  const int row_base = p.cu_seqlens_q[seq];
  const int32_t* table = p.block_tables + static_cast<int64_t>(seq) * p.max_blocks;

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;

  // Workgroup-wide key range, and this wave's.
  const int wg_last = min(qb + 32 * kWaves, query_len);
  const int kv_end = offset + wg_last;  // keys [0, kv_end) are visible to someone here
  const int ntiles = (kv_end + kTileKeys - 1) / kTileKeys;
  const int w_first = qb + 32 * wave;                  // first local query of this wave
  const bool w_active = w_first < query_len;
  const int w_kv_end = offset + min(w_first + 32, query_len);  // no query of the wave looks past
  const int w_kv_full = offset + w_first + 1;          // below this, every query sees the key

  // This lane's query (column l32 of the wave's tile), the same for its HC heads.
  const int my_local = w_first + l32;
  const bool my_valid = my_local < query_len;
  const int my_visible = offset + my_local + 1;

  // Q^T operands: lane holds q[row][head0 + h][16*ks + 8*hsel .. +7] for each k-step.
  u32x4 qop[HC][kKSteps];
  {
    const int local = min(w_active ? (my_valid ? my_local : w_first) : 0, query_len - 1);
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      const int64_t qrow = static_cast<int64_t>(row_base + local) * p.hq + head0 + h;
      const char* qp = static_cast<const char*>(p.q) + (qrow * D + 8 * hsel) * 2;
#pragma unroll
      for (int ks = 0; ks < kKSteps; ++ks) qop[h][ks] = load16(qp + ks * 32);
    }
  }

  f32x16 o[HC][kDBlocks];
  float m_run[HC], l_run[HC];
#pragma unroll
  for (int h = 0; h < HC; ++h) {
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) o[h][db] = f32x16{};
    m_run[h] = -INFINITY;
    l_run[h] = 0.0f;
  }
  const float score_scale = p.scale * kLog2e;

  const char* kpool = static_cast<const char*>(p.k_pool);
  const char* vpool = static_cast<const char*>(p.v_pool);

  // ---- staging. Each thread stages kKUnits 8-element K units and kVUnits (4 keys x 8
  // dims) V units per tile. Their page ids (and fp8 scales) are fetched two tiles
  // ahead, the K/V data one tile ahead, so neither latency sits on the tile loop.
  auto k_key = [&](int u) { return (tid + u * kThreadsMax) / (D / 8); };
  auto k_dim = [&](int u) { return ((tid + u * kThreadsMax) % (D / 8)) * 8; };
  auto v_kq = [&](int u) { return (tid + u * kThreadsMax) % 16; };
  auto v_dim = [&](int u) { return ((tid + u * kThreadsMax) / 16) * 8; };
  auto v_live = [&](int u) { return tid + u * kThreadsMax < kVPairs; };

  int kpg[kKUnits], vpg[kVUnits][4];
  float ksc[kKUnits], vsc[kVUnits][4];
  auto page_of = [&](int key) { return table[min(key, context - 1) >> p.block_shift]; };
  auto fetch_pages = [&](int t) {
    const int key0 = t * kTileKeys;
#pragma unroll
    for (int u = 0; u < kKUnits; ++u) kpg[u] = page_of(key0 + k_key(u));
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) vpg[u][j] = v_live(u) ? page_of(key0 + 4 * v_kq(u) + j) : 0;
    }
    if constexpr (kFp8) {
#pragma unroll
      for (int u = 0; u < kKUnits; ++u) ksc[u] = p.k_scales[static_cast<int64_t>(kpg[u]) * p.hk + kvh];
#pragma unroll
      for (int u = 0; u < kVUnits; ++u) {
#pragma unroll
        for (int j = 0; j < 4; ++j) vsc[u][j] = p.v_scales[static_cast<int64_t>(vpg[u][j]) * p.hk + kvh];
      }
    }
  };
  auto addr = [&](int page, int key, int dim) -> int64_t {
    const int k = min(key, context - 1);
    const int64_t slot = (static_cast<int64_t>(page) << p.block_shift) | (k & p.block_mask);
    return ((slot * p.hk + kvh) * D + dim) * kElemBytes;
  };

  u32x4 kreg[kKUnits];
  u32x4 vreg[kVUnits][4];
  auto load_tile = [&](int t) {
    const int key0 = t * kTileKeys;
#pragma unroll
    for (int u = 0; u < kKUnits; ++u) {
      kreg[u] = Stage<TQ, TKV>::load(kpool + addr(kpg[u], key0 + k_key(u), k_dim(u)),
                                     kFp8 ? ksc[u] : 1.0f);
    }
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
      if (!v_live(u)) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vreg[u][j] = Stage<TQ, TKV>::load(
            vpool + addr(vpg[u][j], key0 + 4 * v_kq(u) + j, v_dim(u)), kFp8 ? vsc[u][j] : 1.0f);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kKUnits; ++u) {
      *reinterpret_cast<u32x4*>(&k_lds[buf][k_key(u) * kKStride + k_dim(u)]) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
      if (!v_live(u)) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int sh = (e & 1) * 16;
        const uint32_t a = (vreg[u][0][e >> 1] >> sh) & 0xffffu;
        const uint32_t b = (vreg[u][1][e >> 1] >> sh) & 0xffffu;
        const uint32_t c = (vreg[u][2][e >> 1] >> sh) & 0xffffu;
        const uint32_t d = (vreg[u][3][e >> 1] >> sh) & 0xffffu;
        *reinterpret_cast<u32x2*>(&v_lds[buf][(v_dim(u) + e) * kVStride + 4 * v_kq(u)]) =
            u32x2{a | (b << 16), c | (d << 16)};
      }
    }
  };

  if (ntiles > 0) {
    fetch_pages(0);
    load_tile(0);
    if (ntiles > 1) fetch_pages(1);
  }

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    store_tile(buf);
    __syncthreads();
    if (t + 1 < ntiles) {
      load_tile(t + 1);
      if (t + 2 < ntiles) fetch_pages(t + 2);
    }

    const int key0 = t * kTileKeys;
    if (!w_active || key0 >= w_kv_end) continue;

    const uint16_t* kt = k_lds[buf];
    const uint16_t* vt = v_lds[buf];

    // S^T = K Q^T for two 32-key blocks; one K fragment feeds every head's MFMA.
    f32x16 s[HC][2];
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      s[h][0] = f32x16{};
      s[h][1] = f32x16{};
    }
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(kt + (kb * 32 + l32) * kKStride + 8 * hsel + ks * 16);
#pragma unroll
        for (int h = 0; h < HC; ++h) s[h][kb] = Mma<TQ>::run(a, qop[h][ks], s[h][kb]);
      }
    }

    // Online softmax per head; P^T operands straight from the score registers.
    const bool need_mask = key0 + kTileKeys > w_kv_full;
    u32x4 pop[HC][4];
#pragma unroll
    for (int h = 0; h < HC; ++h) {
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = s[h][kb][r] * score_scale;
          if (need_mask) {
            const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * hsel + (r & 3);
            v = (key < my_visible && my_valid) ? v : -INFINITY;
          }
          s[h][kb][r] = v;
          tmax = fmaxf(tmax, v);
        }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
      const float m_new = fmaxf(m_run[h], tmax);
      const float mu = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[h] - mu);
      m_run[h] = m_new;
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pv[e] = __builtin_amdgcn_exp2f(s[h][kb][8 * half + e] - mu);
            psum += pv[e];
          }
          pop[h][2 * kb + half] =
              u32x4{Mma<TQ>::pack2(pv[0], pv[1]), Mma<TQ>::pack2(pv[2], pv[3]),
                    Mma<TQ>::pack2(pv[4], pv[5]), Mma<TQ>::pack2(pv[6], pv[7])};
        }
      }
      l_run[h] = l_run[h] * alpha + psum;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o[h][db] *= alpha;
    }

    // O^T += V^T P^T. For k-step ks = 2*kb + half, this lane's eight k-values are
    // keys 32*kb + 16*half + {4h..4h+3, 8+4h..8+4h+3}; V^T is read in that order, and
    // one V^T fragment feeds every head's MFMA.
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
      const uint16_t* vrow = vt + (db * 32 + l32) * kVStride + 4 * hsel;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + 16 * ks);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16 * ks + 8);
        const u32x4 a = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int h = 0; h < HC; ++h) o[h][db] = Mma<TQ>::run(a, pop[h][ks], o[h][db]);
      }
    }
  }

  if (!w_active || !my_valid) return;
#pragma unroll
  for (int h = 0; h < HC; ++h) {
    const float l_tot = l_run[h] + __shfl_xor(l_run[h], 32, kWave);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int64_t orow = (static_cast<int64_t>(row_base + my_local) * p.hq + head0 + h) * D;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + 8 * j + 4 * hsel;
        float r[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = o[h][db][4 * j + i] * inv;
        *reinterpret_cast<u32x2*>(static_cast<char*>(p.out) + (orow + d) * 2) =
            u32x2{Mma<TQ>::pack2(r[0], r[1]), Mma<TQ>::pack2(r[2], r[3])};
      }
    }
  }
}

// ------------------------------------------------------------------ dispatch

namespace {

template <typename TQ, typename TKV, int D>
hipError_t launch_prefill_d(const PagedParams& p, int max_query_len, hipStream_t stream) {
  const int group = p.hq / p.hk;
  constexpr int kPositions = 32 * (kThreadsMax / kWave);
  const int qtiles = (max_query_len + kPositions - 1) / kPositions;
  // Two heads per wave fit the register file up to D = 128 (D = 256 would spill); at
  // config 3 they measured 144 us against 157 us with one head per wave.
  if (group % 2 == 0 && D <= 128) {
    const dim3 grid(p.hk * (group / 2), p.num_seqs, qtiles);
    paged_prefill_kernel<TQ, TKV, D, 2><<<grid, kThreadsMax, 0, stream>>>(p);
  } else {
    const dim3 grid(p.hk * group, p.num_seqs, qtiles);
    paged_prefill_kernel<TQ, TKV, D, 1><<<grid, kThreadsMax, 0, stream>>>(p);
  }
  return hipGetLastError();
}

template <typename TQ, typename TKV>
hipError_t launch_prefill_t(const PagedParams& p, int head_dim, int max_query_len,
                            hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch_prefill_d<TQ, TKV, 64>(p, max_query_len, stream);
    case 128: return launch_prefill_d<TQ, TKV, 128>(p, max_query_len, stream);
    case 256: return launch_prefill_d<TQ, TKV, 256>(p, max_query_len, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool paged_prefill_supported(int q_dtype, int kv_dtype, int head_dim, int hq, int hk,
                             int block_size) {
  (void)hq;
  (void)hk;
  (void)block_size;
  if (q_dtype != kBF16 && q_dtype != kF16) return false;
  if (kv_dtype != q_dtype && kv_dtype != kFP8E4M3) return false;
  return head_dim == 64 || head_dim == 128 || head_dim == 256;
}

hipError_t launch_paged_prefill(const PagedParams& p, int q_dtype, int kv_dtype, int head_dim,
                                int max_query_len, hipStream_t stream) {
  if (q_dtype == kBF16) {
    if (kv_dtype == kFP8E4M3) return launch_prefill_t<bf16_t, fp8_t>(p, head_dim, max_query_len, stream);
    return launch_prefill_t<bf16_t, bf16_t>(p, head_dim, max_query_len, stream);
  }
  if (q_dtype == kF16) {
    if (kv_dtype == kFP8E4M3) return launch_prefill_t<f16_t, fp8_t>(p, head_dim, max_query_len, stream);
    return launch_prefill_t<f16_t, f16_t>(p, head_dim, max_query_len, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mvllm
