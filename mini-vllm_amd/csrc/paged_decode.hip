// Paged decode attention for CDNA4, with split-K ("flash decoding") and a merge.
//
// Behaviour follows the reference's paged_decode_kernel / paged_decode_merge_kernel
// (csrc/paged_attention.cu:97-302): for every query row whose sequence computes one
// token (seq_lens[s] == 1), out = softmax(q K^T * scale) V over the context_lens[s]
// keys that the sequence's block table maps to physical slots
// (slot = table[p >> shift] << shift | (p & mask), paged_attention.cu:87-93).
//
// The work decomposition is this library's own.
//
// Inside a workgroup: one wave per (kv head, chunk of up to four query heads of that
// head's GQA group). The wave holds the queries of its group in registers, so each
// K/V byte is fetched from HBM exactly once however many query heads share it. A
// token's (kv head) row is D elements = D / E lanes of 16 bytes (E = 8 for bf16/fp16,
// 4 for fp32, 16 for fp8); the 64 lanes split into 64 / (D / E) row groups, each
// streaming its own tokens with its own online-softmax state, so the main loop needs
// no cross-row-group traffic and no barrier: a dot product is reduced with 16-lane DPP
// all-reduces only. Row groups are merged once at the end with the reference's
// rescale exp(m_i - M) (paged_attention.cu:284-301).
//
// Across workgroups, two schedules:
//
//  * stream (the decode hot path): a persistent grid of a few workgroups per CU. The
//    decode sequences' keys are laid end to end (an in-kernel prefix scan of
//    context_lens, no host read) and every workgroup streams an equal share of that
//    token axis, so every CU moves the same bytes whatever the length distribution.
//    A share that covers a whole sequence writes its output directly; a sequence cut
//    between workgroups leaves one (m, l, O) partial per piece, in slot
//    (workgroup + sequence), which is unique because shares and sequences are both
//    contiguous ranges of the same axis. A second small kernel merges the pieces.
//    (Merging in the decode kernel instead -- the last workgroup to finish a piece
//    merges, on an atomic counter -- measured slower: every merge then sits at the
//    end of the launch behind a chain of dependent memory round trips.)
//  * grid (fallback, and the by-row mode that also serves prefill rows when no MFMA
//    prefill kernel fits the shape): one workgroup per (row, split) with splits of
//    `split_tokens` keys, page ids staged in LDS, merged by a second kernel.
//
// Fresh-token stream (a decode-only batch over a 16-bit pool): every sequence's last
// key is the step's new token, taken from the q/k/v projection's output rather than
// the pool. Each wave QK-norms and rotates its queries itself (norm_rope_chunk, the
// QK-norm + RoPE kernel's code: this file is compiled with -ffp-contract=off so it
// rounds the same), the share holding a sequence's last key forms that key's row
// likewise, writes it and v to the pool slot, and uses them from registers in its last
// step; the result is the QK-norm + RoPE + KV-write launch followed by the plain
// stream, bit for bit, with one launch fewer.
//
// K/V are read with nontemporal 16-byte loads (they are streamed once); page ids are
// fetched one step ahead of the K/V loads that need them. Scores are kept in the
// log2 domain: s = (q.k) * scale * log2(e), p = 2^(s - m), exactly
// exp((q.k)*scale - max) in real arithmetic, at one v_exp_f32 per score.

#include "common.hpp"
#include "paged_attention.hpp"

namespace mvllm {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
// Tokens per row group per step (each step's K/V rows are requested together).
#ifndef MVLLM_DECODE_UNROLL
#define MVLLM_DECODE_UNROLL 4
#endif
constexpr int kUnroll = MVLLM_DECODE_UNROLL;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ u32x4 load16_stream(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Which query row, sequence and visible context a grid-schedule workgroup serves.
// Returns false when the workgroup has nothing to do in this pass.
__device__ __forceinline__ bool resolve_row(const PagedParams& p, int index, int& seq, int& row,
                                            int& visible) {
  if (p.by_row) {
    // Every query row is a unit: find its sequence by binary search over cu_seqlens_q.
    row = index;
    int lo = 0, hi = p.num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.cu_seqlens_q[mid] <= row) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    const int query_len = p.seq_lens[seq];
    const int local = row - p.cu_seqlens_q[seq];
    // The L queries are the last L positions of the context (causal offset S - L,
    // reference attention.py:76-92 / paged_attention.cu:348-349).
    visible = p.context_lens[seq] - query_len + local + 1;
    return visible > 0;
  }
  seq = index;
  if (p.seq_lens[seq] != 1) return false;  // a prefill chunk: the prefill kernel has it
  row = p.cu_seqlens_q[seq];
  visible = p.context_lens[seq];
  return visible > 0;
}

// Per-wave online-softmax state over a run of keys, for GC query heads.
template <int GC, int E>
struct WaveState {
  float m[GC];
  float l[GC];
  float acc[GC][E];
};

template <typename TKV, int D, int GC>
struct Decode {
  static constexpr int E = Chunk<TKV>::kN;   // elements per 16-byte chunk
  static constexpr int R = D / E;            // lanes per token row
  static constexpr int RG = kWave / R;       // row groups per wave
  static constexpr bool kFp8 = Elem<TKV>::kBytes == 1;
  static_assert(R >= 1 && R <= kWave && (kWave % R) == 0, "head dim / dtype mismatch");
  using State = WaveState<GC, E>;

  template <typename TQ>
  __device__ static void load_queries(const PagedParams& p, int row, int h0, int r,
                                      float (&qf)[GC][E]) {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const int64_t base = (static_cast<int64_t>(row) * p.hq + h0 + h) * D + r * E;
#pragma unroll
      for (int e = 0; e < E; ++e) qf[h][e] = Elem<TQ>::load(p.q, base + e);
    }
  }

  __device__ static void init(State& st) {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      st.m[h] = -INFINITY;
      st.l[h] = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) st.acc[h][e] = 0.0f;
    }
  }

  // Stream keys [sb, se) of one sequence for kv head `kvh` into `st`. Page ids come
  // from `lds_pages` (page i of the run at lds_pages[i - first_page]) when given,
  // otherwise from the sequence's block table; the next step's page ids are requested
  // before this step is computed. (Requesting the next step's K/V rows early as well
  // measured slower: on shuffled pages more requests in flight per CU cost DRAM
  // efficiency.)
  __device__ static void stream(const PagedParams& p, const int32_t* table, const int* lds_pages,
                                int first_page, int kvh, int sb, int se, int g, int r,
                                const float (&qf)[GC][E], float score_scale, State& st) {
    const Fresh none{-1, {}, {}};
    stream_with<false>(p, table, lds_pages, first_page, kvh, sb, se, g, r, qf, score_scale, st,
                       [] {}, none);
  }

  // The new token of a fresh-token stream: token `tok` of the run (< 0: none) takes this
  // lane's chunks `k` and `v` as its K and V rows instead of the pool's.
  struct Fresh {
    int tok;
    u32x4 k, v;
  };

  // stream() with two additions: `prep()` runs once the first step's page ids have been
  // requested (a fresh-token stream forms its queries and the new token's rows there, in
  // qf and `fresh`, so that arithmetic overlaps those loads), and with kFresh the step
  // holding fresh.tok takes that token's rows from `fresh`. (Forming them under the
  // first step's K/V requests instead measured the same, with 60% more registers.)
  template <bool kFresh, typename Prep>
  __device__ static void stream_with(const PagedParams& p, const int32_t* table,
                                     const int* lds_pages, int first_page, int kvh, int sb, int se,
                                     int g, int r, const float (&qf)[GC][E], float score_scale,
                                     State& st, Prep&& prep, const Fresh& fresh) {
    static_assert(!(kFresh && kFp8), "the fresh-token stream serves 16-bit pools");
    const char* kbase = static_cast<const char*>(p.k_pool);
    const char* vbase = static_cast<const char*>(p.v_pool);
    constexpr int kElemBytes = Elem<TKV>::kBytes;
    constexpr int kStep = RG * kUnroll;

    auto page_of = [&](int tok) -> int {
      const int pi = tok >> p.block_shift;
      return lds_pages != nullptr ? lds_pages[pi - first_page] : table[pi];
    };

    int pg[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) pg[u] = page_of(min(sb + u * RG + g, se - 1));
    prep();

    for (int t0 = sb; t0 < se; t0 += kStep) {
      u32x4 kw[kUnroll], vw[kUnroll];
      bool valid[kUnroll];
      float ks[kUnroll], vs[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        int tok = t0 + u * RG + g;
        valid[u] = tok < se;
        tok = valid[u] ? tok : se - 1;
        const int64_t slot = (static_cast<int64_t>(pg[u]) << p.table_shift) + (tok & p.block_mask);
        const int64_t off = slot * p.kv_row_bytes + kvh * p.kv_head_bytes + r * E * kElemBytes;
        kw[u] = load16_stream(kbase + off);
        vw[u] = load16_stream(vbase + off);
        if constexpr (kFp8) {
          ks[u] = p.k_scales[static_cast<int64_t>(pg[u]) * p.hk + kvh];
          vs[u] = p.v_scales[static_cast<int64_t>(pg[u]) * p.hk + kvh];
        }
      }
      if (t0 + kStep < se) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) pg[u] = page_of(min(t0 + kStep + u * RG + g, se - 1));
      }
      if constexpr (kFresh) {
        // The step holding the new token (wave-uniform test): its pool slot, read above
        // before this launch wrote it, is replaced by the rows formed in the launch.
        if (fresh.tok >= 0 && t0 + kStep > fresh.tok) [[unlikely]] {
          // a real branch, taken once per share: without the barrier the compiler turns
          // the substitution into selects executed in every step
          asm volatile("" ::: "memory");
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            if (t0 + u * RG + g == fresh.tok) {
              kw[u] = fresh.k;
              vw[u] = fresh.v;
            }
          }
        }
      }

      float s[kUnroll][GC];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float kf[E];
        Chunk<TKV>::unpack(kw[u], kf);
#pragma unroll
        for (int h = 0; h < GC; ++h) {
          float dot = 0.0f;
#pragma unroll
          for (int e = 0; e < E; ++e) dot = fmaf(qf[h][e], kf[e], dot);
          dot = group_sum<R>(dot);
          // The reference scales after the reduction (paged_attention.cu:181-183).
          float sc = dot * score_scale;
          if constexpr (kFp8) sc *= ks[u];
          s[u][h] = valid[u] ? sc : -INFINITY;
        }
      }

      float pr[kUnroll][GC];
#pragma unroll
      for (int h = 0; h < GC; ++h) {
        float mx = st.m[h];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) mx = fmaxf(mx, s[u][h]);
        // A row group that has seen no valid key yet keeps m = -inf; exponentiate
        // against 0 then, so 2^(-inf - 0) = 0 instead of 2^(-inf + inf) = NaN
        // (the empty-split rule of paged_attention.cu:210-213).
        const float mu = mx == -INFINITY ? 0.0f : mx;
        const float alpha = fast_exp2(st.m[h] - mu);
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          pr[u][h] = fast_exp2(s[u][h] - mu);
          sum += pr[u][h];
        }
        st.l[h] = st.l[h] * alpha + sum;
        st.m[h] = mx;
#pragma unroll
        for (int e = 0; e < E; ++e) st.acc[h][e] *= alpha;
      }

#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float vf[E];
        Chunk<TKV>::unpack(vw[u], vf);
#pragma unroll
        for (int h = 0; h < GC; ++h) {
          float w = pr[u][h];
          if constexpr (kFp8) w *= vs[u];
#pragma unroll
          for (int e = 0; e < E; ++e) st.acc[h][e] = fmaf(w, vf[e], st.acc[h][e]);
        }
      }
    }
  }

  // Combine the wave's row groups: xor partners share r and differ in g. Afterwards
  // every row group holds the totals.
  __device__ static void merge_row_groups(State& st) {
#pragma unroll
    for (int off = R; off < kWave; off <<= 1) {
#pragma unroll
      for (int h = 0; h < GC; ++h) {
        const float mo = __shfl_xor(st.m[h], off, kWave);
        const float lo = __shfl_xor(st.l[h], off, kWave);
        const float mx = fmaxf(st.m[h], mo);
        const float mu = mx == -INFINITY ? 0.0f : mx;
        const float a = fast_exp2(st.m[h] - mu);
        const float b = fast_exp2(mo - mu);
        st.l[h] = st.l[h] * a + lo * b;
        st.m[h] = mx;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float other = __shfl_xor(st.acc[h][e], off, kWave);
          st.acc[h][e] = st.acc[h][e] * a + other * b;
        }
      }
    }
  }

  template <typename TQ>
  __device__ static void write_output(const PagedParams& p, int row, int h0, int r, const State& st) {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const float inv = st.l[h] > 0.0f ? 1.0f / st.l[h] : 0.0f;
      const int64_t base = (static_cast<int64_t>(row) * p.hq + h0 + h) * D + r * E;
#pragma unroll
      for (int e = 0; e < E; ++e) Elem<TQ>::store(p.out, base + e, st.acc[h][e] * inv);
    }
  }

  // Partial of head h0 + h at index (pidx0 + h * pstride).
  __device__ static void write_partial(const PagedParams& p, int64_t pidx0, int64_t pstride, int r,
                                       const State& st) {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const int64_t pidx = pidx0 + h * pstride;
      float* po = p.part_o + pidx * D + r * E;
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        *reinterpret_cast<f32x4*>(po + e) =
            f32x4{st.acc[h][e], st.acc[h][e + 1], st.acc[h][e + 2], st.acc[h][e + 3]};
      }
      if (r == 0) {
        p.part_ml[pidx * 2] = st.m[h];
        p.part_ml[pidx * 2 + 1] = st.l[h];
      }
    }
  }
};

// The (kv head, head chunk) unit of a wave; false when the wave has none.
template <int GC>
__device__ __forceinline__ bool wave_unit(const PagedParams& p, int unit, int& kvh, int& h0) {
  const int chunks = p.hq / p.hk / GC;
  if (unit >= p.hk * chunks) return false;
  kvh = unit / chunks;
  h0 = kvh * (p.hq / p.hk) + (unit % chunks) * GC;
  return true;
}

}  // namespace

// ------------------------------------------------------------ stream schedule

// kFresh: every sequence's last key is the step's new token, formed here from the
// projection's output (FreshParams) instead of read from the pool.
template <typename TQ, typename TKV, int D, int GC, bool kFresh>
__global__ __launch_bounds__(512) void paged_decode_stream_kernel(const PagedParams p,
                                                                  const FreshParams f) {
  using K = Decode<TKV, D, GC>;
  __shared__ int s_prefix[kMaxStreamSeqs + 1];  // decode keys before sequence s

  const int n = p.num_seqs;
  const int tid = threadIdx.x;
  // Prefix scan of the decode sequences' context lengths (0 for prefill chunks), by
  // wave 0: each lane sums a contiguous run, then a 64-lane inclusive scan.
  if (tid < kWave) {
    const int per = (n + kWave - 1) / kWave;
    const int begin = min(tid * per, n);
    const int end = min(begin + per, n);
    int run = 0;
    for (int s = begin; s < end; ++s) run += p.seq_lens[s] == 1 ? max(p.context_lens[s], 0) : 0;
    int incl = run;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int other = __shfl_up(incl, off, kWave);
      if (tid >= off) incl += other;
    }
    int acc = incl - run;
    for (int s = begin; s < end; ++s) {
      s_prefix[s] = acc;
      acc += p.seq_lens[s] == 1 ? max(p.context_lens[s], 0) : 0;
    }
    if (tid == kWave - 1) s_prefix[n] = incl;
  }
  __syncthreads();

  const int64_t total = s_prefix[n];
  const int64_t wgs = decode_stream_shares(total, gridDim.x);
  if (blockIdx.x == 0) {
    for (int s = tid; s <= n; s += blockDim.x) p.seq_prefix[s] = s_prefix[s];
  }
  if (blockIdx.x >= wgs) return;  // whole workgroup: no barrier follows for it
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * total / wgs;
  const int64_t hi = (static_cast<int64_t>(blockIdx.x) + 1) * total / wgs;
  if (lo >= hi) return;  // whole workgroup: no barrier follows for it

  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int g = lane / K::R;
  const int r = lane % K::R;
  int kvh = 0, h0 = 0;
  const bool active = wave_unit<GC>(p, wave, kvh, h0);
  const float score_scale = p.scale * kLog2e;

  // First sequence whose keys include `lo`: the last s with prefix[s] <= lo.
  int a = 0, b = n;  // invariant: prefix[a] <= lo < prefix[b]
  while (b - a > 1) {
    const int mid = (a + b) >> 1;
    if (s_prefix[mid] <= lo) a = mid; else b = mid;
  }
  int seq = a;
  int64_t pos = lo;
  while (pos < hi) {
    while (s_prefix[seq + 1] == s_prefix[seq]) ++seq;  // skip prefill / empty sequences
    const int base = s_prefix[seq];
    const int ctx = s_prefix[seq + 1] - base;
    const int sb = static_cast<int>(pos - base);
    const int se = static_cast<int>(min(hi, static_cast<int64_t>(s_prefix[seq + 1])) - base);
    // A decode-only batch (the fresh-token stream) has row s for sequence s: no load
    // ahead of the raw q/k/v reads that address by row.
    const int row = kFresh ? seq : p.cu_seqlens_q[seq];
    const bool whole = sb == 0 && se == ctx;
    typename K::State st;
    if (active) {
      float qf[GC][K::E];
      K::init(st);
      const int32_t* table = p.block_tables + static_cast<int64_t>(seq) * p.max_blocks;
      if constexpr (kFresh) {
        static_assert(K::E == 8 && K::R == 16, "the fresh-token stream takes 16-bit D = 128");
        // Loads first (all rows of the token, whether or not this run holds it: no
        // divergent loads), the arithmetic in prep() once the page ids are requested.
        const int pos = ctx - 1;
        const bool pos_ok = pos < f.max_positions;
        const int64_t trow = pos_ok ? pos : 0;  // out of range: row 0, NaN rows below
        u32x4 qraw[GC];
#pragma unroll
        for (int h = 0; h < GC; ++h) {
          qraw[h] = load16(static_cast<const char*>(f.q) +
                           (static_cast<int64_t>(row) * f.q_stride + (h0 + h) * D + r * 8) * 2);
        }
        const int64_t kvoff = (static_cast<int64_t>(row) * f.kv_stride + kvh * D + r * 8) * 2;
        const u32x4 kraw = load16(static_cast<const char*>(f.k) + kvoff);
        const u32x4 vraw = load16(static_cast<const char*>(f.v) + kvoff);
        const u32x4 wq = load16(static_cast<const char*>(f.q_weight) + r * 16);
        const u32x4 wk = load16(static_cast<const char*>(f.k_weight) + r * 16);
        float c[8], sn[8];
        Chunk<float>::unpack(load16(f.cos_t + trow * D + r * 8), c);
        Chunk<float>::unpack(load16(f.cos_t + trow * D + r * 8 + 4), c + 4);
        Chunk<float>::unpack(load16(f.sin_t + trow * D + r * 8), sn);
        Chunk<float>::unpack(load16(f.sin_t + trow * D + r * 8 + 4), sn + 4);
        const int new_page = table[pos >> p.block_shift];
        const bool has_new = se == ctx;
        typename K::Fresh fresh{-1, {}, {}};
        auto prep = [&]() {
          if (r < 8) {
#pragma unroll
            for (int e = 0; e < 8; ++e) sn[e] = -sn[e];
          }
          if (!pos_ok) {
#pragma unroll
            for (int e = 0; e < 8; ++e) c[e] = sn[e] = __int_as_float(0x7fc00000);
          }
          // The GC query rows and the key row, one per row group and pass (row group g
          // of pass i forms row 4 i + g: query heads first, then k; a row group past
          // the last row forms k again, unused), then each row's chunk r read by every
          // row group from lane 16 (row % 4) + r. One pass for up to three query heads:
          // a quarter of the arithmetic of every row group forming every row.
          constexpr int kRows = GC + 1;
          constexpr int kPasses = (kRows + K::RG - 1) / K::RG;
          u32x4 formed[kPasses];
#pragma unroll
          for (int i = 0; i < kPasses; ++i) {
            const int rix = i * K::RG + g;
            u32x4 held = kraw;
#pragma unroll
            for (int h = 0; h < GC; ++h) held = rix == h ? qraw[h] : held;
            float wf[8];
            Chunk<TQ>::unpack(rix < GC ? wq : wk, wf);
            formed[i] = norm_rope_chunk<TQ, 16>(held, wf, c, sn, f.eps);
          }
          auto row_of = [&](int rix) {
            const int src = (rix % K::RG) * 16 + r;
            const u32x4& x = formed[rix / K::RG];
            return u32x4{static_cast<uint32_t>(__shfl(static_cast<int>(x[0]), src, kWave)),
                         static_cast<uint32_t>(__shfl(static_cast<int>(x[1]), src, kWave)),
                         static_cast<uint32_t>(__shfl(static_cast<int>(x[2]), src, kWave)),
                         static_cast<uint32_t>(__shfl(static_cast<int>(x[3]), src, kWave))};
          };
#pragma unroll
          for (int h = 0; h < GC; ++h) {
            // rounded to TQ as the unfused kernel stores q, widened as the attention loads it
            Chunk<TQ>::unpack(row_of(h), qf[h]);
          }
          fresh.k = row_of(GC);
          fresh.v = vraw;
          if (has_new) {
            fresh.tok = pos;
            // One wave per kv head writes the pool (the first of its query-head chunks),
            // row group 0's 16 lanes one row each of K and V.
            if (g == 0 && h0 % (p.hq / p.hk) == 0 && new_page >= 0 && new_page < f.num_blocks) {
              const int64_t slot =
                  (static_cast<int64_t>(new_page) << p.table_shift) + (pos & p.block_mask);
              const int64_t off = slot * p.kv_row_bytes + kvh * p.kv_head_bytes + r * 16;
              store16(static_cast<char*>(const_cast<void*>(p.k_pool)) + off, fresh.k);
              store16(static_cast<char*>(const_cast<void*>(p.v_pool)) + off, fresh.v);
            }
          }
        };
        K::template stream_with<true>(p, table, nullptr, 0, kvh, sb, se, g, r, qf, score_scale,
                                      st, prep, fresh);
      } else {
        K::template load_queries<TQ>(p, row, h0, r, qf);
        K::stream(p, table, nullptr, 0, kvh, sb, se, g, r, qf, score_scale, st);
      }
      K::merge_row_groups(st);
      if (g == 0) {
        if (whole) {
          K::template write_output<TQ>(p, row, h0, r, st);
        } else {
          K::write_partial(p, (static_cast<int64_t>(blockIdx.x) + seq) * p.hq + h0, 1, r, st);
        }
      }
    }
    pos = base + se;
    ++seq;
  }
}

// Combine the pieces of every decode sequence cut between stream workgroups. Piece i
// of sequence s lives in slot (first + i + s), first/last being the workgroups owning
// the sequence's first and last key. Grid (sequence, block of kMergeCols float4
// columns of its H_q x D output); in a workgroup, kMergeGroups groups of threads take
// the pieces round robin (group g: pieces g, g + G, ...), each thread folding its
// pieces for one float4 column online (running max, rescaled sums) with kMergeBatch
// pieces' loads in flight at once; the groups' states then meet in LDS and are folded
// in group order. A long sequence cut into dozens of pieces so costs a few round trips
// instead of one per eight pieces, and a batch's sequences spread over H_q D / 4 /
// kMergeCols workgroups each instead of one. The fold order depends on the piece count
// alone, so a call's result does not depend on timing.
constexpr int kMergeCols = 128;
constexpr int kMergeGroups = 4;
constexpr int kMergeBatch = 8;

template <typename TQ, int D>
__global__ __launch_bounds__(kMergeCols * kMergeGroups) void paged_decode_stream_merge_kernel(
    const PagedParams p, int wgs_i) {
  __shared__ float s_m[kMergeGroups][kMergeCols];
  __shared__ float s_l[kMergeGroups][kMergeCols];
  __shared__ f32x4 s_o[kMergeGroups][kMergeCols];
  const int seq = blockIdx.x;
  const int64_t total = p.seq_prefix[p.num_seqs];
  const int64_t wgs = decode_stream_shares(total, wgs_i);
  const int64_t begin = p.seq_prefix[seq];
  const int64_t end = p.seq_prefix[seq + 1];
  if (end == begin || total == 0) return;  // whole workgroup: no barrier follows for it
  const int64_t first = share_owner(begin, total, wgs);
  const int64_t last = share_owner(end - 1, total, wgs);
  if (first == last) return;  // one piece: the decode kernel stored the output
  const bool all_live = total >= wgs;
  const int pieces = static_cast<int>(last - first + 1);
  const int n4 = p.hq * D / 4;
  const int local = threadIdx.x % kMergeCols;
  const int grp = threadIdx.x / kMergeCols;
  const int j = blockIdx.y * kMergeCols + local;
  const bool live = j < n4;
  const int head = live ? (4 * j) / D : 0;
  const int d = live ? 4 * j - head * D : 0;

  float m = -INFINITY, l = 0.0f;
  f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  if (live) {
    for (int i0 = grp; i0 < pieces; i0 += kMergeGroups * kMergeBatch) {
      float mi[kMergeBatch], li[kMergeBatch];
      f32x4 oi[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int i = min(i0 + u * kMergeGroups, pieces - 1);
        const int64_t pidx = (first + i + seq) * p.hq + head;
        mi[u] = p.part_ml[pidx * 2];
        li[u] = p.part_ml[pidx * 2 + 1];
        oi[u] = *reinterpret_cast<const f32x4*>(p.part_o + pidx * D + d);
      }
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int i = i0 + u * kMergeGroups;
        // Beyond the last piece, or a workgroup whose share was empty (fewer keys
        // than workgroups): it wrote nothing and contributes nothing.
        if (i >= pieces || !(all_live || share_nonempty(first + i, total, wgs))) continue;
        const float mn = fmaxf(m, mi[u]);
        const float mu = mn == -INFINITY ? 0.0f : mn;
        const float a = fast_exp2(m - mu);
        const float b = fast_exp2(mi[u] - mu);
        l = l * a + li[u] * b;
        o = o * a + oi[u] * b;
        m = mn;
      }
    }
  }
  s_m[grp][local] = m;
  s_l[grp][local] = l;
  s_o[grp][local] = o;
  __syncthreads();
  if (grp != 0 || !live) return;
  m = -INFINITY;
  l = 0.0f;
  o = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int g = 0; g < kMergeGroups; ++g) {
    const float mg = s_m[g][local];
    const float mn = fmaxf(m, mg);
    const float mu = mn == -INFINITY ? 0.0f : mn;
    const float a = fast_exp2(m - mu);
    const float b = fast_exp2(mg - mu);
    l = l * a + s_l[g][local] * b;
    o = o * a + s_o[g][local] * b;
    m = mn;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const int row = p.cu_seqlens_q[seq];
  const int64_t obase = (static_cast<int64_t>(row) * p.hq + head) * D + d;
#pragma unroll
  for (int k = 0; k < 4; ++k) Elem<TQ>::store(p.out, obase + k, o[k] * inv);
}

// -------------------------------------------------------------- grid schedule

template <typename TQ, typename TKV, int D, int GC>
__global__ __launch_bounds__(512) void paged_decode_grid_kernel(const PagedParams p) {
  using K = Decode<TKV, D, GC>;
  __shared__ int s_pages[kMaxSplitPages];

  int seq, row, visible;
  if (!resolve_row(p, blockIdx.y, seq, row, visible)) return;

  const int nsplit = decode_num_splits(visible, p.split_tokens, p.max_splits);
  const int split = blockIdx.x;
  if (split >= nsplit) return;
  const int per_split = decode_split_len(visible, nsplit);
  const int sb = split * per_split;
  const int se = min(sb + per_split, visible);

  const int partial_row = p.by_row ? row : seq;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int g = lane / K::R;
  const int r = lane % K::R;

  const int32_t* table = p.block_tables + static_cast<int64_t>(seq) * p.max_blocks;
  const int first_page = sb >> p.block_shift;
  const int n_pages = sb < se ? ((se - 1) >> p.block_shift) - first_page + 1 : 0;
  const bool pages_in_lds = n_pages <= kMaxSplitPages;
  if (pages_in_lds) {
    for (int i = threadIdx.x; i < n_pages; i += blockDim.x) s_pages[i] = table[first_page + i];
  }
  __syncthreads();

  int kvh, h0;
  if (!wave_unit<GC>(p, blockIdx.z * (blockDim.x / kWave) + wave, kvh, h0)) return;

  float qf[GC][K::E];
  K::template load_queries<TQ>(p, row, h0, r, qf);
  typename K::State st;
  K::init(st);
  K::stream(p, table, pages_in_lds ? s_pages : nullptr, first_page, kvh, sb, se, g, r, qf,
            p.scale * kLog2e, st);
  K::merge_row_groups(st);
  if (g != 0) return;
  if (nsplit == 1) {
    K::template write_output<TQ>(p, row, h0, r, st);
  } else {
    K::write_partial(p, (static_cast<int64_t>(partial_row) * p.hq + h0) * p.max_splits + split,
                     p.max_splits, r, st);
  }
}

// Combine the split partials of every (row, query head) that was split:
// out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s. One wave per (row, head).
template <typename TQ, int D>
__global__ __launch_bounds__(256) void paged_decode_grid_merge_kernel(const PagedParams p) {
  constexpr int kPerLane = (D + kWave - 1) / kWave;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int head = blockIdx.x * (blockDim.x / kWave) + wave;
  if (head >= p.hq) return;

  int seq, row, visible;
  if (!resolve_row(p, blockIdx.y, seq, row, visible)) return;
  const int nsplit = decode_num_splits(visible, p.split_tokens, p.max_splits);
  if (nsplit == 1) return;  // the decode kernel stored this row directly

  const int partial_row = p.by_row ? row : seq;
  const int64_t prow0 = (static_cast<int64_t>(partial_row) * p.hq + head) * p.max_splits;

  float mmax = -INFINITY;
  for (int s = lane; s < nsplit; s += kWave) mmax = fmaxf(mmax, p.part_ml[(prow0 + s) * 2]);
  mmax = wave_max(mmax);
  const float mu = mmax == -INFINITY ? 0.0f : mmax;

  float total_l = 0.0f;
  for (int s = lane; s < nsplit; s += kWave) {
    const float ls = p.part_ml[(prow0 + s) * 2 + 1];
    if (ls > 0.0f) total_l += __builtin_amdgcn_exp2f(p.part_ml[(prow0 + s) * 2] - mu) * ls;
  }
  total_l = wave_sum(total_l);
  const float inv = total_l > 0.0f ? 1.0f / total_l : 0.0f;

  float o[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) o[i] = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float ls = p.part_ml[(prow0 + s) * 2 + 1];
    if (!(ls > 0.0f)) continue;  // an empty split contributes exactly nothing
    const float w = __builtin_amdgcn_exp2f(p.part_ml[(prow0 + s) * 2] - mu);
    const float* po = p.part_o + (prow0 + s) * D;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int d = lane + i * kWave;
      if (d < D) o[i] = fmaf(w, po[d], o[i]);
    }
  }
  const int64_t base = (static_cast<int64_t>(row) * p.hq + head) * D;
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int d = lane + i * kWave;
    if (d < D) Elem<TQ>::store(p.out, base + d, o[i] * inv);
  }
}

// ------------------------------------------------------------------ dispatch

namespace {

int decode_waves(const PagedParams& p, int gc) {
  const int units = p.hk * (p.hq / p.hk / gc);
  return units < 8 ? units : 8;
}

template <typename TQ, int D>
hipError_t launch_stream_merge(const PagedParams& p, hipStream_t stream) {
  const int n4 = p.hq * D / 4;
  const dim3 mgrid(p.num_seqs, (n4 + kMergeCols - 1) / kMergeCols);
  paged_decode_stream_merge_kernel<TQ, D>
      <<<mgrid, kMergeCols * kMergeGroups, 0, stream>>>(p, p.stream_wgs);
  return hipGetLastError();
}

template <typename TQ, typename TKV, int D, int GC>
hipError_t launch_decode_g(const PagedParams& p, hipStream_t stream) {
  const int units = p.hk * (p.hq / p.hk / GC);
  const int waves = decode_waves(p, GC);
  constexpr int kHeadsPerMergeBlock = 4;
  if (p.stream_wgs > 0) {
    if (units > 8) return hipErrorInvalidValue;  // planner keeps stream mode to <= 8 units
    paged_decode_stream_kernel<TQ, TKV, D, GC, false>
        <<<p.stream_wgs, waves * kWave, 0, stream>>>(p, FreshParams{});
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_stream_merge<TQ, D>(p, stream);
  }
  const dim3 grid(p.max_splits, p.by_row ? p.num_tokens : p.num_seqs, (units + waves - 1) / waves);
  paged_decode_grid_kernel<TQ, TKV, D, GC><<<grid, waves * kWave, 0, stream>>>(p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.max_splits == 1) return err;
  const dim3 mgrid((p.hq + kHeadsPerMergeBlock - 1) / kHeadsPerMergeBlock,
                   p.by_row ? p.num_tokens : p.num_seqs);
  paged_decode_grid_merge_kernel<TQ, D><<<mgrid, kHeadsPerMergeBlock * kWave, 0, stream>>>(p);
  return hipGetLastError();
}

template <typename TQ, typename TKV, int D>
hipError_t launch_decode_d(const PagedParams& p, hipStream_t stream) {
  switch (decode_group_chunk(p.hq / p.hk)) {
    case 4: return launch_decode_g<TQ, TKV, D, 4>(p, stream);
    case 2: return launch_decode_g<TQ, TKV, D, 2>(p, stream);
    default: return launch_decode_g<TQ, TKV, D, 1>(p, stream);
  }
}

template <typename TQ, typename TKV>
hipError_t launch_decode_t(const PagedParams& p, int head_dim, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_decode_d<TQ, TKV, 32>(p, stream);
    case 64: return launch_decode_d<TQ, TKV, 64>(p, stream);
    case 128: return launch_decode_d<TQ, TKV, 128>(p, stream);
    case 256: return launch_decode_d<TQ, TKV, 256>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

namespace {

template <typename T, int GC>
hipError_t launch_fresh_g(const PagedParams& p, const FreshParams& f, hipStream_t stream) {
  constexpr int D = 128;
  const int units = p.hk * (p.hq / p.hk / GC);
  if (units > 8) return hipErrorInvalidValue;  // planner keeps stream mode to <= 8 units
  paged_decode_stream_kernel<T, T, D, GC, true>
      <<<p.stream_wgs, decode_waves(p, GC) * kWave, 0, stream>>>(p, f);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  return launch_stream_merge<T, D>(p, stream);
}

template <typename T>
hipError_t launch_fresh_t(const PagedParams& p, const FreshParams& f, hipStream_t stream) {
  switch (decode_group_chunk(p.hq / p.hk)) {
    case 4: return launch_fresh_g<T, 4>(p, f, stream);
    case 2: return launch_fresh_g<T, 2>(p, f, stream);
    default: return launch_fresh_g<T, 1>(p, f, stream);
  }
}

}  // namespace

hipError_t launch_paged_decode_fresh(const PagedParams& p, const FreshParams& f, int dtype,
                                     int head_dim, hipStream_t stream) {
  if (head_dim != 128 || p.stream_wgs <= 0) return hipErrorInvalidValue;
  switch (dtype) {
    case kF16: return launch_fresh_t<f16_t>(p, f, stream);
    case kBF16: return launch_fresh_t<bf16_t>(p, f, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_paged_decode(const PagedParams& p, int q_dtype, int kv_dtype, int head_dim,
                               hipStream_t stream) {
  if (kv_dtype == kFP8E4M3) {
    if (q_dtype == kBF16) return launch_decode_t<bf16_t, fp8_t>(p, head_dim, stream);
    if (q_dtype == kF16) return launch_decode_t<f16_t, fp8_t>(p, head_dim, stream);
    if (q_dtype == kF32) return launch_decode_t<float, fp8_t>(p, head_dim, stream);
    return hipErrorInvalidValue;
  }
  if (q_dtype != kv_dtype) return hipErrorInvalidValue;
  switch (q_dtype) {
    case kF32: return launch_decode_t<float, float>(p, head_dim, stream);
    case kF16: return launch_decode_t<f16_t, f16_t>(p, head_dim, stream);
    case kBF16: return launch_decode_t<bf16_t, bf16_t>(p, head_dim, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mvllm
