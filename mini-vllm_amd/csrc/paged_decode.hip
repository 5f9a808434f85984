// Paged decode attention for CDNA4, with split-K ("flash decoding") and a merge.
//
// Behaviour follows the reference's paged_decode_kernel / paged_decode_merge_kernel
// (csrc/paged_attention.cu:97-302): for every query row whose sequence computes one
// token (seq_lens[s] == 1), out = softmax(q K^T * scale) V over the context_lens[s]
// keys that the sequence's block table maps to physical slots
// (slot = table[p >> shift] << shift | (p & mask), paged_attention.cu:87-93).
//
// The work decomposition is this library's own:
//
//  * one workgroup per (sequence or row, split); one wave per (kv head, chunk of up
//    to four query heads of that head's GQA group). The wave holds the queries of
//    its whole group in registers, so each K/V byte is fetched from HBM exactly
//    once however many query heads share it.
//  * inside a wave, a token's (kv head) row is D elements = D / E lanes of 16 bytes
//    (E = 8 for bf16/fp16, 4 for fp32, 16 for fp8). The 64 lanes split into
//    64 / (D / E) row groups, each streaming its own tokens with its own online
//    softmax state, so the main loop needs no cross-row-group traffic and no
//    barrier: a dot product is reduced with 16-lane DPP all-reduces only.
//  * the row groups, and then the splits, are merged with the same rescale
//    exp(m_i - M) the reference uses one level up (paged_attention.cu:284-301).
//  * the split's physical page ids are staged once into LDS and shared by all
//    waves of the workgroup (every kv head of the split walks the same pages).
//
// Scores are kept in the log2 domain: s = (q.k) * scale * log2(e), p = 2^(s - m).
// That is exp((q.k)*scale - max) exactly in real arithmetic and costs one v_exp_f32.

#include "common.hpp"
#include "paged_attention.hpp"

namespace mvllm {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kUnroll = 4;  // tokens in flight per row group per iteration

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Which query row, sequence and visible context a decode workgroup serves.
// Returns false when the workgroup has nothing to do in this pass.
__device__ __forceinline__ bool resolve_row(const PagedParams& p, int index, int& seq, int& row,
                                            int& visible) {
  if (p.by_row) {
    // Every query row is a unit (the fallback that also serves prefill rows):
    // find its sequence by binary search over cu_seqlens_q.
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

}  // namespace

template <typename TQ, typename TKV, int D, int GC>
__global__ __launch_bounds__(512) void paged_decode_kernel(const PagedParams p) {
  constexpr int E = Chunk<TKV>::kN;        // elements per 16-byte chunk
  constexpr int R = D / E;                 // lanes per token row
  constexpr int RG = kWave / R;            // row groups per wave
  static_assert(R >= 1 && R <= kWave && (kWave % R) == 0, "head dim / dtype mismatch");
  constexpr bool kFp8 = Elem<TKV>::kBytes == 1;

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
  const int g = lane / R;   // row group
  const int r = lane % R;   // chunk within the row

  const int32_t* table = p.block_tables + static_cast<int64_t>(seq) * p.max_blocks;
  const int first_page = sb >> p.block_shift;
  const int n_pages = sb < se ? ((se - 1) >> p.block_shift) - first_page + 1 : 0;
  const bool pages_in_lds = n_pages <= kMaxSplitPages;
  if (pages_in_lds) {
    for (int i = threadIdx.x; i < n_pages; i += blockDim.x) s_pages[i] = table[first_page + i];
  }
  __syncthreads();

  const int chunks = p.hq / p.hk / GC;                       // head chunks per kv head
  const int unit = blockIdx.z * (blockDim.x / kWave) + wave;  // (kv head, chunk)
  if (unit >= p.hk * chunks) return;
  const int kvh = unit / chunks;
  const int h0 = kvh * (p.hq / p.hk) + (unit % chunks) * GC;

  // Queries of the wave's heads, this lane's E dims, pre-scaled into log2 units.
  float qf[GC][E];
#pragma unroll
  for (int h = 0; h < GC; ++h) {
    const int64_t base = (static_cast<int64_t>(row) * p.hq + h0 + h) * D + r * E;
#pragma unroll
    for (int e = 0; e < E; ++e) qf[h][e] = Elem<TQ>::load(p.q, base + e);
  }
  const float score_scale = p.scale * kLog2e;

  float m[GC], l[GC], acc[GC][E];
#pragma unroll
  for (int h = 0; h < GC; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[h][e] = 0.0f;
  }

  const char* kbase = static_cast<const char*>(p.k_pool);
  const char* vbase = static_cast<const char*>(p.v_pool);
  constexpr int kElemBytes = Elem<TKV>::kBytes;

  for (int t0 = sb; t0 < se; t0 += RG * kUnroll) {
    u32x4 kw[kUnroll], vw[kUnroll];
    bool valid[kUnroll];
    float ks[kUnroll], vs[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int tok = t0 + u * RG + g;
      valid[u] = tok < se;
      tok = valid[u] ? tok : se - 1;
      const int pi = tok >> p.block_shift;
      const int page = pages_in_lds ? s_pages[pi - first_page] : table[pi];
      const int64_t slot = (static_cast<int64_t>(page) << p.block_shift) | (tok & p.block_mask);
      const int64_t off = ((slot * p.hk + kvh) * D + r * E) * kElemBytes;
      kw[u] = load16(kbase + off);
      vw[u] = load16(vbase + off);
      if constexpr (kFp8) {
        ks[u] = p.k_scales[static_cast<int64_t>(page) * p.hk + kvh];
        vs[u] = p.v_scales[static_cast<int64_t>(page) * p.hk + kvh];
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
      float mx = m[h];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) mx = fmaxf(mx, s[u][h]);
      // A row group that has seen no valid key yet keeps m = -inf; exponentiate
      // against 0 then, so 2^(-inf - 0) = 0 instead of 2^(-inf + inf) = NaN
      // (the empty-split rule of paged_attention.cu:210-213).
      const float mu = mx == -INFINITY ? 0.0f : mx;
      const float alpha = fast_exp2(m[h] - mu);
      float sum = 0.0f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        pr[u][h] = fast_exp2(s[u][h] - mu);
        sum += pr[u][h];
      }
      l[h] = l[h] * alpha + sum;
      m[h] = mx;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[h][e] *= alpha;
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
        for (int e = 0; e < E; ++e) acc[h][e] = fmaf(w, vf[e], acc[h][e]);
      }
    }
  }

  // Merge the wave's row groups: xor partners share r and differ in g.
#pragma unroll
  for (int off = R; off < kWave; off <<= 1) {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const float mo = __shfl_xor(m[h], off, kWave);
      const float lo = __shfl_xor(l[h], off, kWave);
      const float mx = fmaxf(m[h], mo);
      const float mu = mx == -INFINITY ? 0.0f : mx;
      const float a = fast_exp2(m[h] - mu);
      const float b = fast_exp2(mo - mu);
      l[h] = l[h] * a + lo * b;
      m[h] = mx;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float other = __shfl_xor(acc[h][e], off, kWave);
        acc[h][e] = acc[h][e] * a + other * b;
      }
    }
  }

  if (g != 0) return;  // every row group now holds the same totals; one writes
  if (nsplit == 1) {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const float inv = l[h] > 0.0f ? 1.0f / l[h] : 0.0f;
      const int64_t base = (static_cast<int64_t>(row) * p.hq + h0 + h) * D + r * E;
#pragma unroll
      for (int e = 0; e < E; ++e) Elem<TQ>::store(p.out, base + e, acc[h][e] * inv);
    }
  } else {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const int64_t prow = (static_cast<int64_t>(partial_row) * p.hq + h0 + h) * p.max_splits + split;
      float* po = p.part_o + prow * D + r * E;
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        *reinterpret_cast<f32x4*>(po + e) = f32x4{acc[h][e], acc[h][e + 1], acc[h][e + 2], acc[h][e + 3]};
      }
      if (r == 0) {
        p.part_ml[prow * 2] = m[h];
        p.part_ml[prow * 2 + 1] = l[h];
      }
    }
  }
}

// Combine the split partials of every (row, query head) that was split:
// out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s. One wave per (row, head).
template <typename TQ, int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(const PagedParams p) {
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

template <typename TQ, typename TKV, int D>
hipError_t launch_decode_d(const PagedParams& p, int gc, hipStream_t stream) {
  const int units = p.hk * (p.hq / p.hk / gc);
  const int waves = units < 8 ? units : 8;
  const dim3 grid(p.max_splits, p.by_row ? p.num_tokens : p.num_seqs, (units + waves - 1) / waves);
  const dim3 block(waves * kWave);
  switch (gc) {
    case 4: paged_decode_kernel<TQ, TKV, D, 4><<<grid, block, 0, stream>>>(p); break;
    case 2: paged_decode_kernel<TQ, TKV, D, 2><<<grid, block, 0, stream>>>(p); break;
    default: paged_decode_kernel<TQ, TKV, D, 1><<<grid, block, 0, stream>>>(p); break;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.max_splits == 1) return err;
  const int heads_per_block = 4;
  const dim3 mgrid((p.hq + heads_per_block - 1) / heads_per_block,
                   p.by_row ? p.num_tokens : p.num_seqs);
  paged_decode_merge_kernel<TQ, D><<<mgrid, heads_per_block * kWave, 0, stream>>>(p);
  return hipGetLastError();
}

template <typename TQ, typename TKV>
hipError_t launch_decode_t(const PagedParams& p, int head_dim, int gc, hipStream_t stream) {
  switch (head_dim) {
    case 32: return launch_decode_d<TQ, TKV, 32>(p, gc, stream);
    case 64: return launch_decode_d<TQ, TKV, 64>(p, gc, stream);
    case 128: return launch_decode_d<TQ, TKV, 128>(p, gc, stream);
    case 256: return launch_decode_d<TQ, TKV, 256>(p, gc, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_paged_decode(const PagedParams& p, int q_dtype, int kv_dtype, int head_dim,
                               hipStream_t stream) {
  const int group = p.hq / p.hk;
  const int gc = group % 4 == 0 ? 4 : (group % 2 == 0 ? 2 : 1);
  if (kv_dtype == kFP8E4M3) {
    if (q_dtype == kBF16) return launch_decode_t<bf16_t, fp8_t>(p, head_dim, gc, stream);
    if (q_dtype == kF16) return launch_decode_t<f16_t, fp8_t>(p, head_dim, gc, stream);
    if (q_dtype == kF32) return launch_decode_t<float, fp8_t>(p, head_dim, gc, stream);
    return hipErrorInvalidValue;
  }
  if (q_dtype != kv_dtype) return hipErrorInvalidValue;
  switch (q_dtype) {
    case kF32: return launch_decode_t<float, float>(p, head_dim, gc, stream);
    case kF16: return launch_decode_t<f16_t, f16_t>(p, head_dim, gc, stream);
    case kBF16: return launch_decode_t<bf16_t, bf16_t>(p, head_dim, gc, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mvllm
