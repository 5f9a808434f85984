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
//  * work item = (sequence, column, query tile): 128 query positions of HW query heads
//    (HW = 2 heads of one GQA group when the group is even) against one kv head. Its
//    cost is the number of 64-key tiles it walks; items are laid end to end in
//    (sequence, column, query tile) order.
//  * stream schedule: one persistent workgroup per CU. An in-kernel prefix scan of the
//    per-sequence costs (no host read of device data) gives every workgroup an equal
//    share of all key tiles, whatever the spread of prefix lengths; an item cut
//    between workgroups leaves (m, l, O) partials that paged_prefill_merge_kernel
//    combines. A share's partial pieces are at most its first and its last, stored
//    in slots 2w and 2w + 1. Shares are assigned XCD by XCD. Grid schedule (more than kMaxStreamSeqs sequences): one
//    workgroup per item, whole.
//  * workgroup = 4 x HS waves: wave (hs, w) owns query positions 32w .. 32w+31 of
//    HCW = HW / HS heads. The launches use HS = HW (one head per wave): for a GQA
//    pair, 8 waves, two per SIMD, one's softmax under the other's MFMAs.
//  * K/V tiles of 64 keys are page-gathered from HBM into LDS, double buffered; page
//    ids (and fp8 scales) are fetched four tiles ahead and K/V two tiles ahead (two
//    register sets), across item boundaries, so each load has two loop iterations to
//    arrive; per-sequence metadata comes through the scalar cache.
//  * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_{bf16,f16}:
//    a lane then owns one query column and 16 keys per 32-key block, so the softmax
//    row max is an in-lane max plus one xor-32 exchange.
//  * O^T = V^T P^T on the same MFMA. The P^T operand comes straight from the score
//    accumulators (converted to bf16/fp16); the MFMA's reduction axis is keys, so the
//    accumulator's key order is used as-is and V^T is read with the same key
//    permutation. V is transposed on its way into LDS.
//  * online softmax in fp32, log2 domain, the score scale folded into the exponent's
//    FMA. The running max is raised only when a row's tile max exceeds it by more than
//    8 (so exponentials stay <= 2^8): O is rescaled a handful of times per item rather
//    than every tile, exactly (O and l always refer to the same max).
//  * causal masking only on tiles that cross the diagonal; tiles past a wave's last
//    visible key are skipped.
//  * fp8-e4m3 pools are dequantised (x * per-(page, kv head) scale) while staging
//    into LDS, and the MFMAs run in the query's 16-bit type.
//
// MFMA 32x32x16 operand layouts (lane l, l32 = l % 32, h = l / 32):
//   A[m][k]: lane holds m = l32, k = 8h .. 8h+7
//   B[k][n]: lane holds n = l32, k = 8h .. 8h+7
//   C[m][n]: lane holds n = l32, m = 8j + 4h + i for j, i in 0..3 (register 4j + i)

#include <climits>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"
#include "paged_attention.hpp"

namespace mvllm {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTileKeys = kPrefillKeyTile;
constexpr float kRescaleSlack = 8.0f;  // log2 units: exponentials stay <= 2^8

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

// Scheduling order for a block of N MFMAs fed by N LDS fragment reads issued kLook
// ahead: kLook reads, then (MFMA, read) pairs, then the last kLook MFMAs.
template <int kLook, int N>
__device__ __forceinline__ void lds_mfma_pipeline() {
  constexpr int kMfma = 0x008, kDsRead = 0x100;
  __builtin_amdgcn_sched_group_barrier(kDsRead, kLook, 0);
#pragma unroll
  for (int i = 0; i < N - kLook; ++i) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(kMfma, kLook, 0);
}

// A 16-byte global load the compiler does not track (like copy_to_lds): the value must not be used
// before an explicit vmcnt wait that names it as an operand.
__device__ __forceinline__ u32x4 load16_untracked(const char* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}

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

namespace {

// A position in the stream of work: unit u = key tile t of item (s, c, q), which has
// nt tiles; context / len of sequence s. Every field is workgroup-uniform.
struct Cursor {
  int u, s, c, q, t, nt, context, len;
  int kvh;  // kv head of column c
};

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Share index of workgroup `bid` of `n`: workgroups are dispatched to the XCDs round
// robin, so this gives the workgroups of one XCD consecutive shares (the items one L2
// serves are few, their K/V tiles reused from it).
__device__ __forceinline__ int xcd_share(int bid, int n) {
  return n % kXcds == 0 ? (bid % kXcds) * (n / kXcds) + bid / kXcds : bid;
}

// The share of workgroup `bid` of `grid` when only `shares` <= grid are used, or -1:
// each XCD takes ceil(shares / 8) consecutive shares (xcd_share when shares == grid).
__device__ __forceinline__ int xcd_share_of(int bid, int grid, int shares) {
  if (grid % kXcds != 0) return bid < shares ? bid : -1;
  const int per = (shares + kXcds - 1) / kXcds;
  const int slot = bid / kXcds;
  const int share = (bid % kXcds) * per + slot;
  return slot < per && share < shares ? share : -1;
}

// Work units of sequence s over all its items (0 for decode rows).
__device__ __forceinline__ int prefill_seq_units(int context, int len, int cols) {
  if (len <= 1) return 0;
  const int qtiles = (len + kPrefillQueryTile - 1) / kPrefillQueryTile;
  int units = 0;
  for (int q = 0; q < qtiles; ++q) units += prefill_item_tiles(context, len, q);
  return units * cols;
}

// Position `k` at unit u of the stream described by the prefix `pre` ([n + 1] work
// units before each sequence, pre[n] > u).
// The rest of a seek once the sequence is known: unit u of sequence a, whose units are
// [base, next).
__device__ __forceinline__ void seek_in(Cursor& k, const PagedParams& p, int a, int base,
                                        int next, int cols, int u) {
  k.u = u;
  k.s = a;
  k.context = sload(p.context_lens + a);
  k.len = sload(p.seq_lens + a);
  const int per_col = (next - base) / cols;
  int r = u - base;
  k.c = r / per_col;
  k.kvh = k.c / (cols / p.hk);
  r -= k.c * per_col;
  k.q = 0;
  k.nt = prefill_item_tiles(k.context, k.len, 0);
  while (r >= k.nt) {
    r -= k.nt;
    ++k.q;
    k.nt = prefill_item_tiles(k.context, k.len, k.q);
  }
  k.t = r;
}

__device__ __forceinline__ void seek(Cursor& k, const PagedParams& p, const int* pre, int n,
                                     int cols, int u) {
  int a = 0, b = n;  // invariant: pre[a] <= u < pre[b]
  while (b - a > 1) {
    const int mid = (a + b) >> 1;
    if (uniform(pre[mid]) <= u) a = mid; else b = mid;
  }
  seek_in(k, p, a, uniform(pre[a]), uniform(pre[a + 1]), cols, u);
}

// This workgroup's work units [u0, u1) and the cursor at u0; false when it has none.
// Every thread must call it: the stream schedule's prefix scan ends in a barrier. The
// stream schedule sets `share` (the workgroup's share, which names its piece slots).
template <int kThreads, bool kGridOnly = false>
__device__ __forceinline__ bool prefill_work(const PagedParams& p, int cols, int& share,
                                             int* s_prefix, Cursor& cur, int& u0, int& u1) {
  const int tid = threadIdx.x;
  const int n = p.num_seqs;
  if (!kGridOnly && p.pf_wgs > 0) {
    // Prefix scan of the sequences' work units by wave 0: each lane sums a contiguous
    // run, then a 64-lane inclusive scan.
    if (tid < kWave) {
      const int per = (n + kWave - 1) / kWave;
      const int begin = min(tid * per, n);
      const int end = min(begin + per, n);
      int run = 0;
      for (int s = begin; s < end; ++s) run += prefill_seq_units(p.context_lens[s], p.seq_lens[s], cols);
      int incl = run;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int other = __shfl_up(incl, off, kWave);
        if (tid >= off) incl += other;
      }
      int acc = incl - run;
      for (int s = begin; s < end; ++s) {
        s_prefix[s] = acc;
        acc += prefill_seq_units(p.context_lens[s], p.seq_lens[s], cols);
      }
      if (tid == kWave - 1) s_prefix[n] = incl;
    }
    __syncthreads();
    const int total = uniform(s_prefix[n]);
    if (blockIdx.x == 0) {
      for (int s = tid; s <= n; s += kThreads) p.pf_prefix[s] = s_prefix[s];
    }
    const int shares =
        static_cast<int>(prefill_stream_shares(total, gridDim.x, p.pf_share_tiles));
    share = xcd_share_of(blockIdx.x, gridDim.x, shares);
    if (share < 0) return false;  // whole workgroup: no barrier follows for it
    u0 = static_cast<int>(share_begin(share, total, shares));
    u1 = static_cast<int>(share_begin(share + 1, total, shares));
    if (u0 >= u1) return false;  // whole workgroup: no barrier follows for it
    seek(cur, p, s_prefix, n, cols, u0);
    return true;
  }
  cur.s = blockIdx.y;
  cur.len = sload(p.seq_lens + cur.s);
  cur.context = sload(p.context_lens + cur.s);
  if (cur.len <= 1) return false;  // a decode row: the decode kernel has it
  const int qtiles = (cur.len + kPrefillQueryTile - 1) / kPrefillQueryTile;
  // Query tile slowest and reversed: the longest tiles are dispatched first.
  cur.q = static_cast<int>(gridDim.z) - 1 - static_cast<int>(blockIdx.z);
  if (cur.q < 0 || cur.q >= qtiles) return false;
  cur.c = blockIdx.x;
  cur.kvh = cur.c / (cols / p.hk);
  cur.nt = prefill_item_tiles(cur.context, cur.len, cur.q);
  cur.t = 0;
  cur.u = 0;
  u0 = 0;
  u1 = cur.nt;
  return true;
}

// The split grid's piece at position `rank` (workgroup blockIdx.x / columns; the first
// pf_ranks - (pieces) positions are empty, then the pieces in rank order), computed by one
// wave from the sequences' sizes (no host read, no other launch; every workgroup
// derives the same schedule). Items (sequence, query tile) are numbered sequence by
// sequence, lane i holding item i:
//  * piece length L = max(fewest tiles, ceil(pct% of the mean tiles per CU)); an item
//    of nt tiles is cut into P = min(pieces, ceil(nt / L)) key ranges of floor-divided
//    tiles (P - 1 < nt / L, so the extra pieces number fewer than 100 cus / (pct cols)
//    and the cut items' pieces fewer than twice that: within the grid's ranks and
//    slots; an item that would still pass them, counted with every earlier item's
//    pieces, stays whole);
//  * ranks go longest piece first (ties by item index), an item's pieces consecutive;
//  * a cut item's pieces hold partial slots slot0 .. slot0 + P - 1 (prefix over the
//    cut items in index order).
// Scans are DPP; the all-pairs rank count reads every item's (longest piece,
// pieces) from LDS with broadcast loads, so no step is a chain of per-item scalar reads.
// False for an empty position (the grid is a host-side bound).
struct SplitPiece {
  int s, q, item, piece, pieces, slot0, tb, te;
};

struct SplitLds {
  int4 rec[kSplitMaxItems];  // item i: (sequence, query tile, tiles, 0)
  int2 kp[kSplitMaxItems];   // item i: (its longest piece, its pieces)
  int out[10];               // the schedule's result for the other waves
};

// Inclusive prefix sum over the wave's 64 lanes: DPP row shifts 1, 2, 4, 8 (within
// each 16-lane row; a lane whose source lies outside its row adds 0), then lane 15's
// row total broadcast into rows 1 and 3 and lane 31's into rows 2 and 3.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

__device__ __forceinline__ bool split_piece_wave(const PagedParams& p, int cols, int rank,
                                                 SplitLds& lds, SplitPiece& out) {
  const int lane = threadIdx.x % kWave;
  const int n = p.num_seqs;
  // Items in sequence order: lane s of each 64-sequence chunk lists its query tiles.
  // (One wave's LDS accesses complete in order, so its lanes read what others wrote.)
  int items = 0;
  for (int base = 0; base < n; base += kWave) {
    int len = 0, ctx = 0;
    if (base + lane < n) {
      len = p.seq_lens[base + lane];
      ctx = p.context_lens[base + lane];
    }
    const int qts = len > 1 ? (len + kPrefillQueryTile - 1) / kPrefillQueryTile : 0;
    const int pre = items + wave_inclusive_scan(qts) - qts;
    for (int q = 0; q < qts && pre + q < kSplitMaxItems; ++q) {
      lds.rec[pre + q] = make_int4(base + lane, q, prefill_item_tiles(ctx, len, q), 0);
    }
    items = __builtin_amdgcn_readlane(pre + qts, kWave - 1);
  }
  items = min(items, kSplitMaxItems);  // the host bound rules out more
  const bool have = lane < items;
  const int4 r = have ? lds.rec[lane] : make_int4(0, 0, 0, 0);
  const int nt = r.z;
  const int total = __builtin_amdgcn_readlane(wave_inclusive_scan(nt), kWave - 1);
  // pct percent of the mean tiles per CU, rounded up
  const int64_t scaled = static_cast<int64_t>(p.pf_piece_pct) * total * cols;
  int piece_len = static_cast<int>((scaled + 100 * p.pf_cus - 1) / (100 * p.pf_cus));
  piece_len = max(piece_len, max(p.pf_share_tiles, 1));
  int pcs = have ? max(min(p.pf_pieces, (nt + piece_len - 1) / piece_len), 1) : 0;
  // Extra pieces (low 16 bits) and cut items' slots (high 16 bits) before this item;
  // both stay below 64 x 64.
  const int both = (have ? pcs - 1 : 0) | ((pcs > 1 ? pcs : 0) << 16);
  const int before = wave_inclusive_scan(both) - both;
  const int extra_before = before & 0xffff, slots_before = before >> 16;
  if (pcs > 1 && (items + extra_before + pcs - 1 > p.pf_ranks || slots_before + pcs > p.pf_slots)) {
    pcs = 1;
  }
  const int cut = pcs > 1 ? pcs : 0;
  const int slot0 = wave_inclusive_scan(cut) - cut;
  // The grid's first positions are the ranks it has beyond the pieces (empty): they
  // end here, while every CU is still free, rather than after the last piece.
  const int ranks = items + __builtin_amdgcn_readlane(wave_inclusive_scan(have ? pcs - 1 : 0), kWave - 1);
  rank -= p.pf_ranks - ranks;
  if (rank < 0) return false;
  const int key = have ? (nt + pcs - 1) / pcs : 0;
  lds.kp[lane] = make_int2(key, pcs);
  // Pieces ranked before this item's first: every item's pair read with 16-byte
  // broadcast loads, all of a half issued before any is used.
  int start = 0;
#pragma unroll
  for (int h = 0; h < kSplitMaxItems; h += kSplitMaxItems / 2) {
    int4 two[kSplitMaxItems / 4];
#pragma unroll
    for (int k = 0; k < kSplitMaxItems / 4; ++k) two[k] = *reinterpret_cast<const int4*>(&lds.kp[h + 2 * k]);
#pragma unroll
    for (int k = 0; k < kSplitMaxItems / 4; ++k) {
      const int j = h + 2 * k;
      if (two[k].x > key || (two[k].x == key && j < lane)) start += two[k].y;
      if (two[k].z > key || (two[k].z == key && j + 1 < lane)) start += two[k].w;
    }
  }
  const uint64_t mine = __builtin_amdgcn_ballot_w64(have && start <= rank && rank < start + pcs);
  if (mine == 0) return false;
  const int i = __builtin_ctzll(mine);
  out.s = __builtin_amdgcn_readlane(r.x, i);
  out.q = __builtin_amdgcn_readlane(r.y, i);
  out.item = i;
  out.pieces = __builtin_amdgcn_readlane(pcs, i);
  out.piece = rank - __builtin_amdgcn_readlane(start, i);
  out.slot0 = __builtin_amdgcn_readlane(slot0, i);
  const int nti = __builtin_amdgcn_readlane(nt, i);
  out.tb = out.piece * nti / out.pieces;
  out.te = (out.piece + 1) * nti / out.pieces;
  return true;
}

// Every wave's copy of the schedule: wave 0 computes it, the workgroup's barrier
// publishes it. False (for the whole workgroup) past the last piece.
__device__ __forceinline__ bool split_piece(const PagedParams& p, int cols, int rank,
                                            SplitLds& lds, SplitPiece& out) {
  if (threadIdx.x < kWave) {
    SplitPiece mine{};
    const bool got = split_piece_wave(p, cols, rank, lds, mine);
    if (threadIdx.x == 0) {
      lds.out[0] = got ? 1 : 0;
      lds.out[1] = mine.s;
      lds.out[2] = mine.q;
      lds.out[3] = mine.item;
      lds.out[4] = mine.piece;
      lds.out[5] = mine.pieces;
      lds.out[6] = mine.slot0;
      lds.out[7] = mine.tb;
      lds.out[8] = mine.te;
    }
  }
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(lds.out[0]) == 0) return false;
  out.s = __builtin_amdgcn_readfirstlane(lds.out[1]);
  out.q = __builtin_amdgcn_readfirstlane(lds.out[2]);
  out.item = __builtin_amdgcn_readfirstlane(lds.out[3]);
  out.piece = __builtin_amdgcn_readfirstlane(lds.out[4]);
  out.pieces = __builtin_amdgcn_readfirstlane(lds.out[5]);
  out.slot0 = __builtin_amdgcn_readfirstlane(lds.out[6]);
  out.tb = __builtin_amdgcn_readfirstlane(lds.out[7]);
  out.te = __builtin_amdgcn_readfirstlane(lds.out[8]);
  return true;
}

}  // namespace

template <typename TQ, typename TKV, int D, int HCW, int HS>
__global__ __launch_bounds__(256 * HS) void paged_prefill_kernel(const PagedParams p) {
  constexpr int kThreads = 256 * HS;
  constexpr int HW = HCW * HS;                  // query heads per work item
  constexpr int kKStride = D + 8;               // K tile row, 16-bit elements (16 B pad)
  constexpr int kVStride = kTileKeys + 4;       // V^T tile row, 16-bit elements (8 B pad)
  constexpr int kKSteps = D / 16;               // MFMA k-steps over the head dim
  constexpr int kDBlocks = D / 32;              // 32-row blocks of O^T
  constexpr int kKUnits = kTileKeys * D / 8 / kThreads;  // 16-byte K pieces per thread
  constexpr int kVKeys = kKUnits < 4 ? kKUnits : 4;       // keys per V staging unit
  constexpr int kVGroups = kTileKeys / kVKeys;
  constexpr int kVUnits = kVGroups * (D / 8) / kThreads;  // V units per thread
  constexpr int kElemBytes = Elem<TKV>::kBytes;
  constexpr bool kFp8 = kElemBytes == 1;
  static_assert(kKUnits >= 1 && kVUnits >= 1 && kVGroups * (D / 8) % kThreads == 0,
                "staging map does not cover the tile");
  static_assert(kTileKeys == kPrefillKeyTile && 32 * 4 == kPrefillQueryTile, "tile sizes");

  __shared__ __align__(16) uint16_t k_lds[2][kTileKeys * kKStride];
  __shared__ __align__(16) uint16_t v_lds[2][D * kVStride];
  __shared__ int s_prefix[kMaxStreamSeqs + 1];

  const int tid = threadIdx.x;
  const int wave = uniform(tid / kWave);
  const int lane = tid % kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int hs = wave / 4;   // head set
  const int wq = wave % 4;   // 32-position query block

  const int n = p.num_seqs;
  const int group = p.hq / p.hk;
  const int chunks = group / HW;
  const int cols = p.hk * chunks;
  const bool stream = p.pf_wgs > 0;
  int share = xcd_share(blockIdx.x, gridDim.x);

  // ---- this workgroup's units [u0, u1) and the cursor at u0.
  Cursor cur;
  int u0, u1;
  if (!prefill_work<kThreads>(p, cols, share, s_prefix, cur, u0, u1)) return;
  auto advance = [&](Cursor& k) __attribute__((always_inline)) {
    ++k.u;
    if (++k.t < k.nt) return;
    if (stream) {
      seek(k, p, s_prefix, n, cols, k.u);
    } else {
      k.t = 0;  // grid items are never walked past their end
    }
  };

  // c_eff = |scale| * log2(e), and the sign of a negative scale moved into Q (exact in
  // 16-bit floats), so the max of raw scores is the max of scaled scores.
  const float raw_c = p.scale * kLog2e;
  const float score_c = fmaxf(fabsf(raw_c), 1e-30f);
  const uint32_t q_sign = raw_c < 0.0f ? 0x80008000u : 0u;

  const char* kpool = static_cast<const char*>(p.k_pool);
  const char* vpool = static_cast<const char*>(p.v_pool);
  const int64_t row_bytes = p.kv_row_bytes;  // one slot's K row
  const int64_t page_bytes = row_bytes << p.table_shift;  // per unit of a table entry

  // ---- staging maps. K unit u: key (idx / (D/8)), dims 8 * (idx % (D/8)) .. +7, so 16
  // lanes read one 16-byte-chunked key row. V unit u: keys kVKeys * (idx % kVGroups)
  // .. + kVKeys - 1 at dims 8 * (idx / kVGroups) .. +7, transposed into V^T.
  auto k_key = [&](int u) __attribute__((always_inline)) { return (tid + u * kThreads) / (D / 8); };
  auto k_dim = [&](int u) __attribute__((always_inline)) { return ((tid + u * kThreads) % (D / 8)) * 8; };
  auto v_grp = [&](int u) __attribute__((always_inline)) { return (tid + u * kThreads) % kVGroups; };
  auto v_dim = [&](int u) __attribute__((always_inline)) { return ((tid + u * kThreads) / kVGroups) * 8; };

  // Two register sets, by the parity of the step they serve (a compile-time index, so
  // the sets stay in distinct registers): page ids are fetched four steps ahead and
  // K/V two steps ahead, each consumed two loop iterations after it was issued.
  int kpg[2][kKUnits], vpg[2][kVUnits][kVKeys];
  float ksc[2][kKUnits], vsc[2][kVUnits][kVKeys];
  auto fetch_pages = [&](const Cursor& k, auto set) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    const int32_t* table = p.block_tables + static_cast<int64_t>(k.s) * p.max_blocks;
    const int key0 = k.t * kTileKeys;
    const int last = k.context - 1;
    const int kvh = k.c / chunks;  // fp8 scales only
#pragma unroll
    for (int u = 0; u < kKUnits; ++u) kpg[S][u] = table[min(key0 + k_key(u), last) >> p.block_shift];
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
#pragma unroll
      for (int j = 0; j < kVKeys; ++j) {
        vpg[S][u][j] = table[min(key0 + kVKeys * v_grp(u) + j, last) >> p.block_shift];
      }
    }
    if constexpr (kFp8) {
#pragma unroll
      for (int u = 0; u < kKUnits; ++u) ksc[S][u] = p.k_scales[static_cast<int64_t>(kpg[S][u]) * p.hk + kvh];
#pragma unroll
      for (int u = 0; u < kVUnits; ++u) {
#pragma unroll
        for (int j = 0; j < kVKeys; ++j) vsc[S][u][j] = p.v_scales[static_cast<int64_t>(vpg[S][u][j]) * p.hk + kvh];
      }
    }
  };

  u32x4 kreg[2][kKUnits];
  u32x4 vreg[2][kVUnits][kVKeys];
  // Byte offset of (page, key within the page, kv head, dims): the page's offset is one
  // 32 x 32 -> 64-bit multiply-add, the rest fits 32 bits (a page is far below 4 GiB).
  const uint32_t page_bytes32 = static_cast<uint32_t>(page_bytes);
  auto pool_offset = [&](int page, int key, uint32_t inner) __attribute__((always_inline)) -> uint64_t {
    return static_cast<uint64_t>(static_cast<uint32_t>(page)) * page_bytes32 +
           (static_cast<uint32_t>(key & p.block_mask) * static_cast<uint32_t>(row_bytes) + inner);
  };
  auto load_tile = [&](const Cursor& k, auto set) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    const int key0 = k.t * kTileKeys;
    const int last = k.context - 1;
    const uint32_t head_off = static_cast<uint32_t>((k.c / chunks) * p.kv_head_bytes);
#pragma unroll
    for (int u = 0; u < kKUnits; ++u) {
      const int key = min(key0 + k_key(u), last);
      const uint64_t off = pool_offset(kpg[S][u], key, head_off + k_dim(u) * kElemBytes);
      kreg[S][u] = Stage<TQ, TKV>::load(kpool + off, kFp8 ? ksc[S][u] : 1.0f);
    }
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
#pragma unroll
      for (int j = 0; j < kVKeys; ++j) {
        const int key = min(key0 + kVKeys * v_grp(u) + j, last);
        const uint64_t off = pool_offset(vpg[S][u][j], key, head_off + v_dim(u) * kElemBytes);
        vreg[S][u][j] = Stage<TQ, TKV>::load(vpool + off, kFp8 ? vsc[S][u][j] : 1.0f);
      }
    }
  };
  auto store_tile = [&](int buf, auto set) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
#pragma unroll
    for (int u = 0; u < kKUnits; ++u) {
      *reinterpret_cast<u32x4*>(&k_lds[buf][k_key(u) * kKStride + k_dim(u)]) = kreg[S][u];
    }
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int sh = (e & 1) * 16;
        uint16_t* dst = &v_lds[buf][(v_dim(u) + e) * kVStride + kVKeys * v_grp(u)];
        // v_perm_b32 selector: low halves (bytes 0,1 of each) or high halves (2,3) of
        // two dwords, the first operand's in the upper half of the result.
        const uint32_t sel = sh == 0 ? 0x05040100u : 0x07060302u;
        if constexpr (kVKeys == 4) {
          *reinterpret_cast<u32x2*>(dst) =
              u32x2{__builtin_amdgcn_perm(vreg[S][u][1][e >> 1], vreg[S][u][0][e >> 1], sel),
                    __builtin_amdgcn_perm(vreg[S][u][3][e >> 1], vreg[S][u][2][e >> 1], sel)};
        } else if constexpr (kVKeys == 2) {
          *reinterpret_cast<uint32_t*>(dst) =
              __builtin_amdgcn_perm(vreg[S][u][1][e >> 1], vreg[S][u][0][e >> 1], sel);
        } else {
          *dst = static_cast<uint16_t>(vreg[S][u][0][e >> 1] >> sh);
        }
      }
    }
  };

  // ---- per-item state of this wave.
  u32x4 qop[HCW][kKSteps];
  f32x16 o[HCW][kDBlocks];
  float m_run[HCW], l_run[HCW];
  int w_first = 0, w_kv_end = 0, w_kv_full = 0, my_local = 0, my_visible = 0, head0 = 0;
  int row_base = 0, piece_t0 = 0, piece_u0 = 0;
  bool w_active = false, my_valid = false;

  auto begin_piece = [&]() __attribute__((always_inline)) {
    const int offset = cur.context - cur.len;
    const int qb = cur.q * kPrefillQueryTile;
    w_first = qb + 32 * wq;
    w_active = w_first < cur.len;
    w_kv_end = offset + min(w_first + 32, cur.len);
    w_kv_full = offset + w_first + 1;
    my_local = w_first + l32;
    my_valid = my_local < cur.len;
    my_visible = offset + my_local + 1;
    row_base = sload(p.cu_seqlens_q + cur.s);
    head0 = (cur.c / chunks) * group + (cur.c % chunks) * HW + hs * HCW;
    piece_t0 = cur.t;
    piece_u0 = cur.u;
    const int local = min(my_local, cur.len - 1);
#pragma unroll
    for (int h = 0; h < HCW; ++h) {
      const int64_t qrow = static_cast<int64_t>(row_base + local) * p.hq + head0 + h;
      const char* qp = static_cast<const char*>(p.q) + (qrow * D + 8 * hsel) * 2;
#pragma unroll
      for (int ks = 0; ks < kKSteps; ++ks) qop[h][ks] = load16(qp + ks * 32) ^ q_sign;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o[h][db] = f32x16{};
      m_run[h] = -INFINITY;
      l_run[h] = 0.0f;
    }
  };

  auto compute = [&](int buf) __attribute__((always_inline)) {
    const int key0 = cur.t * kTileKeys;
    if (!w_active || key0 >= w_kv_end) return;
    const uint16_t* kt = k_lds[buf];
    const uint16_t* vt = v_lds[buf];

    // S^T = K Q^T for two 32-key blocks; one K fragment feeds every head's MFMA.
    f32x16 s[HCW][2];
#pragma unroll
    for (int h = 0; h < HCW; ++h) {
      s[h][0] = f32x16{};
      s[h][1] = f32x16{};
    }
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(kt + (kb * 32 + l32) * kKStride + 8 * hsel + ks * 16);
#pragma unroll
        for (int h = 0; h < HCW; ++h) s[h][kb] = Mma<TQ>::run(a, qop[h][ks], s[h][kb]);
      }
    }

    // Causal mask, on tiles crossing the diagonal only: score (kb, r) of this lane is
    // key key0 + 4*hsel + (32kb + 8(r/4) + r%4); visible while below my_visible.
    if (key0 + kTileKeys > w_kv_full) {
      asm volatile("" ::: "memory");  // keep this a branch: most tiles need no mask
      const int lim = my_valid ? my_visible - key0 - 4 * hsel : INT_MIN;
#pragma unroll
      for (int h = 0; h < HCW; ++h) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (kb * 32 + 8 * (r >> 2) + (r & 3) >= lim) s[h][kb][r] = -INFINITY;
          }
        }
      }
    }

    // Online softmax per head on raw scores; P^T operands straight from the registers.
    u32x4 pop[HCW][4];
#pragma unroll
    for (int h = 0; h < HCW; ++h) {
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[h][kb][r]);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave)) * score_c;
      if (__builtin_amdgcn_ballot_w64(tmax > m_run[h] + kRescaleSlack) != 0) {
        const float m_new = fmaxf(m_run[h], tmax);
        const float alpha = m_new == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[h] - m_new);
        m_run[h] = m_new;
        l_run[h] *= alpha;
#pragma unroll
        for (int db = 0; db < kDBlocks; ++db) o[h][db] *= alpha;
      }
      const float neg_mu = m_run[h] == -INFINITY ? 0.0f : -m_run[h];
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pv[e] = __builtin_amdgcn_exp2f(fmaf(s[h][kb][8 * half + e], score_c, neg_mu));
            psum += pv[e];
          }
          pop[h][2 * kb + half] =
              u32x4{Mma<TQ>::pack2(pv[0], pv[1]), Mma<TQ>::pack2(pv[2], pv[3]),
                    Mma<TQ>::pack2(pv[4], pv[5]), Mma<TQ>::pack2(pv[6], pv[7])};
        }
      }
      l_run[h] += psum;
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
        for (int h = 0; h < HCW; ++h) o[h][db] = Mma<TQ>::run(a, pop[h][ks], o[h][db]);
      }
    }
  };

  auto end_piece = [&]() __attribute__((always_inline)) {
    if (!w_active || !my_valid) return;
    const bool whole = piece_t0 == 0 && cur.t == cur.nt - 1;
    const int64_t slot = 2 * static_cast<int64_t>(share) + (piece_u0 == u0 ? 0 : 1);
#pragma unroll
    for (int h = 0; h < HCW; ++h) {
      const float l_tot = l_run[h] + __shfl_xor(l_run[h], 32, kWave);
      if (whole) {
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
      } else {
        // A piece's output normalised by its own sum, in fp32 (a 16-bit partial would
        // round the result twice), plus its (max, sum) for the merge's weights.
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        const int64_t prow = (slot * HW + hs * HCW + h) * kPrefillQueryTile +
                             (my_local - cur.q * kPrefillQueryTile);
        float* po = p.pf_o + prow * D;
#pragma unroll
        for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int d = db * 32 + 8 * j + 4 * hsel;
            *reinterpret_cast<f32x4*>(po + d) =
                f32x4{o[h][db][4 * j] * inv, o[h][db][4 * j + 1] * inv,
                      o[h][db][4 * j + 2] * inv, o[h][db][4 * j + 3] * inv};
          }
        }
        if (hsel == 0) {
          *reinterpret_cast<float2*>(p.pf_ml + prow * 2) = make_float2(m_run[h], l_tot);
        }
      }
    }
  };

  // ---- the tile loop over [u0, u1). Step x's page ids and K/V live in register set
  // (x - u0) & 1; cursor `lc` is at the last step loaded, `fc` at the last fetched.
  // sched_barrier keeps the scheduler from sinking the prefetches below the
  // computation that is meant to hide their latency.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  Cursor lc = cur;
  fetch_pages(lc, I0{});
  load_tile(lc, I0{});
  if (u0 + 1 < u1) {
    advance(lc);
    fetch_pages(lc, I1{});
    load_tile(lc, I1{});
  }
  Cursor fc = lc;
  if (u0 + 2 < u1) {
    advance(fc);
    fetch_pages(fc, I0{});
  }
  if (u0 + 3 < u1) {
    advance(fc);
    fetch_pages(fc, I1{});
  }
  auto step_body = [&](int step, auto set) __attribute__((always_inline)) {
    if (step == u0 || cur.t == 0) begin_piece();
    store_tile(decltype(set)::value, set);
    __syncthreads();
    if (step + 2 < u1) {
      advance(lc);
      load_tile(lc, set);
    }
    if (step + 4 < u1) {
      advance(fc);
      fetch_pages(fc, set);
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(decltype(set)::value);
    if (step + 1 == u1 || cur.t + 1 == cur.nt) end_piece();
    if (step + 1 < u1) advance(cur);
  };
  for (int step = u0; step < u1; step += 2) {
    step_body(step, I0{});
    if (step + 1 < u1) step_body(step + 1, I1{});
  }
}

// ------------------------------------------------------------- direct-to-LDS staging
//
// 16-bit pools, D = 128, pages of at least 16 keys, scale > 0. Same work items,
// schedules, wave roles, softmax and partial slots as paged_prefill_kernel; what
// differs is how a tile reaches LDS and how the waits are placed:
//  * a wave stages KW = 64 / waves consecutive keys of every tile; they lie in one
//    page, so the page id is a scalar load and every pool address is a scalar page
//    base plus a per-lane constant (the key's row within the page, clamped to the
//    sequence's last key on its last tile).
//  * K goes from HBM straight into LDS with global_load_lds_dwordx4 (1 KB = 4 keys per
//    instruction, lane i to byte 16 i): no registers, no LDS store instructions. Rows
//    are 256 B; chunk c of key r is stored at chunk c ^ (r & 7), so the eight keys an
//    MFMA fragment read serves per LDS cycle fall in distinct banks.
//  * V is loaded into registers two tiles ahead and written transposed (v_perm pairs)
//    into V^T rows of 64 keys, ordered as the P^T operand lists them (per 16 keys:
//    4h..4h+3 then 8+4h..8+4h+3 in chunk 2ks + h), so a PV operand is one
//    ds_read_b128; the chunks of row d are XOR-swizzled by (d ^ d >> 3) & 7.
//  * three K buffers, three V^T buffers and three V register sets, each a separate
//    array picked at compile time (the loop is unrolled by three): the compiler's
//    wait-count pass then sees that the copies in flight write other arrays than
//    the ones a step reads and writes, and does not drain them before every LDS
//    access. Tiles t + 1 and t + 2 are in flight while t is computed.
//  * before a tile's barrier each wave waits (vmcnt) for its own copies of that tile
//    only, so the barrier publishes the whole tile.
template <typename TQ, int HS, bool kStream>
__global__ __launch_bounds__(256 * HS) void paged_prefill_lds_kernel(const PagedParams p) {
  constexpr int D = 128;
  constexpr int kThreads = 256 * HS;
  constexpr int kWaves = 4 * HS;
  constexpr int HW = HS;                  // query heads per work item, one per wave set
  constexpr int KW = kTileKeys / kWaves;  // keys of a tile staged by one wave (16 or 8)
  constexpr int kCopies = KW / 4;         // 1 KB direct loads per wave per tile
  constexpr int KV = KW / 4;              // V keys per lane: 4 key groups x 16 dim chunks
  constexpr int kKSteps = D / 16;
  constexpr int kDBlocks = D / 32;
  constexpr int kRow = D * 2;             // bytes of one key row in LDS
  constexpr int kTileBytes = kTileKeys * kRow;
  constexpr int kVRow = kTileKeys * 2;    // bytes of one V^T row
  // Copies one tile's stage issues per lane (K and V). Every vector-memory load in the
  // tile loop is untracked asm and the stages are issued in tile order, so waiting down
  // to kStageOps outstanding completes everything but the newest stage.
  constexpr int kStageOps = 2 * kCopies;
  static_assert(KV == 2 || KV == 4, "V staging map");
  static_assert(kTileKeys == kPrefillKeyTile && 32 * 4 == kPrefillQueryTile, "tile sizes");

  __shared__ __align__(16) char k_lds0[kTileBytes];
  __shared__ __align__(16) char k_lds1[kTileBytes];
  __shared__ __align__(16) char k_lds2[kTileBytes];
  __shared__ __align__(16) char r_lds0[kTileBytes];
  __shared__ __align__(16) char r_lds1[kTileBytes];
  __shared__ __align__(16) char r_lds2[kTileBytes];
  __shared__ __align__(1024) char v_lds[2][kTileBytes];  // row addresses keep bits 4..6 clear
  __shared__ int s_prefix[kMaxStreamSeqs + 1];
  auto k_arr = [&](auto slot) __attribute__((always_inline)) -> char* {
    constexpr int X = decltype(slot)::value;
    if constexpr (X == 0) return k_lds0; else if constexpr (X == 1) return k_lds1; else return k_lds2;
  };
  auto r_arr = [&](auto slot) __attribute__((always_inline)) -> char* {
    constexpr int X = decltype(slot)::value;
    if constexpr (X == 0) return r_lds0; else if constexpr (X == 1) return r_lds1; else return r_lds2;
  };

  const int tid = threadIdx.x;
  const int wave = uniform(tid / kWave);
  const int lane = tid % kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int hs = wave / 4;  // head of the pair
  const int wq = wave % 4;  // 32-position query block

  const int n = p.num_seqs;
  const int group = p.hq / p.hk;
  const int chunks = group / HW;
  const int cols = p.hk * chunks;
  // Compiled per schedule: the grid's kernel carries none of the stream's cursor
  // seeking (whose registers otherwise spill into the tile loop).
  constexpr bool stream = kStream;
  int share = xcd_share(blockIdx.x, gridDim.x);

  Cursor cur;
  int u0, u1;
  if (!prefill_work<kThreads, !kStream>(p, cols, share, s_prefix, cur, u0, u1)) return;
  auto advance = [&](Cursor& k) __attribute__((always_inline)) {
    ++k.u;
    if (++k.t < k.nt) return;
    if (stream) {
      seek(k, p, s_prefix, n, cols, k.u);
    } else {
      k.t = 0;  // grid items are never walked past their end
    }
  };

  const float score_c = p.scale * kLog2e;  // > 0 (the dispatcher's condition)

  const char* kpool = static_cast<const char*>(p.k_pool);
  const char* vpool = static_cast<const char*>(p.v_pool);
  const uint32_t row_bytes = static_cast<uint32_t>(p.kv_row_bytes);  // one slot's K row
  const uint64_t page_bytes = static_cast<uint64_t>(row_bytes) << p.table_shift;  // per table unit

  // ---- per-lane constants of the staging and fragment maps.
  // K copy j: LDS chunk (lane % 16) of key KW*wave + 4j + lane/16 holds logical chunk
  // (lane % 16) ^ (key & 7) (KW * wave is a multiple of 8).
  uint32_t k_src_chunk[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; ++j) k_src_chunk[j] = (((lane & 15) ^ ((4 * j + (lane >> 4)) & 7)) * 16);
  // V transpose: lane reads keys KW*wave + KV*(lane/16) + j at dims 8*(lane%16) .. +7.
  const int v_chunk = lane & 15;
  const int v_key = KW * wave + KV * (lane >> 4);  // tile-local, a multiple of KV
  // Its V^T destination: row 8*v_chunk + e, logical chunk 2*(key>>4) + ((key>>2)&1),
  // element 4*((key>>3)&1) + (key&3); row d's chunks are swizzled by (d ^ d>>3) & 7,
  // which for d = 8*v_chunk + e is (v_chunk ^ e) & 7.
  const int vt_chunk = (2 * (v_key >> 4) + ((v_key >> 2) & 1)) ^ (v_chunk & 7);
  const uint32_t vt_dst = static_cast<uint32_t>(8 * v_chunk * kVRow + (4 * ((v_key >> 3) & 1) + (v_key & 3)) * 2);
  // Fragment reads. K (kb, ks): key 32kb + l32, chunk 2ks + hsel.
  uint32_t k_rd[kKSteps];
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) k_rd[ks] = l32 * kRow + (((2 * ks + hsel) ^ (l32 & 7)) * 16);
  // V^T (db, ks): row d = 32db + l32, chunk 2ks + hsel; (d ^ d>>3) & 7 =
  // ((l32 ^ l32>>3) & 7) ^ 4(db & 1).
  uint32_t v_rd[2][4];
  {
    const int f0 = (l32 ^ (l32 >> 3)) & 7;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) v_rd[par][ks] = l32 * kVRow + ((((2 * ks + hsel) ^ f0 ^ (4 * par)) & 7) * 16);
    }
  }

  // Page id of this wave's keys of tile k (clamped to the sequence's last key).
  auto page_of = [&](const Cursor& k) __attribute__((always_inline)) -> int {
    const int key0 = min(k.t * kTileKeys + KW * wave, k.context - 1);
    // An s_load result is already uniform; not reading it through readfirstlane lets
    // its wait fall at the first use, a step later.
    return sload(p.block_tables + static_cast<int64_t>(k.s) * p.max_blocks + (key0 >> p.block_shift));
  };
  // Issue tile k's K and V copies into slot `slot`: K rows swizzled, V rows as they are.
  // Per-lane source offsets of copy j within the wave's first key row: key 4j + lane/16.
  uint32_t k_src_off[kCopies], v_src_off[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; ++j) {
    k_src_off[j] = static_cast<uint32_t>(4 * j + (lane >> 4)) * row_bytes + k_src_chunk[j];
    v_src_off[j] = static_cast<uint32_t>(4 * j + (lane >> 4)) * row_bytes + (lane & 15) * 16;
  }
  auto stage = [&](const Cursor& k, int page, auto slot) __attribute__((always_inline)) {
    const uint32_t kdst = lds_address(k_arr(slot) + KW * wave * kRow);
    const uint32_t rdst = lds_address(r_arr(slot) + KW * wave * kRow);
    const int key0 = k.t * kTileKeys + KW * wave;
    const int last = k.context - 1;
    const uint64_t head = static_cast<uint64_t>(static_cast<uint32_t>(page)) * page_bytes +
                          static_cast<uint32_t>(k.kvh * static_cast<uint32_t>(p.kv_head_bytes));
    if (key0 + KW - 1 <= last) {
      // The wave's keys are whole: their first row joins the scalar base.
      const uint64_t base = head + static_cast<uint32_t>(key0 & p.block_mask) * row_bytes;
#pragma unroll
      for (int j = 0; j < kCopies; ++j) {
        copy_to_lds(kpool + base, k_src_off[j], kdst + 4 * j * kRow);
        copy_to_lds(vpool + base, v_src_off[j], rdst + 4 * j * kRow);
      }
    } else {
      // The sequence's last tile: rows past the last key repeat it.
#pragma unroll
      for (int j = 0; j < kCopies; ++j) {
        const uint32_t row = static_cast<uint32_t>(min(key0 + 4 * j + (lane >> 4), last) & p.block_mask) * row_bytes;
        copy_to_lds(kpool + head, row + k_src_chunk[j], kdst + 4 * j * kRow);
        copy_to_lds(vpool + head, row + (lane & 15) * 16, rdst + 4 * j * kRow);
      }
    }
  };
  // Transpose this wave's V rows of slot `slot` (tile-local keys v_key .. v_key + KV - 1,
  // dims 8 * v_chunk .. +7 per lane) into V^T buffer `vbuf`. Row 8 * v_chunk + e holds
  // them in chunk vt_chunk ^ e: a V^T address has the chunk in bits 4..6 and nothing
  // else there, so the swizzle is one XOR of the lane's row-0 address.
  typedef __attribute__((address_space(3))) uint32_t lds_u32;
  typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
  auto store_v = [&](auto slot, int vbuf) __attribute__((always_inline)) {
    const char* raw = r_arr(slot) + v_key * kRow + v_chunk * 16;
    u32x4 vr[KV];
#pragma unroll
    for (int j = 0; j < KV; ++j) vr[j] = *reinterpret_cast<const u32x4*>(raw + j * kRow);
    const uint32_t row0 = lds_address(v_lds[vbuf]) + vt_dst + (vt_chunk & 7) * 16;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // v_perm_b32 selector: low halves (bytes 0,1 of each) or high halves (2,3) of two
      // dwords, the first operand's in the upper half of the result.
      const uint32_t sel = (e & 1) == 0 ? 0x05040100u : 0x07060302u;
      const uint32_t addr = (row0 ^ (e * 16)) + e * kVRow;
      if constexpr (KV == 2) {
        *reinterpret_cast<lds_u32*>(addr) = __builtin_amdgcn_perm(vr[1][e >> 1], vr[0][e >> 1], sel);
      } else {
        *reinterpret_cast<lds_u32x2*>(addr) = u32x2{__builtin_amdgcn_perm(vr[1][e >> 1], vr[0][e >> 1], sel),
                                                    __builtin_amdgcn_perm(vr[3][e >> 1], vr[2][e >> 1], sel)};
      }
    }
  };

  // ---- per-item state of this wave (one head, 32 query positions).
  u32x4 qop[kKSteps];
  f32x16 o[kDBlocks];
  float m_run = -INFINITY, l_run = 0.0f;
  int w_kv_end = 0, w_kv_full = 0, my_local = 0, my_visible = 0, head0 = 0;
  int row_base = 0, piece_t0 = 0, piece_u0 = 0;
  bool w_active = false, my_valid = false;

  auto begin_piece = [&]() __attribute__((always_inline)) {
    const int offset = cur.context - cur.len;
    const int w_first = cur.q * kPrefillQueryTile + 32 * wq;
    w_active = w_first < cur.len;
    w_kv_end = offset + min(w_first + 32, cur.len);
    w_kv_full = offset + w_first + 1;
    my_local = w_first + l32;
    my_valid = my_local < cur.len;
    my_visible = offset + my_local + 1;
    row_base = sload(p.cu_seqlens_q + cur.s);
    head0 = (cur.c / chunks) * group + (cur.c % chunks) * HW + hs;
    piece_t0 = cur.t;
    piece_u0 = cur.u;
    const int local = min(my_local, cur.len - 1);
    const int64_t qrow = static_cast<int64_t>(row_base + local) * p.hq + head0;
    const char* qp = static_cast<const char*>(p.q) + (qrow * D + 8 * hsel) * 2;
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) qop[ks] = load16_untracked(qp + ks * 32);
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) o[db] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.0f;
  };

  auto compute = [&](auto slot, int vbuf) __attribute__((always_inline)) {
    const int key0 = cur.t * kTileKeys;
    if (!w_active || key0 >= w_kv_end) return;
    const char* kt = k_arr(slot);
    const char* vt = v_lds[vbuf];

    // Fragments are read kLook MFMAs ahead of their use, so several LDS reads are in
    // flight behind each MFMA (two in flight left the MFMAs waiting on LDS latency).
    constexpr int kLook = 4;
    f32x16 s[2] = {f32x16{}, f32x16{}};
    {
      auto k_frag = [&](int i) __attribute__((always_inline)) {
        return *reinterpret_cast<const u32x4*>(kt + (i & 1) * 32 * kRow + k_rd[i >> 1]);
      };
      u32x4 fa[kLook];
#pragma unroll
      for (int i = 0; i < kLook; ++i) fa[i] = k_frag(i);
#pragma unroll
      for (int i = 0; i < 2 * kKSteps; ++i) {
        const u32x4 a = fa[i % kLook];
        if (i + kLook < 2 * kKSteps) fa[i % kLook] = k_frag(i + kLook);
        s[i & 1] = Mma<TQ>::run(a, qop[i >> 1], s[i & 1]);
      }
      // Keep that order: the scheduler otherwise reuses one fragment register and
      // waits for each read right before its MFMA.
      lds_mfma_pipeline<kLook, 2 * kKSteps>();
    }

    // Causal mask on tiles crossing the diagonal: score (kb, r) of this lane is key
    // key0 + 4*hsel + 32kb + 8(r/4) + r%4, visible while below my_visible.
    if (key0 + kTileKeys > w_kv_full) {
      asm volatile("" ::: "memory");  // keep this a branch: most tiles need no mask
      const int lim = my_valid ? my_visible - key0 - 4 * hsel : INT_MIN;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (kb * 32 + 8 * (r >> 2) + (r & 3) >= lim) s[kb][r] = -INFINITY;
        }
      }
    }

    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[kb][r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave)) * score_c;
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kRescaleSlack) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_new == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o[db] *= alpha;
    }
    const float neg_mu = m_run == -INFINITY ? 0.0f : -m_run;
    float psum = 0.0f;
    u32x4 pop[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * half + e], score_c, neg_mu));
          psum += pv[e];
        }
        pop[2 * kb + half] = u32x4{Mma<TQ>::pack2(pv[0], pv[1]), Mma<TQ>::pack2(pv[2], pv[3]),
                                   Mma<TQ>::pack2(pv[4], pv[5]), Mma<TQ>::pack2(pv[6], pv[7])};
      }
    }
    l_run += psum;

    // O^T += V^T P^T: operand (db, ks) is row 32db + l32, logical chunk 2ks + hsel.
    {
      auto v_frag = [&](int i) __attribute__((always_inline)) {
        const int db = i & 3, ks = i >> 2;
        return *reinterpret_cast<const u32x4*>(vt + db * 32 * kVRow + v_rd[db & 1][ks]);
      };
      u32x4 fa[kLook];
#pragma unroll
      for (int i = 0; i < kLook; ++i) fa[i] = v_frag(i);
#pragma unroll
      for (int i = 0; i < kDBlocks * 4; ++i) {
        const u32x4 a = fa[i % kLook];
        if (i + kLook < kDBlocks * 4) fa[i % kLook] = v_frag(i + kLook);
        o[i & 3] = Mma<TQ>::run(a, pop[i >> 2], o[i & 3]);
      }
      lds_mfma_pipeline<kLook, kDBlocks * 4>();
    }
  };

  auto end_piece = [&]() __attribute__((always_inline)) {
    if (!w_active || !my_valid) return;
    const bool whole = piece_t0 == 0 && cur.t == cur.nt - 1;
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (whole) {
      const int64_t orow = (static_cast<int64_t>(row_base + my_local) * p.hq + head0) * D;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = db * 32 + 8 * j + 4 * hsel;
          float r[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) r[i] = o[db][4 * j + i] * inv;
          *reinterpret_cast<u32x2*>(static_cast<char*>(p.out) + (orow + d) * 2) =
              u32x2{Mma<TQ>::pack2(r[0], r[1]), Mma<TQ>::pack2(r[2], r[3])};
        }
      }
    } else {
      const int64_t slot = 2 * static_cast<int64_t>(share) + (piece_u0 == u0 ? 0 : 1);
      const int64_t prow = (slot * HW + hs) * kPrefillQueryTile + (my_local - cur.q * kPrefillQueryTile);
      float* po = p.pf_o + prow * D;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = db * 32 + 8 * j + 4 * hsel;
          *reinterpret_cast<f32x4*>(po + d) = f32x4{o[db][4 * j] * inv, o[db][4 * j + 1] * inv,
                                                    o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv};
        }
      }
      if (hsel == 0) *reinterpret_cast<float2*>(p.pf_ml + prow * 2) = make_float2(m_run, l_tot);
    }
  };

  // ---- the tile loop. Tile x uses slot (x - u0) % 3 of every staging array. Every
  // step issues the copies and loads of tile step + 2 (past the end, of the last tile
  // again, so that every step issues the same instructions and the wait counts hold).
  // Page ids are fetched three steps before their tile is staged: pg[slot] holds the
  // page of the next tile staged into `slot`.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  Cursor lc = cur;
  stage(lc, page_of(lc), I0{});
  if (u0 + 1 < u1) advance(lc);
  stage(lc, page_of(lc), I1{});
  Cursor fc = lc;
  int pg[3];
  if (u0 + 2 < u1) advance(fc);
  pg[2] = page_of(fc);
  if (u0 + 3 < u1) advance(fc);
  pg[0] = page_of(fc);
  if (u0 + 4 < u1) advance(fc);
  pg[1] = page_of(fc);

  int vbuf = 0;  // V^T buffer of the current tile: alternates
  auto step_body = [&](int step, auto slot) __attribute__((always_inline)) {
    constexpr int X = decltype(slot)::value;
    constexpr int Y = (X + 2) % 3;  // slot of tile step + 2
    using IY = std::integral_constant<int, Y>;
    // This wave's copies of the tile have landed (only the next tile's stage may still
    // be in flight): transpose its V rows, then all waves meet.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStageOps) : "memory");
    store_v(slot, vbuf);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Query loads of a new item. They are younger than the next tile's stage, so
    // waiting for them (before the first MFMA) completes that stage too.
    const bool fresh = step == u0 || cur.t == 0;
    if (fresh) begin_piece();
    if (step + 2 < u1) advance(lc);
    stage(lc, pg[Y], IY{});
    if (step + 5 < u1) advance(fc);
    pg[Y] = page_of(fc);
    if (fresh) {
      asm volatile("s_waitcnt vmcnt(%8)"
                   : "+v"(qop[0]), "+v"(qop[1]), "+v"(qop[2]), "+v"(qop[3]), "+v"(qop[4]),
                     "+v"(qop[5]), "+v"(qop[6]), "+v"(qop[7])
                   : "n"(kStageOps)
                   : "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(slot, vbuf);
    if (step + 1 == u1 || cur.t + 1 == cur.nt) end_piece();
    if (step + 1 < u1) advance(cur);
    vbuf ^= 1;
  };
  for (int step = u0; step < u1; step += 3) {
    step_body(step, I0{});
    if (step + 1 < u1) step_body(step + 1, I1{});
    if (step + 2 < u1) step_body(step + 2, I2{});
  }
  // No copy may still be writing LDS when the workgroup ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The grid schedule's kernel for 16-bit pools at D = 128, a GQA pair per work item and
// pages of >= 16 keys, software pipelined: the scores of tile t + 1 are computed
// (S^T = K Q^T) while the softmax of tile t runs, so one wave keeps its MFMAs and its
// vector work in flight together instead of alternating between them (with the two
// waves of a SIMD meeting at every tile's barrier, both used to reach their softmax at
// the same time and leave the matrix core idle). Per tile t, in order:
//   wait for this wave's copies of tile t + 1; barrier (tile t + 1's K and raw V rows,
//   and every wave's V^T rows of tile t, are then visible, and every wave is done with
//   tile t - 1); transpose this wave's V rows of tile t + 1 into V^T buffer (t + 1) & 1;
//   stage tile t + 3 into the slots tile t used (K read by S(t) one step earlier);
//   S(t + 1) = K(t + 1) Q^T  ||  softmax of S(t) -> P(t); O^T += V^T(t) P^T(t).
// Staging maps and the softmax are those of paged_prefill_lds_kernel, except that K
// rows are swizzled over 16 chunks (key & 15) instead of 8; K/V slots rotate by three and the score accumulators by two, so the loop is unrolled by
// six with every buffer named at compile time.
template <typename TQ, typename TKV, bool kSplit>
__global__ __launch_bounds__(512) void paged_prefill_pipe_kernel(const PagedParams p) {
  constexpr bool kFp8 = std::is_same_v<TKV, fp8_t>;
  constexpr int D = 128;
  constexpr int kWaves = 8;
  constexpr int HW = 2;                   // query heads per work item, one per wave set
  constexpr int KW = kTileKeys / kWaves;  // keys of a tile staged by one wave
  constexpr int kRawRow = kFp8 ? D : D * 2;  // bytes of one staged pool row
  constexpr int kRowLanes = kRawRow / 16;    // lanes per staged row (16 bytes each)
  constexpr int kCopies = KW * kRowLanes / kWave;  // direct loads per wave per tile (K and V each)
  constexpr int KV = 2;                   // V keys per lane in the transpose
  constexpr int kKSteps = D / 16;
  constexpr int kDBlocks = D / 32;
  constexpr int kRow = D * 2;
  constexpr int kTileBytes = kTileKeys * kRow;
  constexpr int kRawTileBytes = kTileKeys * kRawRow;
  constexpr int kVRow = kTileKeys * 2;
  constexpr int kStageOps = 2 * kCopies;  // vector-memory ops of one tile's stage per lane
  static_assert(KW == 8 && kTileKeys == 64 && 32 * 4 == kPrefillQueryTile, "tile sizes");

  // Staging slots (raw pool rows: K and V of three tiles), the 16-bit K the MFMAs read
  // (for 16-bit pools the staged K itself; for fp8 pools a converted copy, two tiles)
  // and V^T (two tiles).
  __shared__ __align__(16) char k_lds0[kRawTileBytes];
  __shared__ __align__(16) char k_lds1[kRawTileBytes];
  __shared__ __align__(16) char k_lds2[kRawTileBytes];
  __shared__ __align__(16) char r_lds0[kRawTileBytes];
  __shared__ __align__(16) char r_lds1[kRawTileBytes];
  __shared__ __align__(16) char r_lds2[kRawTileBytes];
  __shared__ __align__(16) char kc_lds0[kFp8 ? kTileBytes : 16];  // converted K, even tiles
  __shared__ __align__(16) char kc_lds1[kFp8 ? kTileBytes : 16];  // converted K, odd tiles
  __shared__ __align__(1024) char v_lds0[kTileBytes];  // V^T of even tiles
  __shared__ __align__(1024) char v_lds1[kTileBytes];  // V^T of odd tiles
  auto k_arr = [&](auto slot) __attribute__((always_inline)) -> char* {
    constexpr int X = decltype(slot)::value;
    if constexpr (X == 0) return k_lds0; else if constexpr (X == 1) return k_lds1; else return k_lds2;
  };
  // The K the MFMAs of tile t read: staging slot t % 3, or converted buffer t & 1.
  auto kmma_arr = [&](auto slot, auto par) __attribute__((always_inline)) -> char* {
    if constexpr (kFp8) {
      if constexpr (decltype(par)::value == 0) return kc_lds0; else return kc_lds1;
    } else {
      return k_arr(slot);
    }
  };
  auto r_arr = [&](auto slot) __attribute__((always_inline)) -> char* {
    constexpr int X = decltype(slot)::value;
    if constexpr (X == 0) return r_lds0; else if constexpr (X == 1) return r_lds1; else return r_lds2;
  };
  auto v_arr = [&](auto par) __attribute__((always_inline)) -> char* {
    if constexpr (decltype(par)::value == 0) return v_lds0; else return v_lds1;
  };

  const int tid = threadIdx.x;
  const int wave = uniform(tid / kWave);
  const int lane = tid % kWave;
  const int l32 = lane & 31;
  const int hsel = lane >> 5;
  const int hs = wave / 4;  // head of the pair
  const int wq = wave % 4;  // 32-position query block

  // ---- the work item: (sequence, column, query tile) and the key tiles [tb, te) of
  // it this workgroup walks. Item grid: sequence blockIdx.y, column blockIdx.x, query
  // tiles dispatched longest first, every item whole. Split grid: the piece of rank
  // blockIdx.x / columns (split_piece), column blockIdx.x % columns, so one XCD keeps
  // the same columns (and their K/V) as in the item grid.
  const int group = p.hq / p.hk;
  const int chunks = group / HW;
  int s, qt, c, tb, te;
  SplitPiece piece{};
  if constexpr (kSplit) {
    const int cols = p.hk * chunks;
    c = static_cast<int>(blockIdx.x) % cols;
    __shared__ SplitLds split_lds;
    if (!split_piece(p, cols, static_cast<int>(blockIdx.x) / cols, split_lds, piece)) return;
    s = uniform(piece.s);
    qt = uniform(piece.q);
    tb = uniform(piece.tb);
    te = uniform(piece.te);
  } else {
    s = blockIdx.y;
    qt = static_cast<int>(gridDim.z) - 1 - static_cast<int>(blockIdx.z);
    c = blockIdx.x;
  }
  const int len = sload(p.seq_lens + s);
  const int context = sload(p.context_lens + s);
  if constexpr (!kSplit) {
    if (len <= 1) return;  // a decode row: the decode kernel has it
    const int qtiles = (len + kPrefillQueryTile - 1) / kPrefillQueryTile;
    if (qt >= qtiles) return;
    tb = 0;
    te = prefill_item_tiles(context, len, qt);
  }
  const int kvh = c / chunks;

  const float score_c = p.scale * kLog2e;  // > 0 (the dispatcher's condition)
  const char* kpool = static_cast<const char*>(p.k_pool);
  const char* vpool = static_cast<const char*>(p.v_pool);
  const uint32_t row_bytes = static_cast<uint32_t>(p.kv_row_bytes);
  const uint64_t page_bytes = static_cast<uint64_t>(row_bytes) << p.table_shift;
  const int32_t* table = p.block_tables + static_cast<int64_t>(s) * p.max_blocks;
  const uint32_t head_off = static_cast<uint32_t>(kvh * static_cast<uint32_t>(p.kv_head_bytes));

  // ---- this wave's rows: one head, 32 query positions.
  const int offset = context - len;
  const int w_first = qt * kPrefillQueryTile + 32 * wq;
  const bool w_active = w_first < len;
  const int w_kv_end = offset + min(w_first + 32, len);  // keys its last query sees
  const int w_kv_full = offset + w_first + 1;            // keys all its queries see
  const int w_nt = w_active ? (w_kv_end + kTileKeys - 1) / kTileKeys : 0;  // its tiles
  const int my_local = w_first + l32;
  const bool my_valid = my_local < len;
  const int my_visible = offset + my_local + 1;
  const int row_base = sload(p.cu_seqlens_q + s);
  const int head0 = (c / chunks) * group + (c % chunks) * HW + hs;

  // ---- per-lane constants of the staging and fragment maps (as paged_prefill_lds_kernel).
  // Copy j of a wave's keys: lane -> key kRowLanes-lane row (64 / kRowLanes) j + lane /
  // kRowLanes, 16-byte chunk lane % kRowLanes.
  constexpr int kKeysPerCopy = kWave / kRowLanes;
  uint32_t k_src_off[kCopies], v_src_off[kCopies], k_src_chunk[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; ++j) {
    const int key = kKeysPerCopy * j + lane / kRowLanes;  // wave-local
    if constexpr (kFp8) {
      // raw rows as they are; the conversion places the chunks
      k_src_chunk[j] = (lane % kRowLanes) * 16;
    } else {
      // K rows: chunk c of key r at chunk c ^ (r & 15), so the 16 lanes of a fragment
      // read that one LDS cycle serves (16 keys, one chunk) fall in distinct banks.
      k_src_chunk[j] = (((lane & 15) ^ ((KW * wave + key) & 15)) * 16);
    }
    k_src_off[j] = static_cast<uint32_t>(key) * row_bytes + k_src_chunk[j];
    v_src_off[j] = static_cast<uint32_t>(key) * row_bytes + (lane % kRowLanes) * 16;
  }
  const int v_chunk = lane & 15;
  const int v_key = KW * wave + KV * (lane >> 4);
  const int vt_chunk = (2 * (v_key >> 4) + ((v_key >> 2) & 1)) ^ (v_chunk & 7);
  const uint32_t vt_dst = static_cast<uint32_t>(8 * v_chunk * kVRow + (4 * ((v_key >> 3) & 1) + (v_key & 3)) * 2);
  uint32_t k_rd[kKSteps];
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) k_rd[ks] = l32 * kRow + (((2 * ks + hsel) ^ (l32 & 15)) * 16);
  uint32_t v_rd[2][4];
  {
    const int f0 = (l32 ^ (l32 >> 3)) & 7;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) v_rd[par][ks] = l32 * kVRow + ((((2 * ks + hsel) ^ f0 ^ (4 * par)) & 7) * 16);
    }
  }

  // Page id of this wave's keys of tile t (past the last tile: the last tile again).
  auto page_of = [&](int t) __attribute__((always_inline)) -> int {
    const int key0 = min(min(t, te - 1) * kTileKeys + KW * wave, context - 1);
    return sload(table + (key0 >> p.block_shift));
  };
  // fp8 pools: the page's K and V scales of each staged slot (the wave's keys share a
  // page), loaded with the page id.
  float ks[3] = {0.0f, 0.0f, 0.0f}, vs[3] = {0.0f, 0.0f, 0.0f};
  auto stage = [&](int t, int page, auto slot) __attribute__((always_inline)) {
    constexpr int X = decltype(slot)::value;
    t = min(t, te - 1);
    const uint32_t kdst = lds_address(k_arr(slot) + KW * wave * kRawRow);
    const uint32_t rdst = lds_address(r_arr(slot) + KW * wave * kRawRow);
    const int key0 = t * kTileKeys + KW * wave;
    const int last = context - 1;
    const uint64_t head = static_cast<uint64_t>(static_cast<uint32_t>(page)) * page_bytes + head_off;
    if constexpr (kFp8) {
      const int64_t si = static_cast<int64_t>(page) * p.hk + kvh;
      ks[X] = __int_as_float(sload(reinterpret_cast<const int32_t*>(p.k_scales + si)));
      vs[X] = __int_as_float(sload(reinterpret_cast<const int32_t*>(p.v_scales + si)));
    }
    if (key0 + KW - 1 <= last) {
      const uint64_t base = head + static_cast<uint32_t>(key0 & p.block_mask) * row_bytes;
#pragma unroll
      for (int j = 0; j < kCopies; ++j) {
        copy_to_lds(kpool + base, k_src_off[j], kdst + kKeysPerCopy * j * kRawRow);
        copy_to_lds(vpool + base, v_src_off[j], rdst + kKeysPerCopy * j * kRawRow);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kCopies; ++j) {
        const uint32_t row = static_cast<uint32_t>(min(key0 + kKeysPerCopy * j + lane / kRowLanes, last) &
                                                   p.block_mask) * row_bytes;
        copy_to_lds(kpool + head, row + k_src_chunk[j], kdst + kKeysPerCopy * j * kRawRow);
        copy_to_lds(vpool + head, row + (lane % kRowLanes) * 16, rdst + kKeysPerCopy * j * kRawRow);
      }
    }
  };
  // fp8 pools: eight codes of a raw row -> eight 16-bit elements times the page scale.
  auto dequant8 = [&](const u32x2& w, float scale) __attribute__((always_inline)) -> u32x4 {
    u32x4 out;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
      out[2 * i] = Mma<TQ>::pack2(lo[0] * scale, lo[1] * scale);
      out[2 * i + 1] = Mma<TQ>::pack2(hi[0] * scale, hi[1] * scale);
    }
    return out;
  };
  // fp8 pools: this wave's staged K rows of slot `slot` (tile-local keys KW * wave ..
  // +7, each lane 16 codes of one row) -> converted K buffer `par`, in the swizzled
  // layout the fragment reads use (logical chunk c of key r at chunk c ^ (r & 15)).
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  auto convert_k = [&](auto slot, auto par) __attribute__((always_inline)) {
    constexpr int X = decltype(slot)::value;
    const int key = KW * wave + lane / kRowLanes;
    const int c = 2 * (lane % kRowLanes);
    const u32x4 w = *reinterpret_cast<const u32x4*>(k_arr(slot) + key * kRawRow + (lane % kRowLanes) * 16);
    const uint32_t dst = lds_address(kmma_arr(slot, par) + key * kRow);
    *reinterpret_cast<lds_u32x4*>(dst + ((c ^ (key & 15)) * 16)) = dequant8(u32x2{w[0], w[1]}, ks[X]);
    *reinterpret_cast<lds_u32x4*>(dst + (((c + 1) ^ (key & 15)) * 16)) = dequant8(u32x2{w[2], w[3]}, ks[X]);
  };
  typedef __attribute__((address_space(3))) uint32_t lds_u32;
  auto store_v = [&](auto slot, auto par) __attribute__((always_inline)) {
    constexpr int X = decltype(slot)::value;
    u32x4 vr[KV];
    if constexpr (kFp8) {
      const char* raw = r_arr(slot) + v_key * kRawRow + v_chunk * 8;
#pragma unroll
      for (int j = 0; j < KV; ++j) vr[j] = dequant8(*reinterpret_cast<const u32x2*>(raw + j * kRawRow), vs[X]);
    } else {
      const char* raw = r_arr(slot) + v_key * kRow + v_chunk * 16;
#pragma unroll
      for (int j = 0; j < KV; ++j) vr[j] = *reinterpret_cast<const u32x4*>(raw + j * kRow);
    }
    const uint32_t row0 = lds_address(v_arr(par)) + vt_dst + (vt_chunk & 7) * 16;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) == 0 ? 0x05040100u : 0x07060302u;
      const uint32_t addr = (row0 ^ (e * 16)) + e * kVRow;
      *reinterpret_cast<lds_u32*>(addr) = __builtin_amdgcn_perm(vr[1][e >> 1], vr[0][e >> 1], sel);
    }
  };

  // ---- per-wave state.
  u32x4 qop[kKSteps];
  {
    const int local = min(my_local, len - 1);
    const int64_t qrow = static_cast<int64_t>(row_base + local) * p.hq + head0;
    const char* qp = static_cast<const char*>(p.q) + (qrow * D + 8 * hsel) * 2;
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) qop[ks] = load16_untracked(qp + ks * 32);
  }
  f32x16 o[kDBlocks];
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db) o[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.0f;
  f32x16 sc0[2], sc1[2];  // scores of even / odd tiles

  // S(t) = K(t) Q^T from K slot `slot`, fragments read four MFMAs ahead.
  auto qk = [&](auto slot, auto kpar, f32x16 (&sc)[2]) __attribute__((always_inline)) {
    constexpr int kLook = 4;
    const char* kt = kmma_arr(slot, kpar);
    auto k_frag = [&](int i) __attribute__((always_inline)) {
      return *reinterpret_cast<const u32x4*>(kt + (i & 1) * 32 * kRow + k_rd[i >> 1]);
    };
    sc[0] = f32x16{};
    sc[1] = f32x16{};
    u32x4 fa[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) fa[i] = k_frag(i);
#pragma unroll
    for (int i = 0; i < 2 * kKSteps; ++i) {
      const u32x4 a = fa[i % kLook];
      if (i + kLook < 2 * kKSteps) fa[i % kLook] = k_frag(i + kLook);
      sc[i & 1] = Mma<TQ>::run(a, qop[i >> 1], sc[i & 1]);
    }
  };
  // Causal mask of tile t's scores (tiles crossing this wave's diagonal only).
  auto mask = [&](int t, f32x16 (&sc)[2]) __attribute__((always_inline)) {
    const int key0 = t * kTileKeys;
    if (key0 + kTileKeys > w_kv_full) {
      const int lim = my_valid ? my_visible - key0 - 4 * hsel : INT_MIN;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (kb * 32 + 8 * (r >> 2) + (r & 3) >= lim) sc[kb][r] = -INFINITY;
        }
      }
    }
  };
  // Running max of a tile's scores (raised only past the slack, O and l rescaled with
  // it); returns -max in log2 units, the exponent's offset.
  auto tile_max = [&](const f32x16 (&sc)[2]) __attribute__((always_inline)) -> float {
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sc[kb][r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave)) * score_c;
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kRescaleSlack) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_new == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o[db] *= alpha;
    }
    return m_run == -INFINITY ? 0.0f : -m_run;
  };
  // Score element r of key block kb -> probability: exp2(s * c - max), summed into
  // ps[r % 4] and packed in pairs into the P^T operand pop[2 kb + r / 8].
  auto prob = [&](const f32x16 (&sc)[2], int kb, int r, float neg_mu, float (&pf)[2][16],
                  float (&ps)[4]) __attribute__((always_inline)) {
    pf[kb][r] = __builtin_amdgcn_exp2f(fmaf(sc[kb][r], score_c, neg_mu));
    ps[r & 3] += pf[kb][r];
  };
  auto pack = [&](const float (&pf)[2][16], int kb, int half, u32x4 (&pop)[4]) __attribute__((always_inline)) {
    const float* v = &pf[kb][8 * half];
    pop[2 * kb + half] = u32x4{Mma<TQ>::pack2(v[0], v[1]), Mma<TQ>::pack2(v[2], v[3]),
                               Mma<TQ>::pack2(v[4], v[5]), Mma<TQ>::pack2(v[6], v[7])};
  };
  constexpr int kMfma = 0x008, kDsRead = 0x100, kVec = 0x002 | 0x400;  // VALU and TRANS
  // Phase A of tile t: S(t + 1) = K(t + 1) Q^T from K slot `slot`, each MFMA paired with
  // one K fragment read (four ahead) and one probability of key block 0 of tile t.
  auto phase_a = [&](auto slot, auto kpar, f32x16 (&nxt)[2], const f32x16 (&cur)[2], float neg_mu,
                     float (&pf)[2][16], float (&ps)[4], u32x4 (&pop)[4]) __attribute__((always_inline)) {
    constexpr int kLook = 4;
    const char* kt = kmma_arr(slot, kpar);
    auto k_frag = [&](int i) __attribute__((always_inline)) {
      return *reinterpret_cast<const u32x4*>(kt + (i & 1) * 32 * kRow + k_rd[i >> 1]);
    };
    nxt[0] = f32x16{};
    nxt[1] = f32x16{};
    u32x4 fa[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) fa[i] = k_frag(i);
#pragma unroll
    for (int i = 0; i < 2 * kKSteps; ++i) {
      const u32x4 a = fa[i % kLook];
      if (i + kLook < 2 * kKSteps) fa[i % kLook] = k_frag(i + kLook);
      nxt[i & 1] = Mma<TQ>::run(a, qop[i >> 1], nxt[i & 1]);
      prob(cur, 0, i, neg_mu, pf, ps);
      if (i == 7) pack(pf, 0, 0, pop);
      if (i == 15) pack(pf, 0, 1, pop);
    }
    __builtin_amdgcn_sched_group_barrier(kDsRead, kLook, 0);
#pragma unroll
    for (int i = 0; i < 2 * kKSteps; ++i) {
      __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
      if (i + kLook < 2 * kKSteps) __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
      if (i == 7 || i == 15) {
        __builtin_amdgcn_sched_group_barrier(kVec, 7, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(kVec, 3, 0);
      }
    }
  };
  // Phase B of tile t: O^T += V^T(t) P^T(t) from V^T buffer `par`; the first eight MFMAs
  // (keys 0-31) each paired with two probabilities of key block 1, which the last
  // eight consume.
  auto phase_b = [&](auto par, const f32x16 (&cur)[2], float neg_mu, float (&pf)[2][16],
                     float (&ps)[4], u32x4 (&pop)[4]) __attribute__((always_inline)) {
    constexpr int kLook = 4;
    const char* vt = v_arr(par);
    auto v_frag = [&](int i) __attribute__((always_inline)) {
      const int db = i & 3, ks = i >> 2;
      return *reinterpret_cast<const u32x4*>(vt + db * 32 * kVRow + v_rd[db & 1][ks]);
    };
    u32x4 fa[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) fa[i] = v_frag(i);
#pragma unroll
    for (int i = 0; i < kDBlocks * 4; ++i) {
      const u32x4 a = fa[i % kLook];
      if (i + kLook < kDBlocks * 4) fa[i % kLook] = v_frag(i + kLook);
      o[i & 3] = Mma<TQ>::run(a, pop[i >> 2], o[i & 3]);
      if (i < 8) {
        prob(cur, 1, 2 * i, neg_mu, pf, ps);
        prob(cur, 1, 2 * i + 1, neg_mu, pf, ps);
      }
      if (i == 3) pack(pf, 1, 0, pop);
      if (i == 7) pack(pf, 1, 1, pop);
    }
    __builtin_amdgcn_sched_group_barrier(kDsRead, kLook, 0);
#pragma unroll
    for (int i = 0; i < kDBlocks * 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
      if (i + kLook < kDBlocks * 4) __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
      if (i == 3 || i == 7) {
        __builtin_amdgcn_sched_group_barrier(kVec, 10, 0);
      } else if (i < 8) {
        __builtin_amdgcn_sched_group_barrier(kVec, 6, 0);
      }
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  // ---- prologue: tiles tb .. tb + 2 staged, page ids of the next three fetched; tile
  // tb's V^T built and its scores computed. Slots and buffers go by t - tb.
  stage(tb, page_of(tb), I0{});
  stage(tb + 1, page_of(tb + 1), I1{});
  stage(tb + 2, page_of(tb + 2), I2{});
  int pg[3] = {page_of(tb + 3), page_of(tb + 4), page_of(tb + 5)};  // pg[x]: next tile staged into slot x
  // The queries (the oldest loads) and tile tb have landed. The wait names the query
  // registers: their loads are untracked, and a wait the compiler placed itself would
  // sit in the tile loop (the first scores are conditional), draining every step's
  // fresh copies.
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(qop[0]), "+v"(qop[1]), "+v"(qop[2]), "+v"(qop[3]), "+v"(qop[4]),
                 "+v"(qop[5]), "+v"(qop[6]), "+v"(qop[7])
               : "n"(2 * kStageOps)
               : "memory");
  if constexpr (kFp8) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // tile 0's scales
    convert_k(I0{}, I0{});
  }
  store_v(I0{}, I0{});
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (tb < w_nt) qk(I0{}, I0{}, sc0);

  // Step for tile t: X = (t - tb) % 3 (the slots tile t used, restaged with tile t + 3),
  // Y = (t - tb + 1) % 3 (tile t + 1's slots), P = (t - tb) & 1 (tile t's score and V^T
  // buffers).
  auto step = [&](int t, auto xs, auto par) __attribute__((always_inline)) {
    constexpr int X = decltype(xs)::value;
    constexpr int Y = (X + 1) % 3;
    constexpr int P = decltype(par)::value;
    using IY = std::integral_constant<int, Y>;
    using IQ = std::integral_constant<int, 1 - P>;
    f32x16(&cur)[2] = P == 0 ? sc0 : sc1;
    f32x16(&nxt)[2] = P == 0 ? sc1 : sc0;
    // Tile t + 1 has landed for this wave (tiles t + 2 may still be in flight); the
    // barrier publishes it and tile t's V^T, and retires tile t - 1.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStageOps) : "memory");
    if constexpr (kFp8) {
      // This wave's K rows of tile t + 1, converted before the barrier publishes them
      // (the buffer's last readers, tile t - 1's scores, finished before the previous
      // barrier). Tile t + 1's scales were loaded three steps ago.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      convert_k(IY{}, IQ{});
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    store_v(IY{}, IQ{});
    stage(t + 3, pg[X], xs);
    pg[X] = page_of(t + 6);
    __builtin_amdgcn_sched_barrier(0);
    if (t < w_nt) {
      mask(t, cur);
      const float neg_mu = tile_max(cur);
      float pf[2][16];
      float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      u32x4 pop[4];
      // Scores of tile t + 1 even past this wave's last tile (the slot then holds a
      // staged copy of a valid tile; the result goes unused): no branch, so the
      // probabilities stay interleaved with these MFMAs.
      phase_a(IY{}, IQ{}, nxt, cur, neg_mu, pf, ps, pop);
      phase_b(par, cur, neg_mu, pf, ps, pop);
      l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
    }
  };
  for (int t = tb; t < te; t += 6) {
    step(t, I0{}, I0{});
    if (t + 1 < te) step(t + 1, I1{}, I1{});
    if (t + 2 < te) step(t + 2, I2{}, I0{});
    if (t + 3 < te) step(t + 3, I0{}, I1{});
    if (t + 4 < te) step(t + 4, I1{}, I0{});
    if (t + 5 < te) step(t + 5, I2{}, I1{});
  }
  // No copy may still be writing LDS when the workgroup ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (kSplit) {
    // A cut item: every piece stores its (m, l, O) partial (each lane its own, in the
    // lane order every piece shares), then counts itself in; the last to arrive
    // resets the counter for the next launch and merges the other pieces' partials
    // into its own accumulators before the usual normalise and store.
    //
    // The partials are written and read with relaxed atomic stores and loads at agent
    // (device) scope, which the hardware keeps coherent per location across the XCDs'
    // L2s (scope bits on each access) rather than with a fence: an agent-scope fence
    // writes back and invalidates the whole L2 of the XCD, dropping the K/V lines
    // every other workgroup there is reading (measured: cut pieces ran at 5.6 us per
    // tile against 3.5). Order: a piece's stores complete (vmcnt(0), every wave, then
    // the barrier) before its counter increment is issued; the last piece issues its
    // loads only after the increment has returned, through the barrier that
    // publishes the result.
    if (piece.pieces > 1) {
      __shared__ int split_last;
      const int cols = p.hk * chunks;
      auto slot_of = [&](int j) __attribute__((always_inline)) -> float* {
        return p.pf_part + (static_cast<int64_t>(piece.slot0 + j) * cols + c) * kSplitSlotFloats;
      };
      auto o_at = [&](float* slot, int k) __attribute__((always_inline)) -> float* {
        return slot + ((wave * 16 + k) * kWave + lane) * 4;
      };
      auto ml_at = [&](float* slot) __attribute__((always_inline)) -> float* {
        return slot + kWaves * kWave * 64 + (wave * kWave + lane) * 2;
      };
      auto put = [&](float* at, float v) __attribute__((always_inline)) {
        __hip_atomic_store(at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      };
      auto get = [&](float* at) __attribute__((always_inline)) -> float {
        return __hip_atomic_load(at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      };
      {
        float* mine = slot_of(piece.piece);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const f32x16& a = o[k >> 2];
          const int r = 4 * (k & 3);
          float* at = o_at(mine, k);
#pragma unroll
          for (int e = 0; e < 4; ++e) put(at + e, a[r + e]);
        }
        put(ml_at(mine), m_run);
        put(ml_at(mine) + 1, l_run);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) {
        int* count = p.pf_count + piece.item * cols + c;
        const int before = __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = before == piece.pieces - 1 ? 1 : 0;
        if (last) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        split_last = last;
      }
      __syncthreads();
      if (split_last == 0) return;
      // All pieces folded in piece order from an empty state (this piece's own from
      // registers), so the result is the same whichever piece finishes last.
      float m_acc = -INFINITY, l_acc = 0.0f;
      f32x16 o_acc[kDBlocks];
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o_acc[db] = f32x16{};
      for (int j = 0; j < piece.pieces; ++j) {
        float* other = slot_of(j);
        const bool own = j == piece.piece;
        const float m_o = own ? m_run : get(ml_at(other));
        const float l_o = own ? l_run : get(ml_at(other) + 1);
        const float m_new = fmaxf(m_acc, m_o);
        const float fa = m_acc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_acc - m_new);
        const float fb = m_o == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_o - m_new);
        l_acc = l_acc * fa + l_o * fb;
        m_acc = m_new;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          f32x16& a = o_acc[k >> 2];
          const f32x16& mine = o[k >> 2];
          const int r = 4 * (k & 3);
          float* at = o_at(other, k);
#pragma unroll
          for (int e = 0; e < 4; ++e) a[r + e] = a[r + e] * fa + (own ? mine[r + e] : get(at + e)) * fb;
        }
      }
      m_run = m_acc;
      l_run = l_acc;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o[db] = o_acc[db];
    }
  }
  if (!w_active || !my_valid) return;
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  const int64_t orow = (static_cast<int64_t>(row_base + my_local) * p.hq + head0) * D;
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = db * 32 + 8 * j + 4 * hsel;
      float r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = o[db][4 * j + i] * inv;
      *reinterpret_cast<u32x2*>(static_cast<char*>(p.out) + (orow + d) * 2) =
          u32x2{Mma<TQ>::pack2(r[0], r[1]), Mma<TQ>::pack2(r[2], r[3])};
    }
  }
}

// Combine the pieces of every prefill item cut between stream workgroups. An item
// spread over shares first .. last (the shares holding its first and last key) has
// last - first boundaries inside it (the starts of shares first + 1 .. last); the
// kMergeSub workgroups of each boundary merge their own slice of the item's
// HW x rows x D outputs, so an item's merge is spread over as many CUs as it has
// pieces (the partials come from L2 / MALL: one CU per item left the merge bound by
// that CU's load bandwidth). The item's piece slots are listed in LDS (an empty share
// holds none: slot -1); each thread owns kElems float4 columns of its slice and
// combines the pieces kPieces at a time, with every load of a batch issued together.
constexpr int kMergeSub = 4;
constexpr int kMergeThreads = 256;

template <typename TQ, int D, int HW>
__global__ __launch_bounds__(kMergeThreads) void paged_prefill_merge_kernel(const PagedParams p) {
  constexpr int kElems = 2;
  constexpr int kPieces = 8;
  __shared__ int s_slots[kMaxPrefillWgs];
  const int64_t grid = p.pf_wgs;
  const int bid = static_cast<int>(blockIdx.x % grid);
  const int sub = static_cast<int>(blockIdx.x / grid);
  const int n = p.num_seqs;
  const int group = p.hq / p.hk;
  const int chunks = group / HW;
  const int cols = p.hk * chunks;
  // Find the item at the share's start. With fewer than 64 sequences every lane loads
  // one prefix entry at once and a ballot finds the sequence: one memory round trip
  // where a binary search makes one per step (the merge is short, so this chain is a
  // large part of it).
  const int lane = threadIdx.x % kWave;
  int v = 0;
  int total;
  if (n < kWave) {
    v = p.pf_prefix[min(lane, n)];
    total = __shfl(v, n, kWave);
  } else {
    total = sload(p.pf_prefix + n);
  }
  // The shares the prefill kernel used; boundary b is the start of share b, merged on
  // the XCD that computed share b (workgroups bid and bid + grid share an XCD when the
  // grid is a multiple of 8).
  const int64_t wgs = prefill_stream_shares(total, grid, p.pf_share_tiles);
  const int b = xcd_share_of(bid, static_cast<int>(grid), static_cast<int>(wgs));
  if (b <= 0) return;
  const int64_t x = share_begin(b, total, wgs);
  if (x >= total) return;
  Cursor k;
  if (n < kWave) {
    const uint64_t le = __ballot(lane <= n && v <= x);
    const int a = __popcll(le) - 1;  // pre[a] <= x < pre[a + 1]
    seek_in(k, p, a, uniform(__shfl(v, a, kWave)), uniform(__shfl(v, a + 1, kWave)), cols,
            static_cast<int>(x));
  } else {
    seek(k, p, p.pf_prefix, n, cols, static_cast<int>(x));
  }
  if (k.t == 0) return;  // the share starts an item: nothing is cut here
  const int64_t start = x - k.t;
  const int64_t end = start + k.nt;
  // start < x <= end - 1, so first < b <= last.
  const int64_t first = share_owner(start, total, wgs);
  const int64_t last = share_owner(end - 1, total, wgs);
  const int pieces = static_cast<int>(last - first + 1);
  const int slices = static_cast<int>(last - first) * kMergeSub;
  const int slice = static_cast<int>(b - first - 1) * kMergeSub + sub;
  // Piece i is share first + i: the item's last piece in that share (slot 2w + 1) for
  // the first share unless it starts exactly at the item, its first piece (slot 2w)
  // for the others.
  for (int i = threadIdx.x; i < pieces; i += blockDim.x) {
    const int64_t g = first + i;
    const int64_t gs = share_begin(g, total, wgs);
    const bool empty = gs == share_begin(g + 1, total, wgs);
    s_slots[i] = empty ? -1 : static_cast<int>(2 * g + (i == 0 && gs < start ? 1 : 0));
  }
  __syncthreads();
  const int qb = k.q * kPrefillQueryTile;
  const int rows = min(kPrefillQueryTile, k.len - qb);
  const int head0 = (k.c / chunks) * group + (k.c % chunks) * HW;
  const int row0 = sload(p.cu_seqlens_q + k.s) + qb;
  constexpr int kD4 = D / 4;
  const int n4 = HW * rows * kD4;
  const int lo = static_cast<int>(static_cast<int64_t>(slice) * n4 / slices);
  const int hi = static_cast<int>(static_cast<int64_t>(slice + 1) * n4 / slices);
  const int slot0 = s_slots[0];  // piece 0 holds the item's first key: never empty
  const int nthreads = static_cast<int>(blockDim.x);
  for (int j0 = lo + threadIdx.x; j0 < hi; j0 += kElems * nthreads) {
    int64_t prow[kElems];
    int dcol[kElems];
    float m[kElems], l[kElems];
    f32x4 acc[kElems];
#pragma unroll
    for (int e = 0; e < kElems; ++e) {
      const int j = min(j0 + e * nthreads, hi - 1);
      const int hw = j / (rows * kD4);
      const int rem = j - hw * rows * kD4;
      const int row = rem / kD4;
      dcol[e] = (rem - row * kD4) * 4;
      prow[e] = static_cast<int64_t>(hw) * kPrefillQueryTile + row;
      m[e] = -INFINITY;
      l[e] = 0.0f;
      acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int i0 = 0; i0 < pieces; i0 += kPieces) {
      float2 ml[kPieces][kElems];
      f32x4 oi[kPieces][kElems];
      int slot[kPieces];
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        slot[i] = i0 + i < pieces ? s_slots[i0 + i] : -1;
        const int64_t base = static_cast<int64_t>(slot[i] >= 0 ? slot[i] : slot0) * HW *
                             kPrefillQueryTile;
#pragma unroll
        for (int e = 0; e < kElems; ++e) {
          ml[i][e] = *reinterpret_cast<const float2*>(p.pf_ml + (base + prow[e]) * 2);
          oi[i][e] = *reinterpret_cast<const f32x4*>(p.pf_o + (base + prow[e]) * D + dcol[e]);
        }
      }
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        if (slot[i] < 0) continue;  // past the last piece, or an empty share
#pragma unroll
        for (int e = 0; e < kElems; ++e) {
          // Piece rows are normalised: weight them by l_i * 2^(m_i - max).
          const float mn = fmaxf(m[e], ml[i][e].x);
          const float mu = mn == -INFINITY ? 0.0f : mn;
          const float a = __builtin_amdgcn_exp2f(m[e] - mu);
          const float c = ml[i][e].y * __builtin_amdgcn_exp2f(ml[i][e].x - mu);
          l[e] = l[e] * a + c;
          acc[e] = acc[e] * a + oi[i][e] * c;
          m[e] = mn;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < kElems; ++e) {
      if (j0 + e * nthreads >= hi) continue;
      const int hw = static_cast<int>(prow[e] / kPrefillQueryTile);
      const int row = static_cast<int>(prow[e] - static_cast<int64_t>(hw) * kPrefillQueryTile);
      const float inv = l[e] > 0.0f ? 1.0f / l[e] : 0.0f;
      const int64_t obase = (static_cast<int64_t>(row0 + row) * p.hq + head0 + hw) * D + dcol[e];
      *reinterpret_cast<u32x2*>(static_cast<char*>(p.out) + obase * 2) =
          u32x2{Mma<TQ>::pack2(acc[e][0] * inv, acc[e][1] * inv),
                Mma<TQ>::pack2(acc[e][2] * inv, acc[e][3] * inv)};
    }
  }
}

// ------------------------------------------------------------------ dispatch

namespace {

template <typename TQ, typename TKV, int D, int HCW, int HS>
void launch_prefill_cfg(const PagedParams& p, int max_query_len, hipStream_t stream) {
  constexpr int HW = HCW * HS;
  if (p.pf_wgs > 0) {
    paged_prefill_kernel<TQ, TKV, D, HCW, HS><<<p.pf_wgs, 256 * HS, 0, stream>>>(p);
    paged_prefill_merge_kernel<TQ, D, HW><<<kMergeSub * p.pf_wgs, kMergeThreads, 0, stream>>>(p);
  } else {
    const int cols = p.hk * (p.hq / p.hk / HW);
    const int qtiles = (max_query_len + kPrefillQueryTile - 1) / kPrefillQueryTile;
    const dim3 grid(cols, p.num_seqs, qtiles);
    paged_prefill_kernel<TQ, TKV, D, HCW, HS><<<grid, 256 * HS, 0, stream>>>(p);
  }
}

// The pipelined kernel on the item grid, or on the split grid when the plan cuts items
// (pf_pieces > 1, with the counters and partial slots it names).
template <typename TQ, typename TKV>
void launch_prefill_pipe(const PagedParams& p, int max_query_len, hipStream_t stream) {
  const int cols = p.hk * (p.hq / p.hk / 2);
  if (p.pf_pieces > 1 && p.pf_count != nullptr && p.pf_part != nullptr) {
    paged_prefill_pipe_kernel<TQ, TKV, true><<<cols * p.pf_ranks, 512, 0, stream>>>(p);
    return;
  }
  const int qtiles = (max_query_len + kPrefillQueryTile - 1) / kPrefillQueryTile;
  paged_prefill_pipe_kernel<TQ, TKV, false><<<dim3(cols, p.num_seqs, qtiles), 512, 0, stream>>>(p);
}

template <typename TQ, int HS>
void launch_prefill_lds(const PagedParams& p, int max_query_len, hipStream_t stream) {
  if (p.pf_wgs > 0) {
    paged_prefill_lds_kernel<TQ, HS, true><<<p.pf_wgs, 256 * HS, 0, stream>>>(p);
    paged_prefill_merge_kernel<TQ, 128, HS><<<kMergeSub * p.pf_wgs, kMergeThreads, 0, stream>>>(p);
  } else {
    const int cols = p.hk * (p.hq / p.hk / HS);
    const int qtiles = (max_query_len + kPrefillQueryTile - 1) / kPrefillQueryTile;
    const dim3 grid(cols, p.num_seqs, qtiles);
    if constexpr (HS == 2) {
      if (!p.pf_register_staging) {
        launch_prefill_pipe<TQ, TQ>(p, max_query_len, stream);
        return;
      }
    }
    paged_prefill_lds_kernel<TQ, HS, false><<<grid, 256 * HS, 0, stream>>>(p);
  }
}

template <typename TQ, typename TKV, int D>
hipError_t launch_prefill_d(const PagedParams& p, int max_query_len, hipStream_t stream) {
  // 16-bit pools at D = 128 with pages of >= 16 keys and a positive scale: K copied
  // straight into LDS.
  if constexpr (std::is_same_v<TQ, TKV> && D == 128) {
    if (p.block_shift >= 4 && p.scale > 0.0f && !p.pf_register_staging) {
      if (prefill_item_heads(p.hq / p.hk) == 1) {
        launch_prefill_lds<TQ, 1>(p, max_query_len, stream);
      } else {
        launch_prefill_lds<TQ, 2>(p, max_query_len, stream);
      }
      return hipGetLastError();
    }
  }
  // fp8 pools at D = 128, GQA pairs, pages of >= 16 keys, the grid schedule: the
  // pipelined kernel, codes copied straight into LDS and dequantised there.
  if constexpr (std::is_same_v<TKV, fp8_t> && D == 128) {
    if (p.block_shift >= 4 && p.scale > 0.0f && !p.pf_register_staging && p.pf_wgs == 0 &&
        prefill_item_heads(p.hq / p.hk) == 2) {
      launch_prefill_pipe<TQ, fp8_t>(p, max_query_len, stream);
      return hipGetLastError();
    }
  }
  // Both heads of an even GQA group in one wave (HCW = 2) would share K/V fragments,
  // but needs ~450 registers: one wave per SIMD and no softmax/MFMA overlap. Measured
  // at config 3 it ran 25-40% slower than a wave per head, two waves per SIMD.
  if (prefill_item_heads(p.hq / p.hk) == 1) {
    launch_prefill_cfg<TQ, TKV, D, 1, 1>(p, max_query_len, stream);
  } else {
    launch_prefill_cfg<TQ, TKV, D, 1, 2>(p, max_query_len, stream);
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
