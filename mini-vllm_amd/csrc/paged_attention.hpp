// Internal launch interface of the paged-attention kernels (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Largest number of physical pages one decode split may span and still have its page
// ids staged in LDS (4 KiB). The planner keeps splits at or below 1024 tokens, which is
// at most 1025 pages even at a page size of 1; a caller that understates
// max_context_len gets longer splits, which then read the table from global memory.
constexpr int kMaxSplitPages = 1040;
constexpr int kMaxSplitTokens = 1024;

// The stream schedule scans the context lengths of up to this many sequences in LDS.
constexpr int kMaxStreamSeqs = 4096;

// Query positions per prefill work item (4 waves x 32 MFMA columns) and keys per tile.
constexpr int kPrefillQueryTile = 128;
// Most stream-prefill workgroups (the merge lists an item's pieces in LDS).
constexpr int kMaxPrefillWgs = 2048;
// Stream prefill: the shares used of `wgs` workgroups, each of at least `min_tiles`
// 64-key tiles while that leaves a quarter of the workgroups busy. A share also pays
// for loading its items' queries and for writing and merging (m, l, O) pieces of 128
// query rows: a 512-token chunk behind a 1-2K prefix spread over every CU is cut into
// shares of two or three tiles, most of their time then going to that overhead
// (measured, 31 decode rows + one chunk, whole call: shares of >= 4 tiles 70-80 us
// against 76-81 us with one tile; 4K-16K prefixes 2-7% faster).
constexpr int kPrefillShareTiles = 4;
__host__ __device__ inline int64_t prefill_stream_shares(int64_t total_units, int64_t wgs,
                                                         int min_tiles) {
  const int64_t per = min_tiles > 1 ? min_tiles : 1;
  int64_t shares = (total_units + per - 1) / per;
  const int64_t floor = total_units < wgs / 4 ? total_units : wgs / 4;
  if (shares < floor) shares = floor;
  return shares < 1 ? 1 : (shares < wgs ? shares : wgs);
}
// XCDs (each with its own L2) that workgroups are dispatched to round robin on MI355X.
constexpr int kXcds = 8;
constexpr int kPrefillKeyTile = 64;

// Split grid (prefill): items longer than a piece length (a percentage of the mean work
// per CU, kSplitDefaultPct by default) are cut into key
// ranges ("pieces") run by workgroups of their own in one launch, longest piece first;
// the last piece of an item to finish merges the others' (m, l, O) partials. Every
// workgroup derives the same schedule from the sequences' sizes, one wave lane per
// item, so the items of one call are at most kSplitMaxItems and the columns at most
// kSplitMaxCols (the counters' extent).
constexpr int kSplitMaxItems = 64;
constexpr int kSplitMaxCols = 64;
constexpr int kSplitDefaultPieces = 8;
// Floats of one piece's partial: 8 waves x 64 lanes x (64 of O + (m, l)).
constexpr int kSplitSlotFloats = 8 * 64 * 66;
constexpr int kSplitDefaultPct = 150;
// Host bounds of the split grid over `cols` columns on `cus` CUs with pieces of at least
// pct% of the mean work per CU: the extra pieces of one column number fewer than
// 100 cus / (pct cols); the partial slots of one column (every piece of a cut item
// holds one) at most twice that.
__host__ __device__ inline int split_extra_ranks(int cus, int cols, int pct) {
  return (100 * cus + pct * cols - 1) / (pct * cols);
}
__host__ __device__ inline int split_slots(int cus, int cols, int pct) {
  return 2 * split_extra_ranks(cus, cols, pct);
}

// Query heads per prefill work item: two heads of a GQA group share every K/V tile
// staged in LDS when the group size is even.
__host__ __device__ inline int prefill_item_heads(int group) { return group % 2 == 0 ? 2 : 1; }

// Key tiles the prefill workgroup of query tile q walks for a sequence of `context`
// keys and `len` query tokens: keys [0, context - len + min((q + 1) * 128, len)).
__host__ __device__ inline int prefill_item_tiles(int context, int len, int q) {
  const int last = (q + 1) * kPrefillQueryTile < len ? (q + 1) * kPrefillQueryTile : len;
  return (context - len + last + kPrefillKeyTile - 1) / kPrefillKeyTile;
}

// Stream decode: the workgroups that take a share. Shares of at least
// kMinDecodeShareKeys keys: with few decode keys (a prefill step carrying a handful of
// decode rows) equal shares over every CU would cut each sequence into dozens of
// pieces, whose merge then costs more than the keys. (64 since the merge folds a
// sequence's pieces in several workgroups and thread groups at once; measured
// graph-replayed: one 8192-key sequence 23.8 -> 21.0 us, 16 x 1024 keys 25.4 -> 20.6 us
// against 128, 32 no better; full batches, whose shares are larger, unchanged.) Shared
// by the decode kernel and its merge.
constexpr int64_t kMinDecodeShareKeys = 64;
__host__ __device__ inline int64_t decode_stream_shares(int64_t total_keys, int64_t wgs) {
  const int64_t cap = (total_keys + kMinDecodeShareKeys - 1) / kMinDecodeShareKeys;
  return cap < 1 ? 1 : (cap < wgs ? cap : wgs);
}

// Equal shares of `total` work units over `wgs` workgroups: workgroup w owns
// [floor(w * total / wgs), floor((w + 1) * total / wgs)).
__host__ __device__ inline int64_t share_begin(int64_t w, int64_t total, int64_t wgs) {
  return w * total / wgs;
}
// The workgroup owning unit x: the largest w whose share starts at or before x.
__host__ __device__ inline int64_t share_owner(int64_t x, int64_t total, int64_t wgs) {
  return ((x + 1) * wgs - 1) / total;
}
__host__ __device__ inline bool share_nonempty(int64_t w, int64_t total, int64_t wgs) {
  return (w * total) / wgs < ((w + 1) * total) / wgs;
}

// Query heads per decode wave for a GQA group of `group` heads.
__host__ __device__ inline int decode_group_chunk(int group) {
  return group % 4 == 0 ? 4 : (group % 2 == 0 ? 2 : 1);
}

struct PagedParams {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const float* k_scales;  // [num_blocks, H_k], fp8 pools only
  const float* v_scales;
  void* out;
  const int32_t* block_tables;
  const int32_t* cu_seqlens_q;
  const int32_t* context_lens;
  const int32_t* seq_lens;
  int num_seqs;
  int num_tokens;
  int hq;
  int hk;
  int max_blocks;
  int block_shift;
  int block_mask;
  int table_shift;        // slot of a table entry's first row = entry << table_shift (a
                          // paged pool: block_shift, entries are page ids; 0: entries
                          // are slot ids themselves)
  int64_t kv_row_bytes;   // pool bytes between consecutive slots (a paged pool: H_k D elements)
  int64_t kv_head_bytes;  // pool bytes between kv heads of one slot (a paged pool: D elements)
  int stream_wgs;     // decode: > 0 selects the stream schedule with this many workgroups
  int split_tokens;   // grid decode: nominal keys per split
  int max_splits;     // grid decode: grid extent along the split axis
  int by_row;         // grid decode: 1 = one unit per query row (serves prefill rows too)
  float scale;
  float* part_o;      // split partials, D fp32 each
  float* part_ml;     // split partials' (running max in log2 units, sum)
  int* seq_prefix;    // stream decode: [num_seqs + 1] decode keys before each sequence
  int pf_wgs;         // prefill: > 0 selects the stream schedule with this many workgroups
  int* pf_prefix;     // stream prefill: [num_seqs + 1] work units before each sequence
  float* pf_o;        // stream prefill partials: [2 * pf_wgs][heads][128][D] fp32, each
                      // piece normalised by its own sum
  float* pf_ml;       // their (max in log2 units, sum) per row: [2 * pf_wgs][heads][128][2]
  int pf_share_tiles;       // stream prefill: fewest key tiles per share; split grid:
                            // fewest key tiles per piece
  int pf_register_staging;  // 1: the register-staged prefill kernel even where the
                            // direct-to-LDS one serves (a plan option, for measurement)
  int pf_pieces;      // split grid: > 1 cuts long items into at most this many pieces (a
                      // 1-D grid of pf_ranks x columns); otherwise the (column,
                      // sequence, query tile) grid with every item whole
  int pf_ranks;       // split grid: grid extent in ranks (items + extra pieces bound)
  int pf_slots;       // split grid: partial slots per column
  int pf_cus;         // split grid: the device's CUs
  int pf_piece_pct;   // split grid: piece length, percent of the mean tiles per CU
  int* pf_count;      // split grid: [kSplitMaxItems][columns] arrival counters, zero
                      // before the launch and left zero by it
  float* pf_part;     // split grid: [pf_slots][columns] partials of kSplitSlotFloats
};

// Splits of one row: as many as its visible context needs at `split_tokens` keys
// each, never more than the grid provides. Shared by the decode kernel, the merge
// kernel and the host planner so that all three agree.
__host__ __device__ inline int decode_num_splits(int visible, int split_tokens, int max_splits) {
  int n = (visible + split_tokens - 1) / split_tokens;
  n = n < max_splits ? n : max_splits;
  return n < 1 ? 1 : n;
}

// Balanced split length: visible / n rounded up to a multiple of 16 keys.
__host__ __device__ inline int decode_split_len(int visible, int nsplit) {
  const int per = (visible + nsplit - 1) / nsplit;
  return (per + 15) & ~15;
}

hipError_t launch_paged_decode(const PagedParams& p, int q_dtype, int kv_dtype, int head_dim,
                               hipStream_t stream);

// The decode step's new token, taken by the stream decode from the projection's output
// rather than from the pool: every sequence s of a decode-only batch has its token at
// position context_lens[s] - 1; its q head vectors are QK-normed and rotated in the
// launch (as the QK-norm + RoPE kernel does, the same bits), its k row likewise, and k
// and v go to the pool slot the block table maps that position to (a page id outside
// [0, num_blocks) writes nothing) and into the attention straight from registers.
struct FreshParams {
  const void* q;          // raw q of row i at q + i q_stride (H_q D contiguous elements)
  const void* k;          // raw k and v of row i at k / v + i kv_stride (H_k D elements)
  const void* v;
  int64_t q_stride;       // elements between consecutive rows
  int64_t kv_stride;
  const void* q_weight;   // QK-norm weights, [D]
  const void* k_weight;
  const float* cos_t;     // [max_positions][D]
  const float* sin_t;
  int64_t max_positions;  // a position at or past it gives NaN rows, as the unfused kernel
  int64_t num_blocks;
  float eps;
};

// Stream decode with the new token formed in the launch (16-bit q and pool, head dim
// 128, p.stream_wgs > 0), then the merge, as launch_paged_decode.
hipError_t launch_paged_decode_fresh(const PagedParams& p, const FreshParams& f, int dtype,
                                     int head_dim, hipStream_t stream);

hipError_t launch_paged_prefill(const PagedParams& p, int q_dtype, int kv_dtype, int head_dim,
                                int max_query_len, hipStream_t stream);

// Whether launch_paged_prefill has a kernel for this shape; if not, prefill rows are
// served by the decode kernel in by-row mode.
bool paged_prefill_supported(int q_dtype, int kv_dtype, int head_dim, int hq, int hk,
                             int block_size);

}  // namespace mvllm
