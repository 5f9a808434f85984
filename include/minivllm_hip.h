/* C ABI of libminivllm_hip.so: the MI355X (gfx950) kernels of the Mini-vLLM
 * paged-attention hot path.
 *
 * The reference exposes these ops as the pybind11 module `mini_vllm_C`
 * (csrc/bindings.cpp:8-32,34-95), taking torch tensors. This library replaces that
 * module behind the same Python seam (mini_vllm/kernels/ops.py) with plain pointers,
 * sizes and an explicit stream, so any FFI can bind it.
 *
 * Conventions, all entry points:
 *   - return 0 on success, non-zero on failure; mvllm_last_error() then describes the
 *     failure (thread-local, valid until the next call on the same thread);
 *   - the callee never allocates device memory: the caller passes the output and any
 *     workspace (the reference allocates both with torch inside the call,
 *     csrc/paged_attention.cu:515-521,678);
 *   - work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and the call
 *     never synchronizes: results are ready when the stream reaches this point;
 *   - tensors are dense and row-major (contiguous) in the shapes given per function;
 *   - dtype codes: 0 = float32, 1 = float16, 2 = bfloat16, 3 = float8 e4m3fn (OCP).
 */
#ifndef MINIVLLM_HIP_H
#define MINIVLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVLLM_DTYPE_F32 0
#define MVLLM_DTYPE_F16 1
#define MVLLM_DTYPE_BF16 2
#define MVLLM_DTYPE_FP8_E4M3 3

#define MVLLM_OK 0
#define MVLLM_ERR_INVALID 1     /* an argument violates the contract */
#define MVLLM_ERR_UNSUPPORTED 2 /* valid, but no kernel serves this shape/dtype */
#define MVLLM_ERR_HIP 3         /* the HIP runtime reported an error */
#define MVLLM_ERR_WORKSPACE 4   /* workspace smaller than the plan requires */

/* Description of the most recent failure on this thread ("" if none). */
const char* mvllm_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int mvllm_abi_version(void);

/* Identity of the sources this library was built from: 16 hex digits of a SHA-256 over
 * the kernel sources, their headers and the compiler flags, stamped in by the build
 * ("unstamped" for a build that did not pass one). A loader compares it with the
 * sources beside it and refuses a stale library. */
const char* mvllm_build_id(void);

/* How one paged_attention call will be executed. Filled by mvllm_paged_attention_plan;
 * the caller provides `workspace_bytes` of device memory (256-byte aligned, contents
 * irrelevant) and passes it to mvllm_paged_attention with the same arguments. Calls
 * that overlap in time on one workspace race. */
#define MVLLM_DECODE_NONE 0   /* no decode row: every sequence is a prefill chunk */
#define MVLLM_DECODE_STREAM 1 /* persistent workgroups, equal shares of all decode keys */
#define MVLLM_DECODE_GRID 2   /* one workgroup per (sequence, split) */
#define MVLLM_DECODE_BY_ROW 3 /* one workgroup per (query row, split), prefill rows too */
typedef struct mvllm_paged_plan {
  int32_t decode_mode;       /* MVLLM_DECODE_* */
  int32_t decode_workgroups; /* stream: workgroups launched; grid modes: split-axis extent */
  int32_t split_tokens;      /* grid modes: keys per split */
  int32_t prefill_mfma;      /* 1: prefill rows go to the MFMA prefill kernel */
  uint64_t workspace_bytes;  /* split partials and their index; 0 when none are needed */
  int32_t prefill_workgroups; /* MFMA prefill: > 0 persistent workgroups with balanced
                                 shares of all key tiles (cut items merged after);
                                 0 one workgroup per (sequence, heads, query tile) */
  int32_t prefill_pieces;     /* MFMA prefill on the grid: > 1 items longer than ~1.2x
                                 the mean work per CU are cut into at most this many key
                                 ranges, run in the same launch longest first and merged
                                 by the last to finish; 0 every item whole */
} mvllm_paged_plan;

/* Explicit overrides of the planner's schedule choices, for measurement and for tests
 * that force one schedule; a zero field (or a NULL pointer for all of them) keeps the
 * planner's own choice. The library reads no environment: the schedule depends on
 * the sizes, the device's CU count and these options only. */
typedef struct mvllm_plan_options {
  int32_t decode_schedule;     /* 0 auto; MVLLM_DECODE_STREAM or MVLLM_DECODE_GRID forces
                                  one */
  int32_t decode_wgs_per_cu;   /* stream decode: workgroups per CU (default 1) */
  int32_t decode_waves_per_cu; /* grid decode: waves per CU the splits aim for (default 16) */
  int32_t decode_split_tokens; /* grid decode: keys per split (default from the wave target) */
  int32_t prefill_schedule;    /* 0 auto; 1 forces the stream schedule, 2 the grid */
  int32_t prefill_wgs_per_cu;  /* stream prefill: workgroups per CU (default 1) */
  int32_t prefill_staging;     /* 0 auto (direct-to-LDS copies where served); 1 forces the
                                  register-staged prefill kernel */
  int32_t prefill_share_tiles; /* stream prefill: fewest 64-key tiles per workgroup share
                                  while a quarter of the workgroups stay busy; grid
                                  prefill: fewest tiles per piece of a cut item
                                  (default 4): small work uses fewer workgroups */
  int32_t prefill_pieces;      /* grid prefill: most key-range pieces per item (default
                                  8); 1 keeps every item whole */
  int32_t prefill_piece_pct;   /* grid prefill: an item is cut into pieces of at least this
                                  percentage of the mean key tiles per CU (default 150,
                                  at least 50) */
} mvllm_plan_options;

/* The split prefill grid's arrival counters: regions taken on the current device (one
 * per stream that ran a split launch, at most 32), and the split launches (all devices)
 * that ran every item whole instead because no region was left or because their
 * stream was being captured into a graph (a captured launch must not name a stream's
 * counters: a replay on another stream could overlap it). No counterpart in the
 * reference. Any pointer may be NULL. */
void mvllm_split_stats(int32_t* regions_used, int64_t* whole_no_region,
                       int64_t* whole_capturing);

/* Plan a paged_attention call. Depends only on the host-side sizes below and the
 * options (never on device data), so it is free to call every iteration. Replaces the
 * grid/split selection of the reference's launch_paged_attention / splits_for
 * (csrc/paged_attention.cu:477-521). `options` may be NULL. */
int mvllm_paged_attention_plan(int32_t num_tokens, int32_t num_seqs, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t max_query_len, int32_t max_context_len, int32_t q_dtype,
                               int32_t kv_dtype, const mvllm_plan_options* options,
                               mvllm_paged_plan* plan);

/* Ragged attention over a paged KV cache: every scheduled token of every sequence in
 * one call. Replaces `mini_vllm_C.paged_attention` (csrc/bindings.cpp:23-32,81-94 ->
 * csrc/paged_attention.cu:598-711), called from mini_vllm/kernels/ops.py:239-250.
 *
 *   out, q        [num_tokens, num_q_heads, head_dim]           q_dtype
 *   key_pool,
 *   value_pool    [num_blocks, block_size, num_kv_heads, head_dim] kv_dtype
 *   k_scales,
 *   v_scales      [num_blocks, num_kv_heads] float32, required iff kv_dtype is fp8
 *                 (element = stored value * scale of its (page, kv head)); else NULL
 *   block_tables  [num_seqs, max_blocks_per_seq] int32, -1 padded
 *   cu_seqlens_q  [num_seqs + 1] int32   query rows of sequence s: [cu[s], cu[s+1])
 *   context_lens  [num_seqs] int32       keys sequence s attends over (S)
 *   seq_lens      [num_seqs] int32       query tokens of sequence s (L); L == 1 decodes
 *
 * Query r (0-based) of a sequence sees keys 0 .. S - L + r (causal with offset S - L).
 * max_query_len / max_context_len are host-side bounds over the batch (they size the
 * grid; no device read). scale multiplies q.k (the reference default is 1/sqrt(D)).
 * head_dim in {32, 64, 128, 256}; block_size a power of two; num_q_heads a multiple
 * of num_kv_heads; q_dtype in {f32, f16, bf16}; kv_dtype equals q_dtype, or is fp8
 * (with any q_dtype). `options` (may be NULL) must be the ones the plan was made with. */
int mvllm_paged_attention(void* out, const void* q, const void* key_pool,
                          const void* value_pool, const float* k_scales, const float* v_scales,
                          const int32_t* block_tables, const int32_t* cu_seqlens_q,
                          const int32_t* context_lens, const int32_t* seq_lens,
                          int32_t num_tokens, int32_t num_seqs, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int64_t num_blocks, int32_t max_blocks_per_seq, int32_t max_query_len,
                          int32_t max_context_len, float scale, int32_t q_dtype,
                          int32_t kv_dtype, const mvllm_plan_options* options, void* workspace,
                          uint64_t workspace_bytes, void* stream);

/* mvllm_paged_attention for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc); no
 * counterpart in the reference. The same arguments without the workspace: the split
 * partials go to a static device array of MVLLM_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on (the current device's) until the process ends, and the
 * call allocates nothing. A call whose plan needs more scratch than that returns
 * MVLLM_ERR_UNSUPPORTED (a prefill on the stream schedule needs up to ~66 MB at
 * H_q 16, D 128: plan options prefill_schedule = 2 put it on the grid, which needs
 * none). Nothing in the scratch needs to start at zero. Every call on one GPU shares
 * its array: calls that overlap in time on one GPU (two streams, two threads) race. */
#define MVLLM_NOALLOC_SCRATCH_BYTES (16u << 20)
int mvllm_paged_attention_noalloc(void* out, const void* q, const void* key_pool,
                                  const void* value_pool, const float* k_scales,
                                  const float* v_scales, const int32_t* block_tables,
                                  const int32_t* cu_seqlens_q, const int32_t* context_lens,
                                  const int32_t* seq_lens, int32_t num_tokens, int32_t num_seqs,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int64_t num_blocks,
                                  int32_t max_blocks_per_seq, int32_t max_query_len,
                                  int32_t max_context_len, float scale, int32_t q_dtype,
                                  int32_t kv_dtype, const mvllm_plan_options* options,
                                  void* stream);

/* Dense-cache attention: q, out [batch, query_len, num_q_heads, head_dim] contiguous
 * (token-major); k, v [batch, num_kv_heads, kv_len, head_dim] read through the given
 * element strides (head_dim contiguous), so a cache narrowed out of a larger buffer is
 * read in place. Query i (0-based) attends keys 0 .. kv_len - query_len + i: with
 * query_len == 1 every cached key (the reference's decode_attention), with query_len > 1
 * causally with offset kv_len - query_len (its flash_prefill). Replaces
 * `mini_vllm_C.decode_attention` / `mini_vllm_C.flash_prefill` (csrc/bindings.cpp:15-22,
 * 65-80 -> csrc/decode_attention.cu:360-435, csrc/flash_prefill.cu:282-355), called from
 * mini_vllm/kernels/ops.py:166-197. Served by the paged kernels over virtual 16-position
 * pages of the cache. Requires: dtype f32/f16/bf16 for q, k, v and out; head_dim in {32,
 * 64, 128, 256}; num_q_heads a multiple of num_kv_heads; kv_len >= query_len >= 1; k and
 * v sharing strides, the position and head strides multiples of 16 bytes, the batch
 * stride a multiple of the position stride, pointers 16-byte aligned (otherwise
 * MVLLM_ERR_UNSUPPORTED: the caller's PyTorch path serves it). The workspace (size from
 * mvllm_dense_attention_plan, 256-byte aligned, contents need not be initialised) holds
 * the virtual page tables and the split partials; calls that overlap on one workspace
 * race. */
typedef struct mvllm_dense_args {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  int64_t k_stride_batch, k_stride_head, k_stride_pos; /* elements */
  int64_t v_stride_batch, v_stride_head, v_stride_pos;
  int32_t batch;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t query_len;
  int32_t kv_len;
  int32_t head_dim;
  float scale;
  int32_t dtype;
} mvllm_dense_args;

int mvllm_dense_attention_plan(const mvllm_dense_args* args, uint64_t* workspace_bytes);
int mvllm_dense_attention(const mvllm_dense_args* args, void* workspace, uint64_t workspace_bytes,
                          void* stream);

/* RMSNorm over the last dimension: out = T(w * T(x * rsqrt(mean(x^2) + eps))), the sum
 * of squares in fp32. x, out [rows, dim]; weight [dim]; all of `dtype` (f32/f16/bf16).
 * Replaces `mini_vllm_C.rmsnorm` (csrc/bindings.cpp:9,44-49 -> csrc/rmsnorm.cu:121-169),
 * called from mini_vllm/kernels/ops.py:129-130; also serves QK-norm with dim = D. */
int mvllm_rmsnorm(void* out, const void* x, const void* weight, int64_t rows, int64_t dim,
                  float eps, int32_t dtype, void* stream);

/* Rotate-halves RoPE at explicit positions. x, out [rows, head_dim] where rows =
 * tokens * heads (token-major, heads inner); positions [num_positions] of
 * positions_bytes = 4 (int32) or 8 (int64), token t uses positions[t % num_positions];
 * cos_table, sin_table [max_positions, head_dim] float32. A position outside
 * [0, max_positions) yields NaN for that token instead of an out-of-bounds read.
 * Replaces `mini_vllm_C.rope` (csrc/bindings.cpp:10-13,51-57 -> csrc/rope.cu:115-195),
 * called from mini_vllm/kernels/ops.py:147-148. */
int mvllm_rope(void* out, const void* x, const void* positions, int32_t positions_bytes,
               const float* cos_table, const float* sin_table, int64_t rows, int64_t heads,
               int64_t head_dim, int64_t num_positions, int64_t max_positions, int32_t dtype,
               void* stream);

/* Qwen3's per-head QK-norm then RoPE, q and k in one launch: q_out = rope(rmsnorm(q,
 * q_weight)), k_out = rope(rmsnorm(k, k_weight)), bitwise equal to mvllm_rmsnorm followed
 * by mvllm_rope (same reduction order and rounding points). Replaces the four calls of
 * the reference's Qwen3PagedAttention (model/qwen3_paged.py:73-78: ops.rmsnorm x 2,
 * ops.rope x 2); no counterpart in mini_vllm_C.
 *   q, q_out [num_tokens, num_q_heads, head_dim]; k, k_out [num_tokens, num_kv_heads,
 *   head_dim]; q_weight, k_weight [head_dim]; all of `dtype` (f32/f16/bf16), 16-byte
 *   aligned. positions, cos_table, sin_table as for mvllm_rope. head_dim: 16-byte chunks
 *   per head a power of two from 2 to 64 (bf16: D = 16 .. 512). */
int mvllm_qk_norm_rope(void* q_out, void* k_out, const void* q, const void* k,
                       const void* q_weight, const void* k_weight, const void* positions,
                       int32_t positions_bytes, const float* cos_table, const float* sin_table,
                       int64_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, int64_t num_positions, int64_t max_positions, float eps,
                       int32_t dtype, void* stream);

/* mvllm_qk_norm_rope that also writes the paged KV pools of the layer, in the same
 * launch: each rotated k head row goes to key_pool at slot slot_mapping[token] (pool
 * [num_slots, num_kv_heads, head_dim], i.e. num_blocks x block_size slots, of `dtype`)
 * and v [num_tokens, num_kv_heads, head_dim] is copied to value_pool at the same slot; a
 * slot outside [0, num_slots) writes nothing (negative: padding rows of a captured
 * decode graph). The rotated k is not returned otherwise. Replaces the
 * rmsnorm/rope calls plus PagedKvPool.write's two index_copy_ (model/qwen3_paged.py:
 * 73-80 -> block/kv_pool.py:116-155) for a pool of q's dtype (an fp8 pool takes
 * mvllm_qk_norm_rope then mvllm_kv_write); no counterpart in mini_vllm_C. */
int mvllm_qk_norm_rope_kv_write(void* q_out, void* key_pool, void* value_pool, const void* q,
                                const void* k, const void* v, const void* q_weight,
                                const void* k_weight, const void* positions,
                                int32_t positions_bytes, const float* cos_table,
                                const float* sin_table, const int32_t* slot_mapping,
                                int64_t num_slots, int64_t num_tokens, int32_t num_q_heads,
                                int32_t num_kv_heads,
                                int32_t head_dim, int64_t num_positions, int64_t max_positions,
                                float eps, int64_t q_token_stride, int64_t kv_token_stride,
                                int32_t dtype, void* stream);
/* (q_token_stride / kv_token_stride: elements between consecutive tokens of q and of k
 * and v, whose heads are contiguous within a token; 0 means contiguous tensors. Column
 * views of the fused q/k/v projection's output pass its width, so the prefill path
 * needs no copies.) */

/* A decode step's attention with its new token's QK-norm, RoPE and KV write in the same
 * launch, for a decode-only batch (every sequence computes one token: seq_lens all 1,
 * cu_seqlens_q = 0, 1, ..., num_seqs, so row s is sequence s's) over a float16 or
 * bfloat16 pool with head_dim 128. Sequence s's token
 * sits at position context_lens[s] - 1 and goes to the slot its block table maps that
 * position to. The result equals, bit for bit, mvllm_qk_norm_rope_kv_write (positions
 * context_lens - 1, slot_mapping from the block tables) followed by
 * mvllm_paged_attention over the rotated q: the decode kernel forms the rotated q and
 * k rows itself (the same arithmetic), writes k and v to the pool, and takes the new
 * token's rows from registers, one launch fewer per layer. Replaces, for decode steps,
 * the reference Qwen3PagedAttention's norm/rope, PagedKvPool.write and
 * ops.paged_attention calls (model/qwen3_paged.py:71-95); no counterpart in
 * mini_vllm_C.
 *   out [num_seqs, num_q_heads, 128]; q (raw, before QK-norm) [num_seqs, num_q_heads,
 *   128] and k, v [num_seqs, num_kv_heads, 128] with token strides as for
 *   mvllm_qk_norm_rope_kv_write; q_weight, k_weight [128]; cos_table, sin_table
 *   [max_positions, 128] float32; the pools, tables and metadata as for
 *   mvllm_paged_attention (a table entry outside [0, num_blocks) writes nothing).
 * The workspace is the one mvllm_paged_attention_plan gives for num_tokens = num_seqs,
 * max_query_len = 1 and these options. A plan on the grid schedule (options, or more
 * than 4096 sequences) returns MVLLM_ERR_UNSUPPORTED: the caller then makes the two
 * calls. */
int mvllm_paged_decode_qk_norm_rope(
    void* out, const void* q, const void* k, const void* v, int64_t q_token_stride,
    int64_t kv_token_stride, const void* q_weight, const void* k_weight, const float* cos_table,
    const float* sin_table, int64_t max_positions, float eps, void* key_pool, void* value_pool,
    const int32_t* block_tables, const int32_t* cu_seqlens_q, const int32_t* context_lens,
    const int32_t* seq_lens, int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t max_blocks_per_seq,
    int32_t max_context_len, float scale, int32_t dtype, const mvllm_plan_options* options,
    void* workspace, uint64_t workspace_bytes, void* stream);

/* The token embedding lookup and the first block's input RMSNorm in one launch:
 * h_out[i] = the table row of row i's token (copied), out[i] = rmsnorm(h_out[i],
 * weight), bitwise the lookup then mvllm_rmsnorm. Row i's token is prev[index[i]] when
 * `index` is given and index[i] >= 0, else ids[i]: a decode step's input token is
 * either the one its sequence sampled in the previous step, still on the device
 * (`prev`), or the host's id. A token id outside [0, vocab) gives NaN rows and reads
 * nothing. Replaces the reference forward's Embedding lookup and its first block's
 * attn_norm (model/qwen3_paged.py:219 and 134); no counterpart in mini_vllm_C.
 *   table [vocab, dim], weight [dim], h_out / out [rows, dim], all of `dtype` and
 *   16-byte aligned; ids, index [rows] and prev int64 (index may be NULL, and prev
 *   then too). Dims as mvllm_add_rmsnorm. */
int mvllm_embed_rmsnorm(void* h_out, void* out, const void* table, int64_t vocab,
                        const int64_t* ids, const int64_t* index, const int64_t* prev,
                        int64_t rows, int32_t dim, const void* weight, float eps, int32_t dtype,
                        void* stream);

/* out = T(T(g * T(sigmoid(g))) * u) elementwise over n elements of `dtype`.
 * Replaces `mini_vllm_C.swiglu` (csrc/bindings.cpp:14,59-63 -> csrc/swiglu.cu:87-120),
 * called from mini_vllm/kernels/ops.py:161-162. */
int mvllm_swiglu(void* out, const void* gate, const void* up, int64_t n, int32_t dtype,
                 void* stream);

/* h_out = x + residual (rounded to dtype as torch's add rounds) and out = RMSNorm(h_out)
 * with weight and eps (rounded as mvllm_rmsnorm), all [rows, dim] contiguous: the
 * residual add and the norm after the o and down projections of prefill-sized steps
 * (model/qwen3_paged.py:97-99,111-113) in one pass. Dims beyond 512 16-byte chunks, or
 * not a whole number of chunks, return MVLLM_ERR_UNSUPPORTED; no counterpart in
 * mini_vllm_C. */
int mvllm_add_rmsnorm(void* h_out, void* out, const void* x, const void* residual,
                      const void* weight, int64_t rows, int32_t dim, float eps, int32_t dtype,
                      void* stream);

/* mvllm_swiglu over the fused gate/up projection's output: gate_up [rows, 2 cols] in
 * the 16-column interleave of mvllm_linear_swiglu's weight (columns 32j .. 32j+15: gate
 * columns 16j .. 16j+15; the next 16: the same up columns), out [rows, cols] contiguous;
 * cols a multiple of 16. Rounds as mvllm_swiglu. The prefill-sized MLP of
 * model/qwen3_paged.py:101-111 after one BLAS call over the interleaved weight; no
 * counterpart in mini_vllm_C. */
int mvllm_swiglu_interleaved(void* out, const void* gate_up, int64_t rows, int64_t cols,
                             int32_t dtype, void* stream);

/* Scatter one iteration's keys and values into their pool slots, K and V in one
 * launch. Replaces the two index_copy_ calls of PagedKvPool.write
 * (mini_vllm/block/kv_pool.py:116-155; slot_mapping from mini_vllm/serve/batch.py:158-166).
 *   key_pool,
 *   value_pool   [num_blocks, block_size, num_kv_heads, head_dim] pool_dtype
 *   k_scales,
 *   v_scales     [num_blocks, num_kv_heads] float32, read and updated; required iff
 *                pool_dtype is fp8, else NULL
 *   key, value   [num_tokens, num_kv_heads, head_dim] src_dtype (f32, f16, bf16)
 *   slot_mapping [num_tokens] int32 flat slot (block * block_size + offset); a slot
 *                outside [0, num_blocks * block_size) skips its token (negative:
 *                padding rows of a captured decode graph)
 * pool_dtype == src_dtype copies. An fp8 pool (head_dim 32, 64, 128 or 256; no
 * counterpart in the reference) is quantised per (block, kv head): a call's tokens on
 * consecutive rows of one block form
 * a run (a block must get at most one run per call); a run starting at row 0 opens the
 * block; scale s = max(old scale, least power of two >= max|x| / 448) over the run;
 * rows already in the block are re-encoded as e4m3((code * old) / s) when s grew (an
 * exponent shift: exact unless a value falls into e4m3's subnormals); new rows are
 * e4m3(x / s), round to nearest even, 0 when s is 0. */
int mvllm_kv_write(void* key_pool, void* value_pool, float* k_scales, float* v_scales,
                   const void* key, const void* value, const int32_t* slot_mapping,
                   int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                   int32_t block_size, int64_t num_blocks, int32_t src_dtype,
                   int32_t pool_dtype, void* stream);

/* The skinny projections below read W pre-shuffled into MFMA fragment order ("packed"),
 * made once when the weights are loaded: for each tile of 32 rows (t) and each k-step of
 * 16 elements (s), the 64 x 16 bytes one wave loads for one matrix-core operand lie
 * contiguously, 16 bytes l = 32 h + r holding W[32 t + r][16 s + 8 h .. 16 s + 8 h + 7]
 * at byte offset ((t * k/16 + s) * 64 + l) * 16; rows past n are zeros. The packed
 * buffer holds ceil(n / 32) * 32 * k elements. This packs row-major W [n, k] (fp16 or
 * bf16, k a multiple of 64, both buffers 16-byte aligned) on `stream`. No counterpart in
 * the reference: its projections read torch's row-major weights (model/loader.py). */
int mvllm_linear_pack(void* w_packed, const void* w, int64_t n, int64_t k, int32_t dtype,
                      void* stream);

/* Device bytes of workspace the skinny projections below need for [m, k] x [n, k]^T (n =
 * n0 + n1 + n2 for mvllm_linear_split, 2 n_out for mvllm_linear_swiglu): 0 for k <= 1024,
 * else the fp32 partial sums of its k ranges (4 per 1024 of k, 4 KB (m <= 32) or 8 KB per
 * 32 columns each). 256-byte aligned, contents need not be initialised; calls that
 * overlap in time on one workspace race. */
uint64_t mvllm_linear_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* Skinny projection y[m, n] = x[m, k] w[n, k]^T (torch's x @ w.T, no bias) with w packed
 * as above, fp32 accumulation, for the few rows of a decode step: m <= 64, k a multiple
 * of 64 up to 65536, x and w 16-byte aligned, dtype f16 or bf16; anything else returns
 * MVLLM_ERR_UNSUPPORTED (the caller's BLAS serves it). Replaces the projection matmuls
 * of the caller (model/qwen3_paged.py:71-95,110 -> model/basics.py linear ->
 * torch.matmul); no counterpart in mini_vllm_C. The result is the fp32 sum rounded
 * once, but summed in a different order than a BLAS would, so it may differ from torch
 * in the last bit. The order depends on k alone, so the fused variants below equal
 * this entry bit for bit. */
int mvllm_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                 int32_t dtype, void* workspace, uint64_t workspace_bytes, void* stream);

/* The same projection over w = pack([w0; w1; w2]) (n0 + n1 + n2 rows) with its columns written
 * to three outputs: y0 [m, n0], y1 [m, n1], y2 [m, n2]; n0 and n1 multiples of 32. One
 * launch for the q, k and v projections of model/qwen3_paged.py:71-73. */
int mvllm_linear_split(void* y0, void* y1, void* y2, const void* x, const void* w, int64_t m,
                       int64_t n0, int64_t n1, int64_t n2, int64_t k, int32_t dtype,
                       void* workspace, uint64_t workspace_bytes, void* stream);

/* y = residual + x w^T with residual [m, n]: the projection rounded to the dtype, then
 * the add rounded again, as the two torch ops round them (model/qwen3_paged.py:136-138,
 * `h + wo(...)` and `h + down(...)`). */
int mvllm_linear_residual(void* y, const void* x, const void* w, const void* residual, int64_t m,
                          int64_t n, int64_t k, int32_t dtype, void* workspace,
                          uint64_t workspace_bytes, void* stream);

/* y [m, n_out] = swiglu(x gate^T, x up^T) in one launch (model/qwen3_paged.py:110, the
 * gate and up projections then ops.swiglu), with w_gate_up [2 n_out, k] holding gate and
 * up rows interleaved in groups of 16 (rows 32j .. 32j+15: gate rows 16j .. 16j+15; the
 * next 16: the same up rows); n_out a multiple of 16. Gate and up are rounded to the
 * dtype before the SwiGLU, which rounds as mvllm_swiglu does; w_gate_up is packed. */
int mvllm_linear_swiglu(void* y, const void* x, const void* w_gate_up, int64_t m, int64_t n_out,
                        int64_t k, int32_t dtype, void* workspace, uint64_t workspace_bytes,
                        void* stream);

/* y [m, n] = x [m, k] w [n, k]^T through hipBLASLt, all row-major and contiguous,
 * 16-byte aligned, fp16 or bf16 (dtype), fp32 accumulation: the vendor BLAS product the
 * reference's projections run at prefill sizes (mini_vllm/basics.py:18 linear, x @ w.T
 * through torch, called from model/qwen3_paged.py:71-95, 110 and 141-143), with its
 * per-call set-up kept: the matmul and layout descriptors are made on the first call of
 * each (device, dtype, m, n, k), the algorithm on the first call of each (device, dtype,
 * n, k, 128-row bucket of m) - the fastest of the heuristic's first 16 candidates for
 * the bucket's largest, odd, m, each timed on that call's own operands (one host wait;
 * a call whose stream is being captured takes the heuristic's first untimed); m a
 * multiple of 128 gets its exact shape's candidates, and a shape hipBLASLt refuses the
 * bucket's algorithm for gets the heuristic's first for its own m - and both reused (at
 * most 4096 shapes kept; past that all are dropped and made again as called).
 * `workspace` is the caller's: at least mvllm_blas_workspace_bytes() bytes, 256-byte
 * aligned; calls on one stream may share one (they are ordered). The library allocates
 * no device memory. Calls from several host threads are serialised. A shape hipBLASLt
 * has no algorithm for returns MVLLM_ERR_UNSUPPORTED before any launch. */
int mvllm_blas_linear(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                      int32_t dtype, void* workspace, uint64_t workspace_bytes, void* stream);

/* Bytes of the workspace mvllm_blas_linear takes. */
uint64_t mvllm_blas_workspace_bytes(void);

/* An explicit sweep for mvllm_blas_linear (no counterpart in the reference, which takes
 * torch's heuristic algorithm): times every algorithm hipBLASLt holds that serves
 * y = x w^T at this (m, n, k) on the caller's operands and stream (one warm-up and 3 runs
 * each, one host wait per algorithm: ~0.5 s for a Qwen3-0.6B projection) and keeps the 12
 * fastest as extra candidates that every later algorithm choice of (n, k) also times,
 * each checked against that bucket's m first; choices already made for (n, k) are made
 * again. Leaves y = x w^T. Operands and workspace as mvllm_blas_linear; refused with
 * MVLLM_ERR_UNSUPPORTED while `stream` is being captured (it waits on the host).
 * `timed` (may be NULL) receives the algorithms timed. Serving engines call it once per
 * projection shape at start-up. */
int mvllm_blas_tune(void* y, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                    int32_t dtype, void* workspace, uint64_t workspace_bytes, void* stream,
                    int32_t* timed);

/* Shapes mvllm_blas_linear currently keeps (for tests). */
int mvllm_blas_plans_cached(void);

/* How mvllm_blas_linear chose the algorithm it keeps for a shape. */
typedef struct mvllm_blas_choice {
  int32_t candidates; /* the heuristic's candidates considered */
  int32_t timed;      /* how many were timed (0: the first taken untimed) */
  int32_t chosen;     /* the kept one's index in the heuristic's order */
  float first_us;     /* the heuristic's first, per product (-1 untimed) */
  float chosen_us;    /* the kept one, per product (-1 untimed) */
} mvllm_blas_choice;

/* The choice record for (current device, dtype, m, n, k); MVLLM_ERR_INVALID if that
 * shape has not been called (or was dropped). For reports and tests. */
int mvllm_blas_tuning(int64_t m, int64_t n, int64_t k, int32_t dtype, mvllm_blas_choice* out);

/* h_out = residual + x w^T (rounded as mvllm_linear_residual) and normed = RMSNorm(h_out)
 * with norm_weight and eps (rounded as mvllm_rmsnorm: bit for bit the two entries in
 * sequence), h_out, normed, residual [m, n], norm_weight [n]: the o and down projections
 * of model/qwen3_paged.py:97,111,136-138 with the RMSNorm that follows each (the MLP
 * norm, the next layer's attention norm or the final norm), in two launches instead of
 * three. k > 1024 (the split path), n a multiple of 512 up to 4096, other shapes return
 * MVLLM_ERR_UNSUPPORTED; workspace as for mvllm_linear. */
int mvllm_linear_residual_rmsnorm(void* h_out, void* normed, const void* x, const void* w,
                                  const void* residual, const void* norm_weight, int64_t m,
                                  int64_t n, int64_t k, float eps, int32_t dtype, void* workspace,
                                  uint64_t workspace_bytes, void* stream);

/* Greedy sampling: out[r] (int64) = index of the maximum of logits row r, for `rows`
 * rows of `vocab` logits each, `row_stride` elements apart, dtype f32/f16/bf16. The
 * order is torch.argmax's: NaN above every number, -0 equal to +0, and among equal
 * maxima the first index. Replaces `logits.argmax(dim=-1)` of the greedy sampler
 * (mini_vllm/sampler.py:135-141; the engine's decode step, engine.py); no counterpart in
 * mini_vllm_C. Two launches for rows longer than 16384 logits (segments per workgroup,
 * then one wave per row), one otherwise. */
int mvllm_argmax(int64_t* out, const void* logits, int64_t rows, int64_t vocab,
                 int64_t row_stride, int32_t dtype, void* workspace, uint64_t workspace_bytes,
                 void* stream);
/* Workspace of mvllm_argmax (8-byte aligned, contents need not be initialised): one
 * 8-byte key per 16384-logit segment of each row; 0 for rows of at most 16384 logits.
 * Rows may hold up to 64 segments (1048576 logits). */
uint64_t mvllm_argmax_workspace_bytes(int64_t rows, int64_t vocab);

/* Read-only HBM probe for the benchmark's bandwidth ceiling (no counterpart in the
 * reference, whose ceiling is a device copy, mini_vllm/bench.py:448-466): reads
 * `num_pages` pages of `page_bytes` (4-64 KB, a multiple of 4 KB) from `base`, page i at
 * page_ids[i] (device int32, every id in [0, base_bytes / page_bytes)) or at i when
 * page_ids is NULL, with `workgroups` workgroups of 256 lanes, each lane's 16-byte
 * nontemporal loads of a page all in flight before use; stores one folded word per
 * lane into `sink` (sink_words >= 256 x workgroups). */
int mvllm_read_probe(const void* base, int64_t base_bytes, const int32_t* page_ids,
                     int64_t num_pages, int64_t page_bytes, int32_t workgroups, uint32_t* sink,
                     int64_t sink_words, void* stream);

/* y = a * x + b over n floats: the toolchain smoke test, replacing `mini_vllm_C.hello`
 * (csrc/bindings.cpp:8,37-42 -> csrc/hello.cu:11-21; mini_vllm/kernels/extension.py:349-353). */
int mvllm_axpby(float* y, const float* x, float a, float b, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINIVLLM_HIP_H */
