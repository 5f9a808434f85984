/* Float64 brute-force paged attention: test infrastructure only.
 *
 * An independent restatement of the reference's paged attention semantics
 * (mini_vllm/paged_attention.py:36-110; causal offset attention.py:76-92; slot
 * arithmetic csrc/paged_attention.cu:87-93): for every sequence s, query row r of its
 * L = cu[s+1] - cu[s] rows, and query head h, the output is
 *
 *     softmax_j( scale * q[cu[s]+r][h] . K[slot_s(j)][h / G] ),  j = 0 .. S - L + r
 *     applied to V[slot_s(j)][h / G],
 *
 * slot_s(j) = table[s][j / P] * P + j % P. Everything in double, one query at a time,
 * with no shared code with the torch oracle or the kernels.
 *
 * Returns 0, or -1 when a sequence computes more tokens than it attends over, or -2
 * when a key position falls on a negative (padding) table entry.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

int oracle_paged_attention_f64(const float* q, const float* key_pool, const float* value_pool,
                               const int32_t* block_tables, const int32_t* cu_seqlens_q,
                               const int32_t* context_lens, int32_t num_seqs,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t block_size, int32_t max_blocks, double scale,
                               double* out) {
  const int group = num_q_heads / num_kv_heads;
  int32_t max_ctx = 0;
  for (int s = 0; s < num_seqs; ++s)
    if (context_lens[s] > max_ctx) max_ctx = context_lens[s];
  double* scores = (double*)malloc(sizeof(double) * (size_t)(max_ctx > 0 ? max_ctx : 1));
  int64_t* slots = (int64_t*)malloc(sizeof(int64_t) * (size_t)(max_ctx > 0 ? max_ctx : 1));
  if (!scores || !slots) {
    free(scores);
    free(slots);
    return -3;
  }
  int rc = 0;
  for (int s = 0; s < num_seqs && rc == 0; ++s) {
    const int L = cu_seqlens_q[s + 1] - cu_seqlens_q[s];
    const int S = context_lens[s];
    if (L == 0) continue;
    if (S < L) { rc = -1; break; }
    for (int j = 0; j < S; ++j) {
      const int32_t block = block_tables[(int64_t)s * max_blocks + j / block_size];
      if (block < 0) { rc = -2; break; }
      slots[j] = (int64_t)block * block_size + j % block_size;
    }
    if (rc) break;
    for (int r = 0; r < L; ++r) {
      const int visible = S - L + r + 1;
      const int64_t row = cu_seqlens_q[s] + r;
      for (int h = 0; h < num_q_heads; ++h) {
        const int kvh = h / group;
        const float* qv = q + (row * num_q_heads + h) * head_dim;
        double m = -INFINITY;
        for (int j = 0; j < visible; ++j) {
          const float* kv = key_pool + (slots[j] * num_kv_heads + kvh) * head_dim;
          double dot = 0.0;
          for (int d = 0; d < head_dim; ++d) dot += (double)qv[d] * (double)kv[d];
          scores[j] = dot * scale;
          if (scores[j] > m) m = scores[j];
        }
        double total = 0.0;
        for (int j = 0; j < visible; ++j) {
          scores[j] = exp(scores[j] - m);
          total += scores[j];
        }
        double* o = out + (row * num_q_heads + h) * head_dim;
        for (int d = 0; d < head_dim; ++d) o[d] = 0.0;
        for (int j = 0; j < visible; ++j) {
          const double w = scores[j] / total;
          const float* vv = value_pool + (slots[j] * num_kv_heads + kvh) * head_dim;
          for (int d = 0; d < head_dim; ++d) o[d] += w * (double)vv[d];
        }
      }
    }
  }
  free(scores);
  free(slots);
  return rc;
}
