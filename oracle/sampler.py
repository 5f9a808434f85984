"""CPU restatement of the reference's sampling distribution (mini_vllm/sampler.py:71-124).
Test infrastructure only: imported by tests/, never by the product path.

``sampling_probabilities(logits, temperature, top_k, top_p)`` over numpy arrays, in
float64, row by row:

  * temperature 0: the one-hot of the first maximal logit (sampler.py:116-122);
  * else p = softmax(logits / temperature); in descending order of p (ties in
    vocabulary order: a stable sort), keep rank r while r < top_k (0: no limit) and
    the mass strictly before it is < top_p (1: no limit), and always rank 0
    (sampler.py:100-111); renormalise (sampler.py:113-114).

Pinned in tests/test_sampler_cpu.py by closed forms rather than by restating it: the
temperature-1 distribution is the softmax, top-k keeps exactly k tokens and they are
the k largest logits, a top-p nucleus reaches p and loses that property without its
last member, four equal logits with p = 0.5 / 0.6 keep 2 / 3 tokens, top-k 1 equals
greedy, and kept tokens keep their relative odds.
"""

from __future__ import annotations

import numpy as np

__all__ = ["sampling_probabilities"]


def sampling_probabilities(logits: np.ndarray, temperature, top_k, top_p) -> np.ndarray:
    """``logits``: B x V; the three parameters: one value each or one per row."""
    x = np.asarray(logits, dtype=np.float64)
    batch, vocab = x.shape
    t = np.broadcast_to(np.asarray(temperature, dtype=np.float64), (batch,))
    k = np.broadcast_to(np.asarray(top_k, dtype=np.int64), (batch,))
    p = np.broadcast_to(np.asarray(top_p, dtype=np.float64), (batch,))
    out = np.zeros((batch, vocab), dtype=np.float64)
    for b in range(batch):
        if t[b] == 0.0:
            out[b, int(np.argmax(x[b]))] = 1.0
            continue
        s = x[b] / t[b]
        e = np.exp(s - s.max())
        probs = e / e.sum()
        order = np.argsort(-probs, kind="stable")
        desc = probs[order]
        before = np.concatenate([[0.0], np.cumsum(desc)[:-1]])
        limit = vocab if k[b] == 0 else k[b]
        # top_p = 1 disables the rule, as SamplingParams documents (sampler.py:29-31);
        # applied literally, a running sum over a large vocabulary can reach 1 before
        # its last token and drop the tail
        keep = (np.arange(vocab) < limit) & ((before < p[b]) | (p[b] >= 1.0))
        keep[0] = True
        kept = desc * keep
        out[b, order] = kept / kept.sum()
    return out
