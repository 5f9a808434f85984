"""Regenerate the golden fixtures in this directory (test infrastructure).

The reference ships no golden vectors for paged attention (its tests draw seeded
``randn`` at run time), so the fixtures are produced by this repository's float64
brute-force oracle (oracle/brute.c) on seeded inputs:

  paged_cfg1.npz        BASELINE config 1 (fp32 decode, 4 seqs, ctx {37,128,511,1000},
                        512-block shuffled pool, GQA 16/8, D=128, P=16, seed 0)
  paged_mixed_small.npz a mixed batch: decode rows beside prefill chunks with causal
                        offsets, GQA 8/2, D=64, P=16, seed 5

Each file stores the float64 output and fingerprints of the seeded inputs (sums and
the block tables), so a change in the generator is caught rather than read as a
kernel bug.  Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path[:0] = [str(REPO / "mini-vllm_amd"), str(REPO)]

from mini_vllm.workloads import build_batch, config_batch  # noqa: E402
from oracle import brute  # noqa: E402

CASES = {
    "paged_cfg1": lambda: config_batch(1),
    "paged_mixed_small": lambda: build_batch(
        [300, 1, 17, 50], [1, 1, 17, 8], num_q_heads=8, num_kv_heads=2, head_dim=64, seed=5
    ),
}


def fingerprint(batch) -> dict[str, np.ndarray]:
    return {
        "fp_keys": np.array(batch.key_pool.double().sum().item()),
        "fp_values": np.array(batch.value_pool.double().sum().item()),
        "fp_q": np.array(batch.q.double().sum().item()),
        "block_tables": batch.block_tables.numpy(),
        "contexts": np.array(batch.contexts, dtype=np.int32),
        "query_lens": np.array(batch.query_lens, dtype=np.int32),
    }


def main() -> None:
    for name, make in CASES.items():
        batch = make()
        out = brute.paged_attention_f64(batch.q, batch.key_pool, batch.value_pool,
                                        batch.block_tables, batch.cu_seqlens_q,
                                        batch.context_lens, batch.scale)
        np.savez_compressed(HERE / f"{name}.npz", out=out, **fingerprint(batch))
        print(f"wrote {name}.npz  out {out.shape}")


if __name__ == "__main__":
    main()
