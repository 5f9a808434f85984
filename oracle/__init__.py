"""CPU oracle for the paged-attention hot path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker (or, for the baseline, as the CPU
restatement being timed) -- never as the thing measured or shipped. The product
path (``mini-vllm_amd/``) does not import it.

Contents
  paged_attention.py  gather-then-dense paged attention in torch on the CPU, fp32
                      (or fp64): the reference's CPU path (mini_vllm/paged_attention.py:
                      36-110 over attention.py:68-158 and basics.py:44-65), restated.
  brute.c             an independent float64 brute force of the same function: one
                      (sequence, query, head) at a time, walking the block table per key.
  brute.py            ctypes loader for brute.c (built into oracle/_build/ by the
                      Makefile, or on first use).
  elementwise.py      numpy restatements of rms_norm, apply_rope and silu(g)*u with
                      the reference's rounding points, and bf16/fp16/e4m3 rounding.

Pinning (what fixes each function independently of its own formula) is in the
docstrings and in tests/test_oracle.py: golden vectors under tests/golden/, the
reference's known-answer properties, and closed forms. The reference's kernels are
CUDA and cannot be built here, so there is no oracle/_ref.
"""
