"""CPU restatement of the paged KV write. Test infrastructure only: imported by tests/,
never by the product path.

* ``kv_write_copy`` -- the reference's ``PagedKvPool.write`` (block/kv_pool.py:116-155):
  ``flat_pool.index_copy_(0, slot_mapping, x)`` on the ``num_slots x H_k x D`` view,
  for K and V. Pinned in tests against torch's ``index_copy_`` itself. A negative slot
  skips its token here (the reference would raise on it; the library's callers use -1
  for padding rows).
* ``kv_write_fp8`` -- the fp8-e4m3 quantising write, which has no counterpart in the
  reference (its pools are never fp8). The policy, per (block, kv head), for K and V
  separately:
    - a *run* is a maximal stretch of the call's tokens on consecutive rows of one
      block; a run starting at row 0 opens the block (old scale and rows are dead);
    - s = max(old scale, pow2ceil(amax / 448)) over the run's rows, in fp32 (0 if all
      are 0), pow2ceil = the least power of two >= its argument: scales are powers of
      two, so re-encoding old rows under a grown scale is an exponent shift;
    - if s grew and the old scale was > 0, rows [0, first row) are re-encoded as
      e4m3((decode(code) * old) / s);
    - the run's rows become e4m3(x / s) (0 when s = 0), round to nearest even,
      saturating at 448 (``oracle.elementwise.fp8_e4m3_encode``, pinned against torch's
      ``float8_e4m3fn`` cast);
  every operation one fp32 rounding, so the GPU kernel must match these bytes exactly.
  Pinned by (a) a single run over a fresh block equals a direct per-block quantisation
  of that block at scale pow2ceil(amax / 448) (the quantiser of BASELINE config 4,
  ``workloads.quantize_fp8_per_block``, with that scale), (b) the final scale of a
  block written token by token equals pow2ceil(amax / 448) of the whole block (a closed
  form), and (c) every decoded value within half an e4m3 step of its source at the
  scale it was written with (re-encoding being exact above the subnormals).
"""

from __future__ import annotations

import numpy as np

from oracle.elementwise import fp8_e4m3_decode, fp8_e4m3_encode

__all__ = ["kv_write_copy", "kv_write_fp8", "pow2_ceil", "runs"]


def pow2_ceil(t: np.ndarray) -> np.ndarray:
    """Least power of two >= t, elementwise on float32 (0 stays 0): clear the mantissa
    and, if it was not clear, step the exponent."""
    t = np.asarray(t, dtype=np.float32)
    b = t.view(np.uint32)
    up = np.where((b & 0x7FFFFF) == 0, b, (b & 0x7F800000) + 0x800000).astype(np.uint32)
    return up.view(np.float32)


def kv_write_copy(pool: np.ndarray, slots: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``pool``: num_blocks x P x H_k x D; ``x``: T x H_k x D. Returns the updated pool."""
    out = np.array(pool, copy=True)
    flat = out.reshape(-1, *out.shape[2:])
    for t, slot in enumerate(np.asarray(slots).tolist()):
        if slot >= 0:
            flat[slot] = x[t]
    return out


def runs(slots: np.ndarray, block_size: int) -> list[tuple[int, int]]:
    """(first token, length) of every run: consecutive tokens on consecutive rows of one
    block. Negative slots belong to no run."""
    slots = np.asarray(slots).tolist()
    out = []
    t = 0
    while t < len(slots):
        if slots[t] < 0:
            t += 1
            continue
        n = 1
        while (t + n < len(slots) and slots[t + n] >= 0
               and slots[t + n] // block_size == slots[t] // block_size
               and slots[t + n] % block_size == slots[t] % block_size + n):
            n += 1
        out.append((t, n))
        t += n
    return out


def kv_write_fp8(codes: np.ndarray, scales: np.ndarray, slots: np.ndarray,
                 x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``codes``: num_blocks x P x H_k x D uint8 (e4m3fn bytes); ``scales``: num_blocks x
    H_k float32; ``x``: T x H_k x D (any float; taken as float32). Returns updated
    (codes, scales)."""
    codes = np.array(codes, dtype=np.uint8, copy=True)
    scales = np.array(scales, dtype=np.float32, copy=True)
    x = np.asarray(x, dtype=np.float32)
    block_size = codes.shape[1]
    hk = codes.shape[2]
    f448 = np.float32(448.0)
    for t0, n in runs(slots, block_size):
        slot0 = int(slots[t0])
        block, row0 = slot0 // block_size, slot0 % block_size
        for h in range(hk):
            rows = x[t0:t0 + n, h]
            amax = np.float32(np.abs(rows).max())
            old = np.float32(0.0) if row0 == 0 else scales[block, h]
            s = np.maximum(old, pow2_ceil(np.float32(amax / f448)))
            if old > 0 and s > old:
                prev = fp8_e4m3_decode(codes[block, :row0, h])
                codes[block, :row0, h] = fp8_e4m3_encode(
                    ((prev * old).astype(np.float32) / s).astype(np.float32))
            if s > 0:
                enc = fp8_e4m3_encode((rows / s).astype(np.float32))
            else:
                enc = np.zeros(rows.shape, dtype=np.uint8)
            codes[block, row0:row0 + n, h] = enc
            scales[block, h] = s
    return codes, scales
