"""The seam between the model and its kernels (reference mini_vllm/kernels/ops.py).

Same op names, signatures and ``use_cuda`` switch as the reference, so the model,
engine and tests above it run unchanged:

    rmsnorm(x, weight, eps=1e-6, use_cuda=False)                       ops.py:117-131
    rope(x, positions, cos, sin, use_cuda=False)                       ops.py:134-149
    swiglu(gate, up, use_cuda=False)                                   ops.py:152-163
    paged_attention(q, key_pool, value_pool, block_tables, cu_seqlens_q,
                    context_lens, seq_lens, max_query_len, max_context_len,
                    scale=None, use_cuda=False)                        ops.py:200-254

plus ops that fuse what the reference's caller does in several calls:

    kv_write(key_pool, value_pool, key, value, slot_mapping, use_cuda=False,
             *, k_scale=None, v_scale=None)    PagedKvPool.write: kv_pool.py:116-155
    qk_norm_rope(q, k, q_weight, k_weight, positions, cos, sin, eps=1e-6,
                 use_cuda=False)               qwen3_paged.py:73-78 (2 rmsnorm + 2 rope)
    qk_norm_rope_kv_write(...)                 the two above in one launch
    embed_rmsnorm(table, ids, weight, eps)     the token embedding and the first block's
                                               input norm in one launch (219, 134)
    paged_decode_qk_norm_rope(...)             a decode step's qk_norm_rope_kv_write and
                                               paged_attention in one launch (71-95)

The callee behind ``use_cuda=True`` is ``libminivllm_hip.so`` (HIP for gfx950).

Routing follows the reference (ops.py:82-89): ``use_cuda=True`` means "use a kernel
where one applies". A call the kernels cannot serve -- CPU tensors (the same model
object serves CPU tests and GPU serving), a head dim or dtype mix the library does not
take, a non-contiguous pool, int64 tables -- runs the PyTorch path
(:mod:`mini_vllm.torch_path`) instead, and :func:`dispatch_report` lists every such
decline of the process with its reason. Because a silent fallback is also how a kernel
that never ran ends up in a benchmark, :func:`set_strict` (or the environment variable
``MINIVLLM_STRICT_KERNELS=1`` at import, or the :func:`strict_kernels` context) turns
every decline into a ``RuntimeError`` naming the reason; ``bench.py`` and the GPU
tests run strict. Ops that route by size rather than by capability (projections of
prefill-sized inputs go to the vendor BLAS) are not declines.
"""

from __future__ import annotations

import math
import os
from contextlib import contextmanager
from dataclasses import dataclass

import torch

from mini_vllm import torch_path
from mini_vllm.kernels.extension import load_extension

__all__ = [
    "CUDA_KERNELS",
    "argmax",
    "NOT_YET_FASTER",
    "attention",
    "cuda_kernel_names",
    "dispatch_report",
    "embed_rmsnorm",
    "kv_write",
    "PackedWeight",
    "linear",
    "linear_residual",
    "linear_residual_rmsnorm",
    "linear_split",
    "linear_swiglu",
    "pack_weight",
    "paged_attention",
    "paged_decode_qk_norm_rope",
    "qk_norm_rope",
    "qk_norm_rope_kv_write",
    "rmsnorm",
    "rope",
    "set_strict",
    "strict_kernels",
    "swiglu",
]

# op name -> (has a kernel in libminivllm_hip.so, source file). The keys are the
# method names of the bound extension (`load_extension()`), kept from the reference.
CUDA_KERNELS: dict[str, tuple[bool, str]] = {
    "rmsnorm": (True, "csrc/elementwise.hip"),
    "rope": (True, "csrc/elementwise.hip"),
    "swiglu": (True, "csrc/elementwise.hip"),
    "argmax": (True, "csrc/sampler.hip"),
    "decode_attention": (True, "csrc/dense.hip over the paged decode kernels"),
    "flash_prefill": (True, "csrc/dense.hip over the paged prefill kernels"),
    "paged_attention": (True, "csrc/paged_decode.hip + csrc/paged_prefill.hip"),
    "kv_write": (True, "csrc/kv_write.hip"),
    "qk_norm_rope": (True, "csrc/elementwise.hip"),
    "linear": (True, "csrc/linear.hip (at most 64 rows; vendor BLAS above)"),
    "blas_linear": (True, "csrc/blas.hip (prefill-sized projections on hipBLASLt, set-up kept "
                          "per shape)"),
}

# Kernels that exist but are deliberately not dispatched, with the reason.
NOT_YET_FASTER: dict[str, str] = {}

MAX_PAGED_HEAD_DIM = 256
PAGED_HEAD_DIMS = (32, 64, 128, 256)


# Declines of this process: op name -> {reason: count}.
FALLBACKS: dict[str, dict[str, int]] = {}

_strict = os.environ.get("MINIVLLM_STRICT_KERNELS", "").strip() not in ("", "0")


def set_strict(flag: bool) -> bool:
    """Make every decline raise (True) or fall back to the PyTorch path (False, the
    reference's behaviour and the default); returns the previous setting."""
    global _strict
    previous, _strict = _strict, bool(flag)
    return previous


def is_strict() -> bool:
    return _strict


@contextmanager
def strict_kernels(flag: bool = True):
    """``with strict_kernels():`` -- :func:`set_strict` for the duration of a block."""
    previous = set_strict(flag)
    try:
        yield
    finally:
        set_strict(previous)


def _decline(name: str, reason: str) -> bool:
    """A ``use_cuda=True`` call the kernel cannot serve: recorded and routed to the
    PyTorch path (returns False), or raised in strict mode."""
    if _strict:
        raise RuntimeError(f"{name}: {reason} (strict kernel mode: no PyTorch fallback)")
    counts = FALLBACKS.setdefault(name, {})
    counts[reason] = counts.get(reason, 0) + 1
    return False


def _served(name: str, reason: str | None) -> bool:
    """True when the op's own gate found nothing (``reason`` None), else a decline."""
    return True if reason is None else _decline(name, reason)


def _use_kernel(name: str, use_cuda: bool, x: torch.Tensor) -> bool:
    """Whether ``name`` runs on the HIP kernel for this call (reference ops.py:82-89):
    ``use_cuda`` set, the op implemented and not held back, and device tensors."""
    if not use_cuda:
        return False
    implemented, _source = CUDA_KERNELS[name]
    if not implemented or name in NOT_YET_FASTER:
        return False
    if not x.is_cuda:
        return _decline(name, f"use_cuda=True needs device tensors, got {x.device}")
    return True


def cuda_kernel_names() -> list[str]:
    """The ops that currently have a working kernel."""
    return [name for name, (implemented, _) in CUDA_KERNELS.items() if implemented]


def dispatch_report(use_cuda: bool) -> str:
    """One line per op saying which implementation a run would use, then the calls of
    this process that the kernels declined (and so ran on the PyTorch path)."""
    lines = []
    for name, (implemented, source) in CUDA_KERNELS.items():
        if not implemented:
            note = f"no kernel yet — {source}"
        elif name in NOT_YET_FASTER:
            note = f"kernel from {source} is slower: {NOT_YET_FASTER[name]}"
        elif not use_cuda:
            note = f"kernel exists from {source}; use_cuda is off"
        else:
            lines.append(f"  {name:<18} hip     (kernel from {source})")
            continue
        lines.append(f"  {name:<18} torch   ({note})")
    if FALLBACKS:
        lines.append("  declined calls that ran on the PyTorch path:")
        for name, reasons in FALLBACKS.items():
            for reason, count in reasons.items():
                lines.append(f"    {name:<16} x{count}: {reason}")
    return "\n".join(lines)


# ------------------------------------------------------------------------ ops


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
            use_cuda: bool = False) -> torch.Tensor:
    """RMSNorm over the last dimension (also QK-norm). Kernel: ``csrc/elementwise.hip``.
    The kernel needs ``weight`` in x's dtype (reference ops.py:129); PyTorch would
    promote instead, so a mixed call runs the PyTorch path."""
    if _use_kernel("rmsnorm", use_cuda, x) and _served(
            "rmsnorm", _same_dtype_reason(x, weight, "weight")):
        return load_extension().rmsnorm(x, weight, eps)
    return torch_path.rms_norm(x, weight, eps)


def embed_rmsnorm(table: torch.Tensor, ids: torch.Tensor, weight: torch.Tensor,
                  eps: float = 1e-6, use_cuda: bool = False, index: torch.Tensor | None = None,
                  prev: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``(h, rmsnorm(h))`` for ``h`` = the table rows of the tokens (row i's token:
    ``prev[index[i]]`` where ``index`` is given and ``index[i] >= 0``, else ``ids[i]``):
    the token embedding and the first block's input norm (reference
    model/qwen3_paged.py:219,134). Kernel: ``csrc/elementwise.hip``, one launch, bitwise
    the lookup then :func:`rmsnorm`; otherwise the torch lookup and :func:`rmsnorm`."""
    if _use_kernel("rmsnorm", use_cuda, table) and load_extension().embed_rmsnorm_supported(
            table, ids, weight, index, prev):
        return load_extension().embed_rmsnorm(table, ids, weight, eps, index, prev)
    if index is not None:
        ids = torch.where(index >= 0, prev.index_select(0, index.clamp(min=0)), ids)
    h = table.index_select(0, ids)
    return h, rmsnorm(h, weight, eps, use_cuda=use_cuda)


def _same_dtype_reason(x: torch.Tensor, other: torch.Tensor, what: str) -> str | None:
    if other.dtype != x.dtype:
        return f"{what} is {other.dtype} but x is {x.dtype}; the kernel does not promote"
    if not other.is_cuda:
        return f"{what} is on {other.device}"
    return None


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                eps: float = 1e-6, use_cuda: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """``(h, rmsnorm(h))`` for ``h = residual + x``: a block's residual add and the norm
    after it (reference qwen3_paged.py:97-99,111-113 run them as two ops). Kernel:
    ``csrc/elementwise.hip``, one launch, bit for bit the add then ``rmsnorm``; shapes it
    does not take run the two ops."""
    if _use_kernel("rmsnorm", use_cuda, x):
        ext = load_extension()
        if ext.add_rmsnorm_supported(x, residual, weight):
            return ext.add_rmsnorm(x, residual, weight, eps)
    h = residual + x
    return h, rmsnorm(h, weight, eps, use_cuda=use_cuda)


def rope(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         use_cuda: bool = False) -> torch.Tensor:
    """Rotary embedding at explicit positions. Kernel: ``csrc/elementwise.hip``. The
    kernel takes fp32 tables and a head axis (reference ops.py:147)."""
    if _use_kernel("rope", use_cuda, x) and _served("rope", _rope_reason(x, cos, sin)):
        return load_extension().rope(x, positions, cos, sin)
    return torch_path.apply_rope(x, positions, cos, sin)


def _rope_reason(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> str | None:
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        return f"the cos/sin tables are {cos.dtype}/{sin.dtype}, the kernel takes float32"
    if x.dim() < 3:
        return f"x has {x.dim()} dimensions; the kernel needs a head axis"
    return None


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                 k_weight: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                 sin: torch.Tensor, eps: float = 1e-6,
                 use_cuda: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Qwen3's QK-norm then RoPE for ``q`` (T x H_q x D) and ``k`` (T x H_k x D): the
    reference caller's ``rmsnorm`` + ``rope`` on each (qwen3_paged.py:73-78). Kernel:
    ``csrc/elementwise.hip`` (one launch, bitwise equal to the unfused kernels); a head
    dim or dtype mix the fused kernel does not serve runs the unfused ops."""
    if _use_kernel("qk_norm_rope", use_cuda, q):
        ext = load_extension()
        if (ext.qk_norm_rope_supported(q.dtype, q.shape[-1]) and k.dtype == q.dtype
                and q_weight.dtype == q.dtype and k_weight.dtype == q.dtype
                and _rope_reason(q, cos, sin) is None):
            return ext.qk_norm_rope(q, k, q_weight, k_weight, positions, cos, sin, eps)
        q = rope(rmsnorm(q, q_weight, eps, use_cuda).unsqueeze(0), positions, cos, sin,
                 use_cuda).squeeze(0)
        k = rope(rmsnorm(k, k_weight, eps, use_cuda).unsqueeze(0), positions, cos, sin,
                 use_cuda).squeeze(0)
        return q, k
    q = torch_path.apply_rope(torch_path.rms_norm(q, q_weight, eps).unsqueeze(0), positions,
                              cos, sin).squeeze(0)
    k = torch_path.apply_rope(torch_path.rms_norm(k, k_weight, eps).unsqueeze(0), positions,
                              cos, sin).squeeze(0)
    return q, k


def qk_norm_rope_kv_write(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          q_weight: torch.Tensor, k_weight: torch.Tensor, positions: torch.Tensor,
                          cos: torch.Tensor, sin: torch.Tensor, eps: float,
                          key_pool: torch.Tensor, value_pool: torch.Tensor,
                          slot_mapping: torch.Tensor, use_cuda: bool = False) -> torch.Tensor | None:
    """``qk_norm_rope`` plus the KV-pool write of the rotated k and of v (reference
    qwen3_paged.py:73-80 -> block/kv_pool.py:116-155) in one launch, returning the
    rotated q. Kernel: ``csrc/elementwise.hip``. None where it does not serve the call
    (the PyTorch path, an fp8 pool, a head dim the fused kernel does not take): the
    caller then runs ``qk_norm_rope`` and ``kv_write``."""
    if not _use_kernel("qk_norm_rope", use_cuda, q):
        return None
    ext = load_extension()
    if (not ext.qk_norm_rope_supported(q.dtype, q.shape[-1]) or key_pool.dtype != q.dtype
            or value_pool.dtype != q.dtype or v.dtype != q.dtype or k.dtype != q.dtype
            or q_weight.dtype != q.dtype or k_weight.dtype != q.dtype
            or _rope_reason(q, cos, sin) is not None or not key_pool.is_contiguous()
            or not value_pool.is_contiguous() or slot_mapping.dtype != torch.int32):
        return None
    return ext.qk_norm_rope_kv_write(q, k, v, q_weight, k_weight, positions, cos, sin, eps,
                                     key_pool, value_pool, slot_mapping)


def paged_decode_qk_norm_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              q_weight: torch.Tensor, k_weight: torch.Tensor,
                              cos: torch.Tensor, sin: torch.Tensor, eps: float,
                              key_pool: torch.Tensor, value_pool: torch.Tensor,
                              block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor,
                              context_lens: torch.Tensor, seq_lens: torch.Tensor,
                              max_context_len: int, scale: float,
                              use_cuda: bool = False) -> torch.Tensor | None:
    """A decode-only step's ``qk_norm_rope_kv_write`` (positions ``context_lens - 1``,
    slots from the block tables) and ``paged_attention`` in one launch, bitwise the two
    (reference qwen3_paged.py:71-95). Kernel: ``csrc/paged_decode.hip``. q (raw, one
    row per sequence), k and v may be column views of the fused projection's output.
    None where it does not serve the call (the PyTorch path, an fp8 pool, another head
    dim, a batch the planner puts on the grid): the caller then makes the two calls."""
    if not _use_kernel("paged_attention", use_cuda, q):
        return None
    ext = load_extension()
    if (q.dim() != 3 or k.dtype != q.dtype or v.dtype != q.dtype or q_weight.dtype != q.dtype
            or k_weight.dtype != q.dtype or value_pool.dtype != q.dtype
            or _rope_reason(q, cos, sin) is not None or not key_pool.is_contiguous()
            or not value_pool.is_contiguous()
            or not ext.paged_decode_qk_norm_rope_supported(q, key_pool, seq_lens.shape[0])):
        return None
    return ext.paged_decode_qk_norm_rope(q, k, v, q_weight, k_weight, cos, sin, eps, key_pool,
                                         value_pool, block_tables, cu_seqlens_q, context_lens,
                                         seq_lens, int(max_context_len), scale)


def swiglu(gate: torch.Tensor, up: torch.Tensor, use_cuda: bool = False) -> torch.Tensor:
    """``silu(gate) * up``. Kernel: ``csrc/elementwise.hip``; gate and up of one dtype
    (reference ops.py:161)."""
    if _use_kernel("swiglu", use_cuda, gate) and _served(
            "swiglu", _same_dtype_reason(gate, up, "up")):
        return load_extension().swiglu(gate, up)
    return torch_path.silu(gate) * up


def argmax(logits: torch.Tensor, use_cuda: bool = False,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy sampling, ``logits.argmax(dim=-1)`` over ``B x V`` logits (reference
    sampler.py:135-141). Kernel: ``csrc/sampler.hip`` (one pass over each row, torch's
    tie and NaN order); other shapes and dtypes take torch's reduction. ``out`` (int64
    [B]): written in place and returned."""
    if (_use_kernel("argmax", use_cuda, logits) and logits.dim() == 2 and logits.shape[1] > 0
            and logits.stride(1) == 1 and logits.dtype in (torch.float32, torch.float16, torch.bfloat16)
            and (out is None or (out.is_contiguous() and out.dtype == torch.int64))):
        return load_extension().argmax(logits, out)
    if out is None:
        return logits.argmax(dim=-1)
    return torch.argmax(logits, dim=-1, out=out)


@dataclass(frozen=True)
class PackedWeight:
    """A projection weight W (N x K) as the skinny kernels read it: ``packed`` in their
    fragment order (``torch_path.pack_fragments``; None where no kernel serves it), with
    the row-major ``dense`` kept beside it for the BLAS (prefill-sized inputs) and the
    PyTorch path. Made once, when the weights are loaded, by :func:`pack_weight`."""

    dense: torch.Tensor
    packed: torch.Tensor | None

    @property
    def shape(self) -> torch.Size:
        return self.dense.shape


def pack_weight(w: torch.Tensor, use_cuda: bool = False) -> PackedWeight:
    """``w`` with its fragment-order copy for the skinny kernels (``csrc/linear.hip``,
    ``mvllm_linear_pack``) when they serve it; the dense matrix alone otherwise."""
    packed = None
    if _use_kernel("linear", use_cuda, w):
        ext = load_extension()
        if ext.linear_packable(w):
            packed = ext.linear_pack(w)
    return PackedWeight(w, packed)


def _skinny_ext(x: torch.Tensor, w: PackedWeight, n: int, use_cuda: bool):
    """The extension when the skinny kernel serves ``x`` against ``w``, else None."""
    if not _use_kernel("linear", use_cuda, x) or not isinstance(w, PackedWeight) or w.packed is None:
        return None
    ext = load_extension()
    return ext if ext.linear_supported(x, w.packed, n) else None


def _blas(x: torch.Tensor, dense: torch.Tensor, use_cuda: bool) -> torch.Tensor | None:
    """``x @ dense.T`` through the library's hipBLASLt entry (``csrc/blas.hip``: the
    vendor product with its descriptors and algorithm kept per shape, where torch makes
    them on every call: ~18.5 us of host time a call, more than the GPU time of a
    prefill chunk's projection) when it is dispatched and serves the operands (device
    fp16/bf16, 2-D contiguous), else None: the caller takes torch's product."""
    if "blas_linear" in NOT_YET_FASTER or not (use_cuda and x.is_cuda and x.dim() == 2):
        return None
    ext = load_extension()
    return ext.blas_linear(x, dense) if ext.blas_linear_supported(x, dense) else None


def _prefill_product(x: torch.Tensor, dense: torch.Tensor, use_cuda: bool) -> torch.Tensor:
    """``x @ dense.T`` for a prefill-sized ``x``: the vendor BLAS (the library's entry,
    else torch's)."""
    y = _blas(x, dense, use_cuda)
    return y if y is not None else x @ dense.t()


def linear(x: torch.Tensor, w: torch.Tensor | PackedWeight, use_cuda: bool = False) -> torch.Tensor:
    """``x @ w.T`` (no bias), the projections of model/basics.py ``linear``.

    Kernels: ``csrc/linear.hip`` for decode-sized ``x`` (at most 64 rows of f16/bf16, K a
    multiple of 64) against a :class:`PackedWeight`: a weight-bandwidth-bound skinny
    GEMM. Larger ``x`` (prefill chunks) and other shapes take the vendor BLAS, as every
    projection does in the reference: for device fp16/bf16 through ``csrc/blas.hip``
    (hipBLASLt with the per-shape set-up kept and the fastest candidate algorithm),
    else through torch - a dispatch by size, all paths on the device.
    """
    dense = w.dense if isinstance(w, PackedWeight) else w
    ext = _skinny_ext(x, w, dense.shape[0], use_cuda)
    if ext is not None:
        return ext.linear(x, w.packed, dense.shape[0])
    if not skinny(x, use_cuda):
        return _prefill_product(x, dense, use_cuda)
    return x @ dense.t()


def skinny(x: torch.Tensor, use_cuda: bool) -> bool:
    """Whether the projections of ``x`` (decode-sized: at most 64 rows) run on the
    skinny projection kernels, fused with their neighbours (``linear_split``,
    ``linear_residual``, ``linear_swiglu``)."""
    if not _use_kernel("linear", use_cuda, x):
        return False
    return (x.dim() == 2 and 1 <= x.shape[0] <= 64 and x.dtype in (torch.float16, torch.bfloat16)
            and x.shape[1] % 64 == 0 and x.shape[1] <= 65536)


def linear_split(x: torch.Tensor, w: PackedWeight, sizes: tuple[int, ...],
                 use_cuda: bool = False, views: bool = False) -> tuple[torch.Tensor, ...]:
    """``x @ w.T`` cut column-wise into contiguous tensors of ``sizes`` (the q, k, v
    projections over their concatenated weights). Kernel: ``csrc/linear.hip``. With
    ``views`` the BLAS path (prefill-sized inputs) returns column views of its one
    output instead of copies, for a consumer that reads strided tokens."""
    ext = _skinny_ext(x, w, w.shape[0], use_cuda)
    if ext is not None and len(sizes) <= 3 and all(s % 32 == 0 for s in sizes[:-1]):
        return ext.linear_split(x, w.packed, tuple(sizes))
    y = x @ w.dense.t() if skinny(x, use_cuda) else _prefill_product(x, w.dense, use_cuda)
    parts = y.split(list(sizes), dim=-1)
    return parts if views else tuple(t.contiguous() for t in parts)


def linear_residual(x: torch.Tensor, w: PackedWeight, residual: torch.Tensor,
                    use_cuda: bool = False) -> torch.Tensor:
    """``residual + x @ w.T``, the projection and the add each rounded as torch rounds
    them. Kernel: ``csrc/linear.hip``."""
    ext = _skinny_ext(x, w, w.shape[0], use_cuda)
    if ext is not None and residual.is_contiguous() and residual.dtype == x.dtype:
        return ext.linear_residual(x, w.packed, residual)
    return residual + linear(x, w.dense, use_cuda=use_cuda)


def linear_residual_rmsnorm(x: torch.Tensor, w: PackedWeight, residual: torch.Tensor,
                            norm_weight: torch.Tensor, eps: float = 1e-6,
                            use_cuda: bool = False) -> tuple[torch.Tensor, torch.Tensor] | None:
    """(h, rmsnorm(h)) for h = residual + x @ w.T, bit for bit ``linear_residual`` then
    ``rmsnorm``, in two launches (``csrc/linear.hip``: split partial sums, then a row
    reduction that adds the residual and normalises). None where the kernel does not
    serve the shape (K <= 1024, N not a multiple of 512, ...): the caller runs the two
    ops. Not dispatched on the PyTorch path either (None)."""
    ext = _skinny_ext(x, w, w.shape[0], use_cuda)
    if (ext is None or not ext.linear_residual_rmsnorm_supported(x, w.shape[0])
            or not residual.is_contiguous() or residual.dtype != x.dtype
            or norm_weight.dtype != x.dtype or not norm_weight.is_contiguous()):
        return None
    return ext.linear_residual_rmsnorm(x, w.packed, residual, norm_weight, eps)


def linear_swiglu(x: torch.Tensor, w_gate_up: PackedWeight, use_cuda: bool = False) -> torch.Tensor:
    """``swiglu(x @ gate.T, x @ up.T)`` over ``torch_path.interleave_gate_up(gate, up)``.
    Kernel: ``csrc/linear.hip``."""
    n = w_gate_up.shape[0]
    ext = _skinny_ext(x, w_gate_up, n, use_cuda)
    if ext is not None and n % 32 == 0:
        return ext.linear_swiglu(x, w_gate_up.packed, n // 2)
    y = linear(x, w_gate_up.dense, use_cuda=use_cuda)
    if _use_kernel("swiglu", use_cuda, y) and y.dim() == 2 and n % 32 == 0:
        # prefill-sized: SwiGLU straight off the interleaved product, no gate/up copies
        return load_extension().swiglu_interleaved(y)
    gate, up = torch_path.split_gate_up(y)
    return swiglu(gate, up, use_cuda=use_cuda)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              mask: torch.Tensor | str | None = None, use_cuda: bool = False) -> torch.Tensor:
    """Dense-cache grouped attention ``B x H x L x D`` (reference ops.py:166-197).

    ``L == 1`` is decode (every cached key visible), ``L > 1`` prefill. Kernels:
    ``decode_attention`` / ``flash_prefill`` of the extension (``csrc/dense.hip``: the
    paged decode and MFMA prefill kernels over virtual 16-position pages of the cache,
    read through its strides). They bake the causal structure in, so they serve decode
    with ``mask`` None or "causal" and prefill with "causal" only (reference
    ``_kernel_can_attend``, ops.py:278-305); an explicit mask tensor, fp64, or a shape
    or stride layout the library refuses goes to the PyTorch path below.
    """
    is_decode = q.shape[-2] == 1
    name = "decode_attention" if is_decode else "flash_prefill"
    if _use_kernel(name, use_cuda, q) and _served(name, None if _kernel_can_attend(
            q, k, v, mask, is_decode) else "a mask, dtype mix or layout the kernel does not bake in"):
        ext = load_extension()
        if _served(name, None if ext.dense_supported(q, k, v) else
                   "a head dim or cache stride layout the library does not take"):
            scale = 1.0 / math.sqrt(q.shape[-1])
            return getattr(ext, name)(q, k, v, scale)
    b, hq, L, d = q.shape
    hk, S = k.shape[1], k.shape[2]
    g = hq // hk
    qs = q.reshape(b, hk, g, L, d)
    scores = (qs @ k.unsqueeze(2).transpose(-2, -1).contiguous()) / math.sqrt(d)
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"unknown mask shorthand {mask!r}, expected 'causal'")
        rows = torch.arange(L, device=q.device).unsqueeze(1)
        cols = torch.arange(S, device=q.device).unsqueeze(0)
        mask = torch.zeros(L, S, dtype=scores.dtype, device=q.device).masked_fill(
            cols > rows + (S - L), float("-inf"))
    if mask is not None:
        scores = scores + mask
    return (torch_path.softmax(scores, dim=-1) @ v.unsqueeze(2)).reshape(b, hq, L, d)


def _kernel_can_attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       mask: torch.Tensor | str | None, is_decode: bool) -> bool:
    """Whether the dense kernels may serve this call (reference ops.py:278-305): the
    mask must be one they bake in, the dtypes shared and not fp64, S >= L, and the head
    dimension contiguous."""
    causal = isinstance(mask, str) and mask == "causal"
    if is_decode:
        if mask is not None and not causal:
            return False
    elif not causal:
        return False
    if q.dim() != 4 or q.dtype != k.dtype or q.dtype != v.dtype or q.dtype == torch.float64:
        return False
    if k.shape[-2] < q.shape[-2]:
        return False
    return k.shape[-2] > 0 and q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1


def paged_attention(
    q: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    context_lens: torch.Tensor,
    seq_lens: torch.Tensor,
    max_query_len: int,
    max_context_len: int,
    scale: float | None = None,
    use_cuda: bool = False,
    *,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """Ragged attention over a paged cache. Kernels: ``csrc/paged_{decode,prefill}.hip``.

    ::

        q:    T x H_q x D              every scheduled token, sequences concatenated
        pools num_blocks x P x H_k x D
        out:  T x H_q x D

    ``max_query_len``/``max_context_len`` are host integers (they size the grid without
    a device read). ``k_scale``/``v_scale`` (``num_blocks x H_k`` fp32, keyword-only)
    accompany a ``float8_e4m3fn`` pool: element = stored value x scale of its
    (page, kv head).
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if _use_kernel("paged_attention", use_cuda, q) and _served(
            "paged_attention", _kernel_can_page(q, key_pool, value_pool, block_tables,
                                                (cu_seqlens_q, context_lens, seq_lens))):
        return load_extension().paged_attention(
            q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, seq_lens,
            int(max_query_len), int(max_context_len), scale, k_scale, v_scale,
        )
    return torch_path.paged_attention_gathered(
        q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, scale,
        k_scale=k_scale, v_scale=v_scale,
    )


def _kernel_can_page(q: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                     block_tables: torch.Tensor, metadata: tuple[torch.Tensor, ...] = ()) -> str | None:
    """Why the paged kernels cannot serve this call, or None when they can: the
    reference's ``_kernel_can_page`` (ops.py:257-275) with this library's head-dim set
    (32, 64, 128, 256 where the reference takes any D <= 256) and float8 pools."""
    if q.dim() != 3:
        return f"q is {list(q.shape)}, not T x H_q x D"
    if q.dtype == torch.float64:
        return "float64 is not supported; the accumulators here are fp32"
    fp8 = key_pool.dtype == torch.float8_e4m3fn and value_pool.dtype == torch.float8_e4m3fn
    if not fp8 and (key_pool.dtype != q.dtype or value_pool.dtype != q.dtype):
        return f"q ({q.dtype}) and the pools ({key_pool.dtype}, {value_pool.dtype}) must share a dtype"
    if q.shape[-1] not in PAGED_HEAD_DIMS:
        return (f"head dim {q.shape[-1]} is not served; this build takes "
                f"{', '.join(map(str, PAGED_HEAD_DIMS))}")
    if not (q.is_contiguous() and key_pool.is_contiguous() and value_pool.is_contiguous()):
        return "q and the pools must be contiguous; the kernel walks them by slot arithmetic"
    if block_tables.dtype != torch.int32 or not block_tables.is_contiguous():
        return "block_tables must be contiguous int32"
    if any(t.dtype != torch.int32 for t in metadata):
        return "cu_seqlens_q, context_lens and seq_lens must be int32"
    if not all(t.is_cuda for t in (key_pool, value_pool, block_tables, *metadata)):
        return "the pools and the metadata must be device tensors"
    return None


def kv_write(key_pool: torch.Tensor, value_pool: torch.Tensor, key: torch.Tensor,
             value: torch.Tensor, slot_mapping: torch.Tensor, use_cuda: bool = False, *,
             k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
    """Scatter ``T x H_k x D`` keys/values into one layer's ``num_blocks x P x H_k x D``
    pools at ``slot_mapping`` (int32, flat slot = block x P + offset; negative = skip).
    Kernel: ``csrc/kv_write.hip``, K and V in one launch. A ``float8_e4m3fn`` pool is
    quantised with per-(block, kv head) scales ``k_scale``/``v_scale`` updated in place
    (policy: include/minivllm_hip.h)."""
    if _use_kernel("kv_write", use_cuda, key) and _served("kv_write", _kv_write_reason(
            key_pool, value_pool, key, value, slot_mapping)):
        load_extension().kv_write(key_pool, value_pool, key, value, slot_mapping,
                                  k_scale=k_scale, v_scale=v_scale)
        return
    torch_path.kv_write(key_pool, value_pool, key, value, slot_mapping,
                        k_scale=k_scale, v_scale=v_scale)


def _kv_write_reason(key_pool: torch.Tensor, value_pool: torch.Tensor, key: torch.Tensor,
                     value: torch.Tensor, slot_mapping: torch.Tensor) -> str | None:
    if not (key_pool.is_cuda and value_pool.is_cuda and value.is_cuda and slot_mapping.is_cuda):
        return "the pools, values and slot_mapping must be device tensors"
    if not (key_pool.is_contiguous() and value_pool.is_contiguous()):
        return "the pools must be contiguous"
    if slot_mapping.dtype != torch.int32:
        return f"slot_mapping is {slot_mapping.dtype}, the kernel takes int32"
    if key.dtype in (torch.float64, torch.float8_e4m3fn) or key.dtype != value.dtype:
        return f"keys/values of {key.dtype}/{value.dtype} are not served"
    if key_pool.dtype != key.dtype and key_pool.dtype != torch.float8_e4m3fn:
        return f"a {key_pool.dtype} pool with {key.dtype} keys is not served"
    return None
