"""The seam between the model and its kernels (reference mini_vllm/kernels/ops.py).

Same op names, signatures and ``use_cuda`` switch as the reference, so the model,
engine and tests above it run unchanged:

    rmsnorm(x, weight, eps=1e-6, use_cuda=False)                       ops.py:117-131
    rope(x, positions, cos, sin, use_cuda=False)                       ops.py:134-149
    swiglu(gate, up, use_cuda=False)                                   ops.py:152-163
    paged_attention(q, key_pool, value_pool, block_tables, cu_seqlens_q,
                    context_lens, seq_lens, max_query_len, max_context_len,
                    scale=None, use_cuda=False)                        ops.py:200-254

plus two ops that fuse what the reference's caller does in several calls:

    kv_write(key_pool, value_pool, key, value, slot_mapping, use_cuda=False,
             *, k_scale=None, v_scale=None)    PagedKvPool.write: kv_pool.py:116-155
    qk_norm_rope(q, k, q_weight, k_weight, positions, cos, sin, eps=1e-6,
                 use_cuda=False)               qwen3_paged.py:73-78 (2 rmsnorm + 2 rope)

The callee behind ``use_cuda=True`` is ``libminivllm_hip.so`` (HIP for gfx950).

One deliberate difference: ``use_cuda=True`` never falls back. The reference routes a
call its kernel cannot serve (CPU tensors, a non-contiguous pool, int64 tables ...)
silently to the PyTorch path; here such a call raises ``RuntimeError`` naming the
reason, because a silent fallback is exactly how a kernel that never ran ends up in
a benchmark. ``use_cuda=False`` selects the PyTorch path (:mod:`mini_vllm.torch_path`)
explicitly, as in the reference. Ops that have no kernel in this library yet
(``attention``, the dense-cache decode/prefill) follow the reference's rule for
unimplemented kernels and use the PyTorch path, which :func:`dispatch_report` states.
"""

from __future__ import annotations

import math
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
    "kv_write",
    "PackedWeight",
    "linear",
    "linear_residual",
    "linear_residual_rmsnorm",
    "linear_split",
    "linear_swiglu",
    "pack_weight",
    "paged_attention",
    "qk_norm_rope",
    "qk_norm_rope_kv_write",
    "rmsnorm",
    "rope",
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
}

# Kernels that exist but are deliberately not dispatched, with the reason.
NOT_YET_FASTER: dict[str, str] = {}

MAX_PAGED_HEAD_DIM = 256
PAGED_HEAD_DIMS = (32, 64, 128, 256)


def _use_kernel(name: str, use_cuda: bool, x: torch.Tensor) -> bool:
    """Whether ``name`` runs on the HIP kernel; raises instead of falling back."""
    if not use_cuda:
        return False
    implemented, _source = CUDA_KERNELS[name]
    if not implemented or name in NOT_YET_FASTER:
        return False
    if not x.is_cuda:
        raise RuntimeError(
            f"{name}: use_cuda=True needs device tensors, got {x.device}; pass use_cuda=False "
            "to run the PyTorch path"
        )
    return True


def cuda_kernel_names() -> list[str]:
    """The ops that currently have a working kernel."""
    return [name for name, (implemented, _) in CUDA_KERNELS.items() if implemented]


def dispatch_report(use_cuda: bool) -> str:
    """One line per op saying which implementation a run would use."""
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
    return "\n".join(lines)


# ------------------------------------------------------------------------ ops


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
            use_cuda: bool = False) -> torch.Tensor:
    """RMSNorm over the last dimension (also QK-norm). Kernel: ``csrc/elementwise.hip``."""
    if _use_kernel("rmsnorm", use_cuda, x):
        return load_extension().rmsnorm(x, weight, eps)
    return torch_path.rms_norm(x, weight, eps)


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
    """Rotary embedding at explicit positions. Kernel: ``csrc/elementwise.hip``."""
    if _use_kernel("rope", use_cuda, x):
        return load_extension().rope(x, positions, cos, sin)
    return torch_path.apply_rope(x, positions, cos, sin)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                 k_weight: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                 sin: torch.Tensor, eps: float = 1e-6,
                 use_cuda: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Qwen3's QK-norm then RoPE for ``q`` (T x H_q x D) and ``k`` (T x H_k x D): the
    reference caller's ``rmsnorm`` + ``rope`` on each (qwen3_paged.py:73-78). Kernel:
    ``csrc/elementwise.hip`` (one launch, bitwise equal to the unfused kernels); a head
    dim the fused kernel does not serve runs the unfused kernels."""
    if _use_kernel("qk_norm_rope", use_cuda, q):
        ext = load_extension()
        if ext.qk_norm_rope_supported(q.dtype, q.shape[-1]):
            return ext.qk_norm_rope(q, k, q_weight, k_weight, positions, cos, sin, eps)
        q = ext.rope(ext.rmsnorm(q, q_weight, eps).unsqueeze(0), positions, cos, sin).squeeze(0)
        k = ext.rope(ext.rmsnorm(k, k_weight, eps).unsqueeze(0), positions, cos, sin).squeeze(0)
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
            or value_pool.dtype != q.dtype or v.dtype != q.dtype):
        return None
    return ext.qk_norm_rope_kv_write(q, k, v, q_weight, k_weight, positions, cos, sin, eps,
                                     key_pool, value_pool, slot_mapping)


def swiglu(gate: torch.Tensor, up: torch.Tensor, use_cuda: bool = False) -> torch.Tensor:
    """``silu(gate) * up``. Kernel: ``csrc/elementwise.hip``."""
    if _use_kernel("swiglu", use_cuda, gate):
        return load_extension().swiglu(gate, up)
    return torch_path.silu(gate) * up


def argmax(logits: torch.Tensor, use_cuda: bool = False) -> torch.Tensor:
    """Greedy sampling, ``logits.argmax(dim=-1)`` over ``B x V`` logits (reference
    sampler.py:135-141). Kernel: ``csrc/sampler.hip`` (one pass over each row, torch's
    tie and NaN order); other shapes and dtypes take torch's reduction."""
    if (_use_kernel("argmax", use_cuda, logits) and logits.dim() == 2 and logits.shape[1] > 0
            and logits.stride(1) == 1 and logits.dtype in (torch.float32, torch.float16, torch.bfloat16)):
        return load_extension().argmax(logits)
    return logits.argmax(dim=-1)


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


def linear(x: torch.Tensor, w: torch.Tensor | PackedWeight, use_cuda: bool = False) -> torch.Tensor:
    """``x @ w.T`` (no bias), the projections of model/basics.py ``linear``.

    Kernel: ``csrc/linear.hip`` for decode-sized ``x`` (at most 64 rows of f16/bf16, K a
    multiple of 64) against a :class:`PackedWeight`: a weight-bandwidth-bound skinny
    GEMM. Larger ``x`` (prefill chunks) is a real GEMM and goes to the vendor BLAS
    through torch, as every projection does in the reference; that is a dispatch by
    size, both paths on the device. A plain tensor weight always takes the BLAS.
    """
    dense = w.dense if isinstance(w, PackedWeight) else w
    ext = _skinny_ext(x, w, dense.shape[0], use_cuda)
    if ext is not None:
        return ext.linear(x, w.packed, dense.shape[0])
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
    parts = (x @ w.dense.t()).split(list(sizes), dim=-1)
    return parts if views else tuple(t.contiguous() for t in parts)


def linear_residual(x: torch.Tensor, w: PackedWeight, residual: torch.Tensor,
                    use_cuda: bool = False) -> torch.Tensor:
    """``residual + x @ w.T``, the projection and the add each rounded as torch rounds
    them. Kernel: ``csrc/linear.hip``."""
    ext = _skinny_ext(x, w, w.shape[0], use_cuda)
    if ext is not None and residual.is_contiguous() and residual.dtype == x.dtype:
        return ext.linear_residual(x, w.packed, residual)
    return residual + x @ w.dense.t()


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
    y = x @ w_gate_up.dense.t()
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
    if _use_kernel(name, use_cuda, q) and _kernel_can_attend(q, k, v, mask, is_decode):
        ext = load_extension()
        if ext.dense_supported(q, k, v):
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
    if _use_kernel("paged_attention", use_cuda, q):
        _check_kernel_can_page(q, key_pool, value_pool, block_tables)
        return load_extension().paged_attention(
            q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, seq_lens,
            int(max_query_len), int(max_context_len), scale, k_scale, v_scale,
        )
    return torch_path.paged_attention_gathered(
        q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens, scale,
        k_scale=k_scale, v_scale=v_scale,
    )


def _check_kernel_can_page(q: torch.Tensor, key_pool: torch.Tensor, value_pool: torch.Tensor,
                           block_tables: torch.Tensor) -> None:
    """The reference's ``_kernel_can_page`` gate (ops.py:257-275), raising instead of
    declining, plus this library's head-dim set."""
    if q.dim() != 3:
        raise RuntimeError(f"paged_attention: expected q shaped T x H_q x D, got {list(q.shape)}")
    if q.dtype == torch.float64:
        raise RuntimeError("paged_attention: float64 is not supported; the accumulators here are fp32")
    if q.shape[-1] not in PAGED_HEAD_DIMS:
        raise RuntimeError(
            f"paged_attention: head dim {q.shape[-1]} is not supported; this build serves "
            f"{', '.join(map(str, PAGED_HEAD_DIMS))}"
        )
    if not (q.is_contiguous() and key_pool.is_contiguous() and value_pool.is_contiguous()):
        raise RuntimeError(
            "paged_attention: q and the pools must be contiguous; the kernel walks them by "
            "slot arithmetic rather than by stride"
        )
    if block_tables.dtype != torch.int32:
        raise RuntimeError("paged_attention: the metadata tensors must be int32")
    if not block_tables.is_contiguous():
        raise RuntimeError("paged_attention: block_tables must be contiguous")


def kv_write(key_pool: torch.Tensor, value_pool: torch.Tensor, key: torch.Tensor,
             value: torch.Tensor, slot_mapping: torch.Tensor, use_cuda: bool = False, *,
             k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> None:
    """Scatter ``T x H_k x D`` keys/values into one layer's ``num_blocks x P x H_k x D``
    pools at ``slot_mapping`` (int32, flat slot = block x P + offset; negative = skip).
    Kernel: ``csrc/kv_write.hip``, K and V in one launch. A ``float8_e4m3fn`` pool is
    quantised with per-(block, kv head) scales ``k_scale``/``v_scale`` updated in place
    (policy: include/minivllm_hip.h)."""
    if _use_kernel("kv_write", use_cuda, key):
        load_extension().kv_write(key_pool, value_pool, key, value, slot_mapping,
                                  k_scale=k_scale, v_scale=v_scale)
        return
    torch_path.kv_write(key_pool, value_pool, key, value, slot_mapping,
                        k_scale=k_scale, v_scale=v_scale)
