"""A decode step's attention merged straight into the o projection
(``mvllm_paged_attention_o_proj``, ``ops.paged_attention_o_proj``) on the MI355X.

The fused path must give what the two ops it replaces give: ``paged_attention`` (its
output checked against the CPU oracle elsewhere) followed by ``linear_residual_rmsnorm``
(h = residual + attn @ W_o.T, then RMSNorm). The attention output it merges is the one
``paged_attention`` stores (same piece order, same rounding), so the only difference is
the projection's summation order (per head rather than per 256 elements). h is two
roundings (the product, then the residual add): it must agree with the two ops and with
float64 math on ``paged_attention``'s output within two ulps of its operands' size;
normed within the carried difference of h plus its own roundings."""

from __future__ import annotations

import pytest
import torch

from mini_vllm.kernels import ops
from mini_vllm.workloads import build_batch

pytestmark = pytest.mark.gpu


def _eps(t: torch.Tensor) -> float:
    return 2.0**-7 if t.dtype == torch.bfloat16 else 2.0**-10


def _check_h(got: torch.Tensor, want: torch.Tensor, residual: torch.Tensor, proj: torch.Tensor,
             ulps: float = 2.0) -> None:
    """h = T(residual + T(proj)): two roundings, each at most one ulp of its operands'
    size, so |got - want| <= ulps x eps x (|residual| + |proj|) elementwise (where the
    two nearly cancel the result's own ulp is far smaller than either rounding)."""
    bound = ulps * _eps(got) * (residual.float().abs() + proj.float().abs()) + 2.0**-100
    err = (got.float() - want.float()).abs()
    assert (err <= bound).all(), f"h off by {(err / bound).max().item():.2f} of the bound"


def _check_normed(got: torch.Tensor, want: torch.Tensor, h_got: torch.Tensor,
                  h_want: torch.Tensor, norm_w: torch.Tensor, ulps: float = 3.0) -> None:
    """normed = T(T(h x inv) x w): a difference in h carries over scaled by inv |w|, plus
    the two roundings of normed itself."""
    inv = torch.rsqrt(h_want.float().pow(2).mean(-1, keepdim=True) + 1e-6)
    carried = (h_got.float() - h_want.float()).abs() * inv * norm_w.float().abs()
    bound = carried * 1.01 + ulps * _eps(got) * torch.maximum(got.float().abs(), want.float().abs())
    err = (got.float() - want.float()).abs()
    assert (err <= bound + 2.0**-100).all(), f"normed off by {(err / (bound + 1e-30)).max().item():.2f}"


def _case(device, rows, n, kv_dtype=None, dtype=torch.bfloat16, seed=0):
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, 3000, (rows,), generator=gen).tolist()
    b = build_batch(ctx, [1] * rows, dtype=dtype, kv_dtype=kv_dtype, num_q_heads=16,
                    num_kv_heads=8, head_dim=128, seed=seed, device=device)
    w = (torch.randn(n, 16 * 128, generator=gen) * 0.02).to(dtype).to(device)
    h = torch.randn(rows, n, generator=gen).to(dtype).to(device)
    norm_w = (torch.rand(n, generator=gen) + 0.5).to(dtype).to(device)
    return b, ops.pack_weight(w, use_cuda=True), h, norm_w


def _fused(ext, b, wp, h, norm_w, eps=1e-6):
    out = ext.paged_attention_o_proj(b.q, b.key_pool, b.value_pool, b.block_tables,
                                     b.cu_seqlens_q, b.context_lens, b.seq_lens,
                                     b.max_context_len, b.scale, wp.packed, h, norm_w, eps,
                                     b.k_scale, b.v_scale)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("rows", [1, 7, 32, 33, 64])
@pytest.mark.parametrize("n", [512, 1024, 2048])
def test_fused_equals_attention_then_projection(extension, device, rows, n):
    b, wp, h, norm_w = _case(device, rows, n, seed=rows + n)
    h1, n1 = _fused(extension, b, wp, h, norm_w)
    attn = extension.paged_attention(*b.args()).view(rows, -1)
    h2, n2 = extension.linear_residual_rmsnorm(attn, wp.packed, h, norm_w, 1e-6)
    torch.cuda.synchronize()
    proj = attn.double() @ wp.dense.double().T  # float64: the exact product to ~1e-16
    _check_h(h1, h2, h, proj)
    _check_normed(n1, n2, h1, h2, norm_w)
    # h against float64 math on paged_attention's output: one rounding of the product,
    # one of the residual add
    want = (h.double() + proj.to(h.dtype).double()).to(h.dtype)
    _check_h(h1, want, h, proj)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_fused_over_fp8_and_16_bit_pools_and_repeated_calls(extension, device, kv_dtype):
    """fp8 pools (scales applied in the decode) and three calls in a row on the same
    workspace give the same bits (the merge order is fixed)."""
    b, wp, h, norm_w = _case(device, 32, 1024, kv_dtype=kv_dtype, seed=3)
    first = _fused(extension, b, wp, h, norm_w)
    for _ in range(2):
        again = _fused(extension, b, wp, h, norm_w)
        assert torch.equal(again[0], first[0]) and torch.equal(again[1], first[1])
    attn = extension.paged_attention(*b.args(), k_scale=b.k_scale, v_scale=b.v_scale).view(32, -1)
    h2, n2 = extension.linear_residual_rmsnorm(attn, wp.packed, h, norm_w, 1e-6)
    torch.cuda.synchronize()
    proj = attn.double() @ wp.dense.double().T
    _check_h(first[0], h2, h, proj)
    _check_normed(first[1], n2, first[0], h2, norm_w)


def test_fused_float16(extension, device):
    b, wp, h, norm_w = _case(device, 16, 1024, dtype=torch.float16, seed=5)
    h1, n1 = _fused(extension, b, wp, h, norm_w)
    attn = extension.paged_attention(*b.args()).view(16, -1)
    h2, n2 = extension.linear_residual_rmsnorm(attn, wp.packed, h, norm_w, 1e-6)
    torch.cuda.synchronize()
    proj = attn.double() @ wp.dense.double().T
    _check_h(h1, h2, h, proj)
    _check_normed(n1, n2, h1, h2, norm_w)


def test_the_op_declines_what_it_does_not_serve(extension, device):
    """A prefill row, more than 64 rows or head dim 64: ops returns None (the caller runs
    the two ops); the binding raises before any launch. While the fused path is held
    back (``ops.NOT_YET_FASTER``: measured no faster) ops returns None for every call."""
    b, wp, h, norm_w = _case(device, 4, 1024, seed=7)
    args = (b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q, b.context_lens,
            b.seq_lens, b.max_context_len, b.scale, wp, h, norm_w)
    served = ops.paged_attention_o_proj(*args, use_cuda=True)
    assert (served is None) == ("paged_attention_o_proj" in ops.NOT_YET_FASTER)
    mixed = build_batch([100, 40], [1, 8], dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8,
                        head_dim=128, seed=8, device=device)
    h9 = torch.zeros(9, 1024, dtype=torch.bfloat16, device=device)
    assert ops.paged_attention_o_proj(
        mixed.q, mixed.key_pool, mixed.value_pool, mixed.block_tables, mixed.cu_seqlens_q,
        mixed.context_lens, mixed.seq_lens, mixed.max_context_len, mixed.scale, wp, h9, norm_w,
        use_cuda=True) is None
    with pytest.raises(RuntimeError, match="one decode row"):
        extension.paged_attention_o_proj(
            mixed.q, mixed.key_pool, mixed.value_pool, mixed.block_tables, mixed.cu_seqlens_q,
            mixed.context_lens, mixed.seq_lens, mixed.max_context_len, mixed.scale, wp.packed, h9,
            norm_w, 1e-6)
    small = build_batch([50, 60], [1, 1], dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8,
                        head_dim=64, seed=9, device=device)
    h2 = torch.zeros(2, 1024, dtype=torch.bfloat16, device=device)
    w64 = ops.pack_weight(torch.zeros(1024, 16 * 64, dtype=torch.bfloat16, device=device),
                          use_cuda=True)
    assert ops.paged_attention_o_proj(
        small.q, small.key_pool, small.value_pool, small.block_tables, small.cu_seqlens_q,
        small.context_lens, small.seq_lens, small.max_context_len, small.scale, w64, h2, norm_w,
        use_cuda=True) is None
