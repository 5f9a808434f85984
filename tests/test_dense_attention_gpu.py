"""Dense-cache attention kernels (``decode_attention`` / ``flash_prefill`` of the
extension, ``mvllm_dense_attention``, reached through ``ops.attention``) on the MI355X
(``-m gpu``).

The reference serves its dense-cache model with csrc/decode_attention.cu (L = 1: every
cached key visible) and csrc/flash_prefill.cu (L > 1: causal with offset S - L), both
reading K/V through (batch, head, position) strides. Here both run on the paged kernels
over virtual 16-position pages of the cache. Bar: the float64 oracle
(oracle/dense_attention.py, pinned in tests/test_oracle.py) within the attention
tolerances of the paged kernels (max-abs 2e-5 fp32, 1e-2 fp16, 2e-2 bf16).
"""

from __future__ import annotations

import pytest
import torch

from conftest import ATTN_ATOL, assert_max_abs
from mini_vllm.kernels import ops
from oracle.dense_attention import dense_attention as oracle

pytestmark = pytest.mark.gpu


def _qkv(b, hq, hk, L, S, d, dtype, seed, s_max=None):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, L, d, generator=gen).to(dtype).cuda()
    s_max = s_max or S
    k = torch.randn(b, hk, s_max, d, generator=gen).to(dtype).cuda()[:, :, :S]
    v = torch.randn(b, hk, s_max, d, generator=gen).to(dtype).cuda()[:, :, :S]
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,S", [(1, 1), (3, 17), (64, 1000), (2, 4097)])
def test_decode_matches_the_oracle(extension, device, b, S, dtype):
    q, k, v = _qkv(b, 16, 8, 1, S, 128, dtype, seed=b * 7 + S)
    got = extension.decode_attention(q, k, v, 128 ** -0.5)
    assert got.shape == (b, 16, 1, 128) and got.dtype == dtype
    assert_max_abs(got, oracle(q, k, v), ATTN_ATOL[dtype], f"decode B={b} S={S}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hq,hk,d", [(8, 1, 64), (4, 4, 32), (32, 8, 256)])
def test_decode_gqa_groups_and_head_dims(extension, device, hq, hk, d, dtype):
    q, k, v = _qkv(5, hq, hk, 1, 300, d, dtype, seed=hq + d)
    assert_max_abs(extension.decode_attention(q, k, v, d ** -0.5), oracle(q, k, v),
                   ATTN_ATOL[dtype], f"H_q={hq} H_k={hk} D={d}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,L,S", [(1, 2, 2), (2, 37, 37), (3, 64, 200), (2, 512, 1536),
                                   (1, 300, 301)])
def test_prefill_matches_the_oracle(extension, device, b, L, S, dtype):
    q, k, v = _qkv(b, 16, 8, L, S, 128, dtype, seed=b + L + S)
    got = extension.flash_prefill(q, k, v, 128 ** -0.5)
    assert got.shape == (b, 16, L, 128) and got.dtype == dtype
    assert_max_abs(got, oracle(q, k, v), ATTN_ATOL[dtype], f"prefill B={b} L={L} S={S}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_narrowed_cache_is_read_in_place(extension, device, dtype):
    """A cache narrowed out of a larger buffer (the dense model's preallocated cache)
    is read through its strides: batch stride H_k x S_max x D, not H_k x S x D."""
    for L, S in ((1, 333), (48, 333)):
        q, k, v = _qkv(4, 16, 8, L, S, 128, dtype, seed=S + L, s_max=1024)
        assert not k.is_contiguous()
        got = (extension.decode_attention if L == 1 else extension.flash_prefill)(q, k, v, 128 ** -0.5)
        assert_max_abs(got, oracle(q, k, v), ATTN_ATOL[dtype], f"narrowed L={L}")


def test_position_major_cache_layout(extension, device):
    """A cache stored B x S x H_k x D and viewed as B x H_k x S x D (position stride
    H_k D, head stride D)."""
    gen = torch.Generator().manual_seed(9)
    b, hq, hk, S, d = 3, 16, 8, 160, 128
    q = torch.randn(b, hq, 1, d, generator=gen).to(torch.bfloat16).cuda()
    k = torch.randn(b, S, hk, d, generator=gen).to(torch.bfloat16).cuda().transpose(1, 2)
    v = torch.randn(b, S, hk, d, generator=gen).to(torch.bfloat16).cuda().transpose(1, 2)
    assert extension.dense_supported(q, k, v)
    assert_max_abs(extension.decode_attention(q, k, v, d ** -0.5), oracle(q, k, v),
                   ATTN_ATOL[torch.bfloat16], "position-major")


def test_ops_attention_routes_to_the_kernels(extension, device):
    """``ops.attention`` serves decode (mask None or "causal") and causal prefill on the
    kernels, and gives the PyTorch path whatever they cannot serve."""
    q, k, v = _qkv(2, 16, 8, 1, 90, 128, torch.bfloat16, seed=1)
    got = ops.attention(q, k, v, use_cuda=True)
    assert torch.equal(got, extension.decode_attention(q, k, v, 128 ** -0.5))
    assert torch.equal(ops.attention(q, k, v, mask="causal", use_cuda=True), got)
    qp, kp, vp = _qkv(2, 16, 8, 20, 90, 128, torch.bfloat16, seed=2)
    got = ops.attention(qp, kp, vp, mask="causal", use_cuda=True)
    assert torch.equal(got, extension.flash_prefill(qp, kp, vp, 128 ** -0.5))
    assert_max_abs(got, oracle(qp, kp, vp), ATTN_ATOL[torch.bfloat16])
    # head dim 48: not served by the library, the PyTorch path answers
    q48, k48, v48 = _qkv(2, 4, 2, 1, 30, 48, torch.float32, seed=3)
    assert not extension.dense_supported(q48, k48, v48)
    with ops.strict_kernels(False):  # the reference's fallback for what the kernels decline
        assert_max_abs(ops.attention(q48, k48, v48, use_cuda=True), oracle(q48, k48, v48), 1e-5)
    # an explicit mask tensor is never handed to the kernels
    mask = torch.zeros(20, 90, device="cuda")
    mask[:, 50:] = float("-inf")
    want = ops.attention(qp.float(), kp.float(), vp.float(), mask=mask)
    with ops.strict_kernels(False):
        assert_max_abs(ops.attention(qp.float(), kp.float(), vp.float(), mask=mask, use_cuda=True),
                       want, 1e-6)
    with pytest.raises(RuntimeError, match="strict kernel mode"):
        ops.attention(qp.float(), kp.float(), vp.float(), mask=mask, use_cuda=True)


def test_refusals_match_the_reference(extension, device):
    q, k, v = _qkv(2, 16, 8, 3, 10, 128, torch.bfloat16, seed=4)
    with pytest.raises(RuntimeError, match="the L == 1 case"):
        extension.decode_attention(q, k, v, 0.1)
    with pytest.raises(RuntimeError, match="must be a multiple of H_k"):
        extension.flash_prefill(q[:, :12], k[:, :5], v[:, :5], 0.1)
    with pytest.raises(RuntimeError, match="S >= L > 0"):
        extension.flash_prefill(q, k[:, :, :2], v[:, :, :2], 0.1)
    with pytest.raises(RuntimeError, match="must share a dtype"):
        extension.flash_prefill(q, k.float(), v, 0.1)
    with pytest.raises(RuntimeError, match="the cache is empty"):
        extension.decode_attention(q[:, :, :1], k[:, :, :0], v[:, :, :0], 0.1)
    with pytest.raises(RuntimeError, match="head dimension must be contiguous"):
        extension.decode_attention(q[:, :, :1, :64], k[..., ::2], v[..., ::2], 0.1)
