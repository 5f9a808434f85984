"""Skinny projection kernel (``ops.linear`` / ``mvllm_linear``) on the MI355X (``-m gpu``).

The reference computes projections with ``x @ w.T`` through the vendor BLAS
(model/basics.py ``linear``); the kernel must return the same function. Both sum in
fp32 and round once, in different orders, so the bar is: every element within one
unit in the last place (of the output dtype) of the fp32 product ``x.float() @
w.float().T`` rounded to that dtype, plus the spread of two fp32 summation orders
(4 sqrt(K) 2^-24 sum_k |x_k w_k|, which only matters where the sum cancels to near
zero), and within two ulps of torch's own result.
"""

from __future__ import annotations

import pytest
import torch

from mini_vllm import torch_path
from mini_vllm.kernels import ops

pytestmark = pytest.mark.gpu


def _ulp(ref: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One unit in the last place of each element of ``ref`` (fp32) in ``dtype``."""
    mant = {torch.bfloat16: 7, torch.float16: 10}[dtype]
    mag = ref.abs().clamp_min(torch.finfo(dtype).tiny)
    return torch.exp2(torch.floor(torch.log2(mag)) - mant)


def _check(extension, m, n, k, dtype, seed=0):
    gen = torch.Generator(device="cpu").manual_seed(seed + 131 * m + 7 * n + k)
    x = torch.randn(m, k, generator=gen).to(dtype).cuda()
    w = (torch.randn(n, k, generator=gen) * 0.05).to(dtype).cuda()
    got = extension.linear(x, w)
    torch.cuda.synchronize()
    ref32 = x.float() @ w.float().t()
    ulp = _ulp(ref32, dtype)
    spread = 4 * k ** 0.5 * 2.0 ** -24 * (x.float().abs() @ w.float().abs().t())
    tol = ulp * 1.0001 + spread
    err = (got.float() - ref32.to(dtype).float()).abs()
    assert (err <= tol).all(), f"M={m} N={n} K={k}: {int((err > tol).sum())} elements off by > 1 ulp"
    blas = x @ w.t()
    assert ((got.float() - blas.float()).abs() <= 2 * ulp * 1.0001 + spread).all()
    return got


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 7, 32, 33, 64])
def test_rows_up_to_64(extension, device, m, dtype):
    _check(extension, m, 1000, 1024, dtype)


@pytest.mark.parametrize("n,k", [(1, 64), (31, 128), (32, 3072), (33, 2048), (4096, 1024),
                                 (6144, 1024), (1024, 3072)])
def test_shapes_of_the_model(extension, device, n, k):
    """Column counts on and off the 32-column tile, K of every projection of the
    Qwen3-0.6B shape (1024, 2048, 3072) and the smallest served."""
    _check(extension, 32, n, k, torch.bfloat16)


def test_lm_head_shape(extension, device):
    """The tied-embedding logits projection: N = 151936, K = 1024."""
    _check(extension, 17, 151936, 1024, torch.bfloat16)


def test_ops_dispatch_by_size(extension, device):
    """``ops.linear`` takes the kernel for at most 64 rows and the BLAS above, and the
    extension refuses what the kernel does not serve."""
    x = torch.randn(65, 256, dtype=torch.bfloat16, device="cuda")
    w = torch.randn(48, 256, dtype=torch.bfloat16, device="cuda")
    assert not extension.linear_supported(x, w)
    torch.testing.assert_close(ops.linear(x, w, use_cuda=True), x @ w.t())
    with pytest.raises(RuntimeError, match="skinny kernel"):
        extension.linear(x, w)
    x = torch.randn(4, 96, dtype=torch.bfloat16, device="cuda")  # K not a multiple of 64
    w = torch.randn(48, 96, dtype=torch.bfloat16, device="cuda")
    assert not extension.linear_supported(x, w)
    torch.testing.assert_close(ops.linear(x, w, use_cuda=True), x @ w.t())
    x = torch.randn(4, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.randn(48, 128, dtype=torch.bfloat16, device="cuda")
    assert extension.linear_supported(x, w)
    got = ops.linear(x, w, use_cuda=True)
    assert got.shape == (4, 48) and got.dtype == torch.bfloat16


def test_known_answer_identity(extension, device):
    """x @ I = x exactly (each output is one product of an element and 1)."""
    x = torch.randn(9, 128, dtype=torch.bfloat16, device="cuda")
    eye = torch.eye(128, dtype=torch.bfloat16, device="cuda")
    assert torch.equal(extension.linear(x, eye), x)


def _operands(m, n, k, dtype, seed):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(m, k, generator=gen).to(dtype).cuda()
    w = (torch.randn(n, k, generator=gen) * 0.05).to(dtype).cuda()
    return x, w, gen


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 20, 64])
def test_split_equals_separate_projections(extension, device, m, dtype):
    """q/k/v over the concatenated weights, bitwise the three separate projections
    (each column's sum is formed the same way wherever its tile lies)."""
    x, wq, gen = _operands(m, 2048, 1024, dtype, 11 + m)
    wk = (torch.randn(1024, 1024, generator=gen) * 0.05).to(dtype).cuda()
    wv = (torch.randn(1000, 1024, generator=gen) * 0.05).to(dtype).cuda()
    q, k, v = extension.linear_split(x, torch.cat((wq, wk, wv)), (2048, 1024, 1000))
    for got, w in ((q, wq), (k, wk), (v, wv)):
        assert got.is_contiguous() and torch.equal(got, extension.linear(x, w))
    a, b = extension.linear_split(x, torch.cat((wq, wk)), (2048, 1024))
    assert torch.equal(a, q) and torch.equal(b, k)
    with pytest.raises(RuntimeError, match="multiples of 32"):
        extension.linear_split(x, torch.cat((wq, wk)), (2040, 1032))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(1, 1024, 2048), (37, 1024, 3072), (64, 1000, 64)])
def test_residual_equals_add_after_projection(extension, device, m, n, k, dtype):
    """residual + x w^T in one launch, bitwise torch's add of the rounded projection."""
    x, w, gen = _operands(m, n, k, dtype, 23 + m)
    r = torch.randn(m, n, generator=gen).to(dtype).cuda()
    got = extension.linear_residual(x, w, r)
    assert torch.equal(got, r + extension.linear(x, w))
    assert torch.equal(ops.linear_residual(x, w, r, use_cuda=True), got)
    with pytest.raises(RuntimeError, match="residual"):
        extension.linear_residual(x, w, r[:, :-1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,i", [(1, 3072), (48, 3072), (5, 48)])
def test_swiglu_equals_gate_up_then_swiglu(extension, device, m, i, dtype):
    """gate/up + SwiGLU in one launch over the 16-row interleave, bitwise the two
    projections followed by the SwiGLU kernel."""
    x, gate, gen = _operands(m, i, 1024, dtype, 37 + m)
    up = (torch.randn(i, 1024, generator=gen) * 0.05).to(dtype).cuda()
    wgu = torch_path.interleave_gate_up(gate, up)
    got = extension.linear_swiglu(x, wgu)
    want = ops.swiglu(extension.linear(x, gate), extension.linear(x, up), use_cuda=True)
    assert got.shape == (m, i) and torch.equal(got, want)
    assert torch.equal(ops.linear_swiglu(x, wgu, use_cuda=True), got)
