"""Prefill projection GEMM (``csrc/gemm.hip``, ``mvllm_gemm``) on the MI355X (``-m gpu``).

y = x w^T with fp32 accumulation and one rounding, against an fp32 torch reference of
the same product (the tolerance is the output dtype's rounding plus fp32 summation
order) and against torch's own BLAS product in the same dtype.
"""

from __future__ import annotations

import pytest
import torch

from mini_vllm.kernels import ops

pytestmark = pytest.mark.gpu

PROJECTIONS = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072)}


def _check(ext, m, n, k, dtype, seed=0):
    gen = torch.Generator().manual_seed(seed + m + n + k)
    x = torch.randn(m, k, generator=gen).to(dtype).cuda()
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dtype).cuda()
    y = ext.gemm(x, w)
    ref = x.float() @ w.float().t()
    err = (y.float() - ref).abs()
    tol = ref.abs() * (2.0**-8 if dtype == torch.bfloat16 else 2.0**-11) + 1e-4 * k**0.5 * 0.02
    assert bool((err <= tol).all()), f"max err {err.max():.3g} at {divmod(int(err.argmax()), n)}"
    blas = x @ w.t()
    ulp = 2.0**-7 if dtype == torch.bfloat16 else 2.0**-10
    assert bool(((y.float() - blas.float()).abs() <= blas.float().abs() * 2 * ulp + 1e-3).all())
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", list(PROJECTIONS))
@pytest.mark.parametrize("m", [2048, 1000, 130, 1])
def test_prefill_projections_match_fp32(extension, device, name, m, dtype):
    n, k = PROJECTIONS[name]
    _check(extension, m, n, k, dtype)


@pytest.mark.parametrize("m,n,k", [(257, 64, 64), (64, 192, 128), (3000, 128, 4096)])
def test_other_shapes(extension, device, m, n, k):
    _check(extension, m, n, k, torch.bfloat16)


def test_deterministic_and_held_back_from_dispatch(extension, device):
    """Repeated calls give the same bits. While the GEMM is listed in NOT_YET_FASTER
    (slower than the vendor BLAS here), ops.linear keeps prefill projections on the
    BLAS."""
    x = torch.randn(2048, 2048, device=device, dtype=torch.bfloat16)
    w = torch.randn(1024, 2048, device=device, dtype=torch.bfloat16) * 0.02
    first = extension.gemm(x, w)
    assert torch.equal(extension.gemm(x, w), first)
    assert "gemm" in ops.NOT_YET_FASTER
    assert torch.equal(ops.linear(x, w, use_cuda=True), x @ w.t())


def test_refusals(extension, device):
    x = torch.randn(16, 100, device=device, dtype=torch.bfloat16)
    w = torch.randn(64, 100, device=device, dtype=torch.bfloat16)
    assert not extension.gemm_supported(x, w)
    with pytest.raises(RuntimeError, match="not served"):
        extension.gemm(x, w)
    assert not extension.gemm_supported(x.float()[:, :64].contiguous(), w.float()[:, :64].contiguous())
    # ops.linear falls back to the BLAS for shapes the GEMM does not serve
    assert torch.equal(ops.linear(x, w, use_cuda=True), x @ w.t())
