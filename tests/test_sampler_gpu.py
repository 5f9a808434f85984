"""Greedy sampling kernel (``ops.argmax`` / ``mvllm_argmax``) on the MI355X (``-m gpu``).

The reference's greedy rows take ``logits.argmax(dim=-1)`` (mini_vllm/sampler.py:
135-141). Index work is bit-exact: the kernel must return torch's indices, including
its order on ties (first index), signed zeros (equal) and NaN (above every number).
"""

from __future__ import annotations

import pytest
import torch

from mini_vllm.kernels import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,vocab", [(1, 1), (3, 7), (4, 8), (32, 151936), (65, 1000),
                                        (5, 16385), (2, 300001), (1, 1048576)])
def test_matches_torch_argmax(extension, device, rows, vocab, dtype):
    gen = torch.Generator().manual_seed(rows * 31 + vocab)
    logits = torch.randn(rows, vocab, generator=gen).to(dtype).cuda()
    assert torch.equal(extension.argmax(logits), logits.argmax(dim=-1))


def test_ties_signed_zeros_and_nan(extension, device):
    """Equal maxima: the first index; -0 == +0 (the earlier zero wins); NaN beats every
    number and the first NaN wins; -inf rows and a row of one value."""
    x = torch.full((7, 50), -1.0)
    x[0, [5, 9, 40]] = 3.0                      # ties -> 5
    x[1, :] = -0.5
    x[1, 12], x[1, 30] = -0.0, 0.0              # -0 first, then +0: equal -> 12
    x[2, 30], x[2, 12] = -0.0, 0.0              # +0 first at 12 -> 12
    x[3, 44], x[3, 7], x[3, 8] = float("nan"), 1e30, float("nan")  # first NaN -> 8
    x[4, :] = float("-inf")                     # all -inf -> 0
    x[5, 49] = float("inf")                     # inf -> 49
    x[6, :] = 2.5                               # constant -> 0
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        logits = x.to(dtype).cuda()
        got = extension.argmax(logits)
        assert torch.equal(got, logits.argmax(dim=-1)), dtype
        assert got.tolist() == [5, 12, 12, 8, 0, 49, 0]


def test_strided_rows_and_ops_dispatch(extension, device):
    """Rows farther apart than their length (a narrowed logits buffer) and ``ops.argmax``
    routing: the kernel for 2-D f32/f16/bf16 rows, torch otherwise."""
    base = torch.randn(9, 1200, dtype=torch.bfloat16, device="cuda")
    view = base[:, 100:1100]
    assert not view.is_contiguous()
    assert torch.equal(extension.argmax(view), view.argmax(dim=-1))
    assert torch.equal(ops.argmax(view, use_cuda=True), view.argmax(dim=-1))
    x3 = torch.randn(2, 3, 40, device="cuda")
    assert torch.equal(ops.argmax(x3, use_cuda=True), x3.argmax(dim=-1))
    xd = torch.randn(4, 40, device="cuda", dtype=torch.float64)
    assert torch.equal(ops.argmax(xd, use_cuda=True), xd.argmax(dim=-1))
    with pytest.raises(RuntimeError, match="contiguous rows"):
        extension.argmax(base.t())
