"""Skinny projection kernels (``ops.linear`` and its fused variants, ``mvllm_linear*``)
on the MI355X (``-m gpu``).

The reference computes projections with ``x @ w.T`` through the vendor BLAS
(model/basics.py ``linear``); the kernel must return the same function. Both sum in
fp32 and round once, in different orders, so the bar is: every element within one
unit in the last place (of the output dtype) of the fp32 product ``x.float() @
w.float().T`` rounded to that dtype, plus the spread of two fp32 summation orders
(4 sqrt(K) 2^-24 sum_k |x_k w_k|, which only matters where the sum cancels to near
zero), and within two ulps of torch's own result. The fused variants (q/k/v split,
residual add, gate/up + SwiGLU) must equal the plain kernel followed by the unfused
ops bit for bit, and the weight packing must equal its PyTorch definition
(``torch_path.pack_fragments``) bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from mini_vllm import torch_path
from mini_vllm.kernels import ops
from mini_vllm.kernels.extension import DTYPE_CODES

pytestmark = pytest.mark.gpu


def _ulp(ref: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One unit in the last place of each element of ``ref`` (fp32) in ``dtype``."""
    mant = {torch.bfloat16: 7, torch.float16: 10}[dtype]
    mag = ref.abs().clamp_min(torch.finfo(dtype).tiny)
    return torch.exp2(torch.floor(torch.log2(mag)) - mant)


def _operands(m, n, k, dtype, seed):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(m, k, generator=gen).to(dtype).cuda()
    w = (torch.randn(n, k, generator=gen) * 0.05).to(dtype).cuda()
    return x, w, gen


def _lin(extension, x, w):
    return extension.linear(x, extension.linear_pack(w), w.shape[0])


def _check(extension, m, n, k, dtype, seed=0):
    x, w, _ = _operands(m, n, k, dtype, seed + 131 * m + 7 * n + k)
    got = _lin(extension, x, w)
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
@pytest.mark.parametrize("n,k", [(33, 64), (1000, 1088), (100, 3072)])
def test_pack_equals_its_definition(extension, device, n, k, dtype):
    """mvllm_linear_pack writes the fragment order torch_path.pack_fragments defines
    (ragged last tile zero-padded), and piece (t, s, l) holds the row/column slice it
    names."""
    _, w, _ = _operands(1, n, k, dtype, 3 + n)
    packed = extension.linear_pack(w)
    want = torch_path.pack_fragments(w)
    assert packed.shape == want.shape and torch.equal(packed, want)
    pieces = packed.view(-1, 64, 8)
    steps = k // 16
    for t, s, l in ((0, 0, 0), (0, steps - 1, 63), (n // 32, 1, 37)):
        r, h = 32 * t + (l & 31), l >> 5
        got = pieces[t * steps + s, l]
        if r < n:
            assert torch.equal(got, w[r, 16 * s + 8 * h:16 * s + 8 * h + 8])
        else:
            assert not got.any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 7, 32, 33, 64])
def test_rows_up_to_64(extension, device, m, dtype):
    _check(extension, m, 1000, 1024, dtype)


@pytest.mark.parametrize("n,k", [(1, 64), (31, 128), (32, 3072), (33, 2048), (4096, 1024),
                                 (6144, 1024), (1024, 3072), (40, 1088), (96, 4160),
                                 (64, 65536)])
def test_shapes_of_the_model(extension, device, n, k):
    """Column counts on and off the 32-column tile, K of every projection of the
    Qwen3-0.6B shape (1024, 2048, 3072), the smallest and largest served, K split
    unevenly over the waves (1088 = 68 k-steps over 8 waves) and K past one batch per
    wave (4160 over 16 waves; 65536: 16 batches of 16 k-steps per wave)."""
    _check(extension, 32, n, k, torch.bfloat16)


def test_lm_head_shape(extension, device):
    """The tied-embedding logits projection: N = 151936, K = 1024."""
    _check(extension, 17, 151936, 1024, torch.bfloat16)


def test_ops_dispatch_by_size(extension, device):
    """``ops.linear`` takes the kernel for at most 64 rows against a packed weight and
    the BLAS otherwise, and the extension refuses what the kernel does not serve."""
    w = torch.randn(48, 256, dtype=torch.bfloat16, device="cuda")
    pw = ops.pack_weight(w, use_cuda=True)
    assert pw.packed is not None and pw.dense is w
    x = torch.randn(65, 256, dtype=torch.bfloat16, device="cuda")
    assert not extension.linear_supported(x, pw.packed, 48)
    torch.testing.assert_close(ops.linear(x, pw, use_cuda=True), x @ w.t())
    with pytest.raises(RuntimeError, match="skinny kernel"):
        extension.linear(x, pw.packed, 48)
    x = torch.randn(4, 256, dtype=torch.bfloat16, device="cuda")
    assert not extension.linear_supported(x, pw.packed, 100)  # more rows than the buffer packs
    assert extension.linear_supported(x, pw.packed, 48)
    got = ops.linear(x, pw, use_cuda=True)
    assert got.shape == (4, 48) and torch.equal(got, extension.linear(x, pw.packed, 48))
    torch.testing.assert_close(ops.linear(x, w, use_cuda=True), x @ w.t())  # dense: BLAS
    w96 = torch.randn(48, 96, dtype=torch.bfloat16, device="cuda")  # K not a multiple of 64
    assert not extension.linear_packable(w96)
    assert ops.pack_weight(w96, use_cuda=True).packed is None
    x96 = torch.randn(4, 96, dtype=torch.bfloat16, device="cuda")
    torch.testing.assert_close(ops.linear(x96, ops.pack_weight(w96, use_cuda=True), use_cuda=True),
                               x96 @ w96.t())


def test_known_answer_identity(extension, device):
    """x @ I = x exactly (each output is one product of an element and 1)."""
    x = torch.randn(9, 128, dtype=torch.bfloat16, device="cuda")
    eye = torch.eye(128, dtype=torch.bfloat16, device="cuda")
    assert torch.equal(_lin(extension, x, eye), x)


def test_c_abi_refusals(extension, device):
    """Shapes and dtypes the kernel does not serve are refused by the library, not run,
    and so is a K > 1024 call without its partial-sum workspace."""
    x, w, _ = _operands(4, 64, 128, torch.bfloat16, 6)
    packed = extension.linear_pack(w)
    y = torch.empty(4, 64, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    bf16 = DTYPE_CODES[torch.bfloat16]
    lib = extension.lib
    call = lambda m, k, dtype=bf16, out=y.data_ptr(): lib.mvllm_linear(
        out, x.data_ptr(), packed.data_ptr(), m, 64, k, dtype, 0, 0, stream)
    assert call(65, 128) == 2
    assert call(4, 96) == 2
    assert call(4, 128, DTYPE_CODES[torch.float32]) == 2
    assert call(4, 128, out=0) == 1
    assert lib.mvllm_linear_split(y.data_ptr(), y.data_ptr(), 0, x.data_ptr(), packed.data_ptr(),
                                  4, 40, 24, 0, 128, bf16, 0, 0, stream) == 1
    assert lib.mvllm_linear_pack(packed.data_ptr(), w.data_ptr(), 64, 96, bf16, stream) == 2
    assert call(4, 128) == 0
    assert torch.equal(y, extension.linear(x, packed, 64))
    assert lib.mvllm_linear_workspace_bytes(4, 64, 1024) == 0
    need = lib.mvllm_linear_workspace_bytes(4, 64, 2048)
    assert need == 2 * 8 * 32 * 32 * 4  # 2 tiles x 8 waves x one 32 x 32 fp32 tile
    x2, w2, _ = _operands(4, 64, 2048, torch.bfloat16, 7)
    p2 = extension.linear_pack(w2)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    args = (y.data_ptr(), x2.data_ptr(), p2.data_ptr(), 4, 64, 2048, bf16)
    assert lib.mvllm_linear(*args, 0, 0, stream) == 4  # MVLLM_ERR_WORKSPACE
    assert lib.mvllm_linear(*args, ws.data_ptr(), need - 1, stream) == 4
    assert lib.mvllm_linear(*args, ws.data_ptr(), need, stream) == 0
    assert torch.equal(y, extension.linear(x2, p2, 64))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 20, 64])
def test_split_equals_separate_projections(extension, device, m, dtype):
    """q/k/v over the concatenated weights, bitwise the three separate projections
    (each column's sum is formed the same way wherever its tile lies)."""
    x, wq, gen = _operands(m, 2048, 1024, dtype, 11 + m)
    wk = (torch.randn(1024, 1024, generator=gen) * 0.05).to(dtype).cuda()
    wv = (torch.randn(1000, 1024, generator=gen) * 0.05).to(dtype).cuda()
    packed = extension.linear_pack(torch.cat((wq, wk, wv)))
    q, k, v = extension.linear_split(x, packed, (2048, 1024, 1000))
    for got, w in ((q, wq), (k, wk), (v, wv)):
        assert got.is_contiguous() and torch.equal(got, _lin(extension, x, w))
    packed2 = extension.linear_pack(torch.cat((wq, wk)))
    a, b = extension.linear_split(x, packed2, (2048, 1024))
    assert torch.equal(a, q) and torch.equal(b, k)
    with pytest.raises(RuntimeError, match="multiples of 32"):
        extension.linear_split(x, packed2, (2040, 1032))
    pw = ops.PackedWeight(torch.cat((wq, wk, wv)), packed)
    got = ops.linear_split(x, pw, (2048, 1024, 1000), use_cuda=True)
    assert all(torch.equal(g, r) for g, r in zip(got, (q, k, v)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(1, 1024, 2048), (37, 1024, 3072), (64, 1000, 64)])
def test_residual_equals_add_after_projection(extension, device, m, n, k, dtype):
    """residual + x w^T in one launch, bitwise torch's add of the rounded projection."""
    x, w, gen = _operands(m, n, k, dtype, 23 + m)
    r = torch.randn(m, n, generator=gen).to(dtype).cuda()
    pw = ops.pack_weight(w, use_cuda=True)
    got = extension.linear_residual(x, pw.packed, r)
    assert torch.equal(got, r + extension.linear(x, pw.packed, n))
    assert torch.equal(ops.linear_residual(x, pw, r, use_cuda=True), got)
    with pytest.raises(RuntimeError, match="residual must be"):
        extension.linear_residual(x, pw.packed, r.float())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,i", [(1, 3072), (48, 3072), (5, 48)])
def test_swiglu_equals_gate_up_then_swiglu(extension, device, m, i, dtype):
    """gate/up + SwiGLU in one launch over the 16-row interleave, bitwise the two
    projections followed by the SwiGLU kernel."""
    x, gate, gen = _operands(m, i, 1024, dtype, 37 + m)
    up = (torch.randn(i, 1024, generator=gen) * 0.05).to(dtype).cuda()
    pw = ops.pack_weight(torch_path.interleave_gate_up(gate, up), use_cuda=True)
    got = extension.linear_swiglu(x, pw.packed, i)
    want = ops.swiglu(_lin(extension, x, gate), _lin(extension, x, up), use_cuda=True)
    assert got.shape == (m, i) and torch.equal(got, want)
    assert torch.equal(ops.linear_swiglu(x, pw, use_cuda=True), got)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(1, 1024, 2048), (32, 1024, 3072), (33, 1024, 2048),
                                   (64, 2048, 1088), (7, 4096, 4096), (3, 1024, 5120),
                                   (9, 2048, 3072), (2, 1024, 4096)])
def test_residual_rmsnorm_equals_the_unfused_pair(extension, device, m, n, k, dtype):
    """(h, normed) of the fused launch pair, bitwise linear_residual then the RMSNorm
    kernel (random norm weight, eps 1e-6). The K values give 8, 12, 16 and 20 split
    waves, so every batch of partial loads (4, 8, 12 or 16 waves at a time, one round
    or several) is run."""
    x, w, gen = _operands(m, n, k, dtype, 41 + m + k)
    r = torch.randn(m, n, generator=gen).to(dtype).cuda()
    nw = (torch.rand(n, generator=gen) + 0.5).to(dtype).cuda()
    pw = ops.pack_weight(w, use_cuda=True)
    h, normed = extension.linear_residual_rmsnorm(x, pw.packed, r, nw, 1e-6)
    want_h = extension.linear_residual(x, pw.packed, r)
    assert torch.equal(h, want_h)
    assert torch.equal(normed, ops.rmsnorm(want_h, nw, 1e-6, use_cuda=True))
    got = ops.linear_residual_rmsnorm(x, pw, r, nw, 1e-6, use_cuda=True)
    assert got is not None and torch.equal(got[0], h) and torch.equal(got[1], normed)


def test_residual_rmsnorm_refuses_what_it_does_not_serve(extension, device):
    """K <= 1024 or N not a multiple of 512: ops returns None (the caller runs the two
    ops), the extension raises."""
    x, w, gen = _operands(4, 1024, 1024, torch.bfloat16, 3)
    r = torch.randn(4, 1024, generator=gen).to(torch.bfloat16).cuda()
    nw = torch.ones(1024, dtype=torch.bfloat16, device="cuda")
    pw = ops.pack_weight(w, use_cuda=True)
    assert ops.linear_residual_rmsnorm(x, pw, r, nw, use_cuda=True) is None
    with pytest.raises(RuntimeError, match="not served"):
        extension.linear_residual_rmsnorm(x, pw.packed, r, nw, 1e-6)
    x, w, gen = _operands(4, 1000, 2048, torch.bfloat16, 4)
    pw = ops.pack_weight(w, use_cuda=True)
    r = torch.randn(4, 1000, generator=gen).to(torch.bfloat16).cuda()
    assert ops.linear_residual_rmsnorm(x, pw, r, nw[:1000], use_cuda=True) is None

