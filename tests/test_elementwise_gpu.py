"""RMSNorm / QK-norm, RoPE and SwiGLU kernels on the MI355X (``-m gpu``).

Each kernel is compared with (a) the numpy oracle (oracle/elementwise.py) that rounds
where the reference rounds, and (b) the reference's own PyTorch expression evaluated
by PyTorch-ROCm on the same GPU, which is what the reference's kernel tests use
(test_swiglu_cuda.py:43-56, test_rope_cuda.py:154-205, test_rmsnorm_cuda.py:117-224).
RoPE and SwiGLU are expected bit-exact against (b); RMSNorm within one rounding of
the storage type (its fp32 sum of squares is reduced in a different order).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mini_vllm import torch_path
from mini_vllm.kernels import ops
from oracle import elementwise as ew

pytestmark = pytest.mark.gpu

NAMES = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
ULP = {torch.float32: 2**-23, torch.bfloat16: 2**-7, torch.float16: 2**-10}


def within_ulps(got: torch.Tensor, want: np.ndarray, dtype, ulps: float = 1.0) -> None:
    g = got.float().cpu().numpy()
    tol = np.abs(want) * ULP[dtype] * ulps + 1e-30
    bad = np.abs(g - want) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} elements beyond {ulps} ulp; max {np.abs(g - want).max()}"


# -------------------------------------------------------------------- rmsnorm


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(7, 1024), (33, 16, 128), (5, 8, 128), (3, 96), (2, 4096), (4, 6000), (1, 13)])
def test_rmsnorm_matches_the_oracle(extension, device, dtype, shape):
    x = (torch.randn(shape) * 2).to(dtype)
    w = (torch.rand(shape[-1]) + 0.5).to(dtype)
    got = extension.rmsnorm(x.to(device), w.to(device), 1e-6)
    want = ew.rms_norm(x.float().numpy(), w.float().numpy(), 1e-6, NAMES[dtype])
    within_ulps(got, want, dtype, ulps=1.0 if dtype != torch.float32 else 8.0)
    on_gpu = torch_path.rms_norm(x.to(device), w.to(device), 1e-6)
    within_ulps(got, on_gpu.float().cpu().numpy(), dtype, ulps=1.0 if dtype != torch.float32 else 8.0)


def test_rmsnorm_unit_weight_gives_unit_rms(extension, device):
    x = torch.randn(64, 1024, device=device) * 5
    out = extension.rmsnorm(x, torch.ones(1024, device=device), 1e-6)
    rms = out.double().pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-5)


def test_rmsnorm_zero_row_stays_finite(extension, device):
    out = extension.rmsnorm(torch.zeros(4, 128, device=device), torch.ones(128, device=device), 1e-6)
    assert torch.equal(out, torch.zeros_like(out))


def test_rmsnorm_reduces_in_fp32(extension, device):
    """A row of large equal bf16 values: a bf16 accumulator would overflow the mean."""
    x = torch.full((2, 1024), 3.0e4, dtype=torch.bfloat16, device=device)
    out = extension.rmsnorm(x, torch.ones(1024, dtype=torch.bfloat16, device=device), 1e-6)
    assert torch.allclose(out.float(), torch.ones(2, 1024, device=device), atol=1e-2)


def test_rmsnorm_misaligned_and_strided_inputs(extension, device):
    base = torch.randn(9, 129, dtype=torch.bfloat16, device=device)
    x = base[:, 1:]                       # 2-byte offset rows, not 16-byte aligned
    w = torch.rand(128, dtype=torch.bfloat16, device=device) + 0.5
    got = extension.rmsnorm(x, w, 1e-6)
    want = ew.rms_norm(x.float().cpu().numpy(), w.float().cpu().numpy(), 1e-6, "bf16")
    within_ulps(got, want, torch.bfloat16)
    xt = torch.randn(128, 6, dtype=torch.bfloat16, device=device).t()  # non-contiguous
    got = extension.rmsnorm(xt, w, 1e-6)
    within_ulps(got, ew.rms_norm(xt.float().cpu().numpy(), w.float().cpu().numpy(), 1e-6, "bf16"),
                torch.bfloat16)


def test_rmsnorm_refusals(extension, device):
    x = torch.randn(4, 8, device=device)
    with pytest.raises(RuntimeError, match="float64"):
        extension.rmsnorm(x.double(), torch.ones(8, device=device).double())
    with pytest.raises(RuntimeError, match="mixed dtypes"):
        extension.rmsnorm(x, torch.ones(8, device=device, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="last dimension"):
        extension.rmsnorm(x, torch.ones(9, device=device))


# ----------------------------------------------------------------------- rope


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("pos_dtype", [torch.int64, torch.int32])
def test_rope_matches_the_oracle_and_torch_bitwise(extension, device, dtype, pos_dtype):
    cos, sin = torch_path.rope_tables(128, 4096)
    x = torch.randn(1, 37, 16, 128).to(dtype)
    positions = torch.randint(0, 4096, (37,), dtype=pos_dtype)
    got = extension.rope(x.to(device), positions.to(device), cos.to(device), sin.to(device))
    want = ew.apply_rope(x.float().numpy(), positions.numpy(), cos.numpy(), sin.numpy(),
                         NAMES[dtype])
    assert np.array_equal(got.float().cpu().numpy(), want)
    on_gpu = torch_path.apply_rope(x.to(device), positions.to(device), cos.to(device), sin.to(device))
    assert torch.equal(got, on_gpu)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 80, 12, 256])
def test_rope_head_dims_vector_and_scalar_paths(extension, device, dtype, head_dim):
    # 64/80/256 take the 16-byte-chunk kernel for every dtype; 12 (halves of 6) does not
    # divide into chunks and takes the per-pair kernel.
    cos, sin = torch_path.rope_tables(head_dim, 300)
    x = torch.randn(2, 9, 3, head_dim).to(dtype)
    positions = torch.randint(0, 300, (9,), dtype=torch.int64)
    got = extension.rope(x.to(device), positions.to(device), cos.to(device), sin.to(device))
    want = ew.apply_rope(x.float().numpy(), positions.numpy(), cos.numpy(),
                         sin.numpy(), NAMES[dtype])
    assert np.array_equal(got.float().cpu().numpy(), want.reshape(got.shape))


def test_rope_misaligned_input_takes_the_pair_kernel(extension, device):
    cos, sin = (t.to(device) for t in torch_path.rope_tables(128, 64))
    base = torch.randn(1 + 5 * 2 * 128, dtype=torch.bfloat16, device=device)
    x = base[1:].view(1, 5, 2, 128)
    pos = torch.arange(5, device=device)
    assert torch.equal(extension.rope(x, pos, cos, sin),
                       torch_path.apply_rope(x.contiguous(), pos, cos, sin))


def test_rope_position_zero_is_identity_and_norms_are_kept(extension, device):
    cos, sin = (t.to(device) for t in torch_path.rope_tables(128, 64))
    x = torch.randn(1, 8, 4, 128, device=device)
    assert torch.equal(extension.rope(x, torch.zeros(8, dtype=torch.long, device=device), cos, sin), x)
    out = extension.rope(x, torch.arange(8, device=device), cos, sin)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = out[..., :64] ** 2 + out[..., 64:] ** 2
    assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)


def test_rope_decode_token_equals_its_prefill_position(extension, device):
    cos, sin = (t.to(device) for t in torch_path.rope_tables(128, 512))
    x = torch.randn(1, 50, 8, 128, dtype=torch.bfloat16, device=device)
    full = extension.rope(x, torch.arange(50, device=device), cos, sin)
    one = extension.rope(x[:, 37:38].contiguous(), torch.tensor([37], device=device), cos, sin)
    assert torch.equal(full[:, 37:38], one)


def test_rope_positions_broadcast_over_a_batch(extension, device):
    cos, sin = (t.to(device) for t in torch_path.rope_tables(64, 128))
    x = torch.randn(3, 10, 4, 64, device=device)
    pos = torch.arange(5, 15, device=device)
    got = extension.rope(x, pos, cos, sin)
    assert torch.equal(got, torch_path.apply_rope(x, pos, cos, sin))


def test_rope_out_of_range_position_is_nan_not_a_fault(extension, device):
    cos, sin = (t.to(device) for t in torch_path.rope_tables(64, 16))
    x = torch.randn(1, 3, 2, 64, device=device)
    out = extension.rope(x, torch.tensor([1, 99, -3], device=device), cos, sin)
    torch.cuda.synchronize()
    assert torch.isfinite(out[0, 0]).all()
    assert torch.isnan(out[0, 1]).all() and torch.isnan(out[0, 2]).all()


def test_rope_refusals(extension, device):
    cos, sin = (t.to(device) for t in torch_path.rope_tables(64, 16))
    x = torch.randn(4, 64, device=device)
    with pytest.raises(RuntimeError, match="head axis"):
        extension.rope(x, torch.arange(4, device=device), cos, sin)
    with pytest.raises(RuntimeError, match="float32"):
        extension.rope(x[None, :, None], torch.arange(4, device=device), cos.half(), sin.half())
    with pytest.raises(RuntimeError, match="broadcast"):
        extension.rope(torch.randn(1, 6, 2, 64, device=device), torch.arange(4, device=device), cos, sin)


# --------------------------------------------------------------------- swiglu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(64, 3072), (3, 1001), (1,)])
def test_swiglu_is_bitwise_equal_to_torch(extension, device, dtype, shape):
    g = (torch.randn(shape) * 4).to(dtype).to(device)
    u = torch.randn(shape).to(dtype).to(device)
    got = extension.swiglu(g, u)
    assert torch.equal(got, torch_path.silu(g) * u)
    want = ew.swiglu(g.float().cpu().numpy(), u.float().cpu().numpy(), NAMES[dtype])
    within_ulps(got, want, dtype, ulps=1.0 if dtype != torch.float32 else 4.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_swiglu_over_every_16_bit_input(extension, device, dtype):
    """Every finite 16-bit gate value against torch's expression, bit for bit (sign of
    zero included). In bit order, whole waves fall inside |g| < 32 (the short
    instruction path) or outside it (the general one); shuffled, most waves mix both
    and take the general path; a run of one magnitude exercises each path alone."""
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    g = bits.view(dtype)
    g = g[torch.isfinite(g.float())]
    gen = torch.Generator().manual_seed(5)
    u = (torch.randn(g.numel(), generator=gen) * 2).to(dtype).to(device)
    small = g[g.float().abs() < 32]
    for gate in (g, g[torch.randperm(g.numel(), generator=gen)], small.repeat(2)[: g.numel()]):
        gate = gate.to(device)
        up = u[: gate.numel()]
        got = extension.swiglu(gate, up)
        want = torch_path.silu(gate) * up
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,dim", [(1, 128), (37, 1024), (2048, 1024), (5, 2048)])
def test_add_rmsnorm_is_the_add_then_rmsnorm(extension, device, dtype, rows, dim):
    """One pass for a block's residual add and the RMSNorm after it: h bitwise torch's
    add, the normed rows bitwise the rmsnorm kernel on that h; ops routes to it."""
    gen = torch.Generator().manual_seed(rows * 3 + dim)
    x = (torch.randn(rows, dim, generator=gen) * 2).to(dtype).to(device)
    r = torch.randn(rows, dim, generator=gen).to(dtype).to(device)
    w = (torch.rand(dim, generator=gen) + 0.5).to(dtype).to(device)
    h, normed = extension.add_rmsnorm(x, r, w, 1e-6)
    want_h = r + x
    assert torch.equal(h, want_h)
    assert torch.equal(normed, extension.rmsnorm(want_h, w, 1e-6))
    h2, n2 = ops.add_rmsnorm(x, r, w, 1e-6, use_cuda=True)
    assert torch.equal(h2, h) and torch.equal(n2, normed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,dim,vocab", [(1, 128, 50), (32, 1024, 151936), (300, 1024, 4000),
                                            (5, 2048, 77)])
@pytest.mark.parametrize("indexed", [False, True])
def test_embed_rmsnorm_is_the_lookup_then_rmsnorm(extension, device, dtype, rows, dim, vocab,
                                                  indexed):
    """The token embedding and the first block's input norm in one launch: h bitwise the
    table rows (index_select), the normed rows bitwise the rmsnorm kernel on them; with
    an index, row i's token is prev[index[i]] where index[i] >= 0 and the row's own id
    where it is -1 (a decode graph's previous tokens and host ids); ops routes to it, and
    its torch path (use_cuda=False) picks the same tokens."""
    gen = torch.Generator().manual_seed(rows + dim + vocab)
    table = (torch.randn(vocab, dim, generator=gen) * 0.5).to(dtype).to(device)
    w = (torch.rand(dim, generator=gen) + 0.5).to(dtype).to(device)
    own = torch.randint(0, vocab, (rows,), generator=gen).to(device)
    index = prev = None
    ids = own
    if indexed:
        prev = torch.randint(0, vocab, (rows + 40,), generator=gen).to(device)
        index = torch.randint(-1, rows + 40, (rows,), generator=gen).to(device)
        index[0] = -1
        ids = torch.where(index >= 0, prev.index_select(0, index.clamp(min=0)), own)
    h, normed = extension.embed_rmsnorm(table, own, w, 1e-6, index=index, prev=prev)
    want_h = table.index_select(0, ids)
    assert torch.equal(h, want_h)
    assert torch.equal(normed, extension.rmsnorm(want_h, w, 1e-6))
    h2, n2 = ops.embed_rmsnorm(table, own, w, 1e-6, use_cuda=True, index=index, prev=prev)
    assert torch.equal(h2, h) and torch.equal(n2, normed)
    h3, _ = ops.embed_rmsnorm(table, own, w, 1e-6, use_cuda=False, index=index, prev=prev)
    assert torch.equal(h3, want_h)


def test_embed_rmsnorm_out_of_range_ids_give_nan_rows(extension, device):
    """A token id outside [0, vocab) reads nothing and yields NaN rows; its neighbours are
    unaffected. The torch path (use_cuda=False) agrees on the valid rows."""
    table = torch.randn(10, 256, dtype=torch.bfloat16, device=device)
    w = torch.ones(256, dtype=torch.bfloat16, device=device)
    ids = torch.tensor([3, -1, 10, 9], device=device)
    h, normed = extension.embed_rmsnorm(table, ids, w, 1e-6)
    torch.cuda.synchronize()
    for i in (1, 2):
        assert torch.isnan(h[i]).all() and torch.isnan(normed[i]).all()
    ok = torch.tensor([0, 3], device=device)
    valid = ids.index_select(0, ok)
    h_t, n_t = ops.embed_rmsnorm(table, valid, w, 1e-6, use_cuda=False)
    assert torch.equal(h.index_select(0, ok), h_t)
    assert torch.equal(normed.index_select(0, ok), extension.rmsnorm(h_t, w, 1e-6))


def test_embed_rmsnorm_refusals_and_fallback(extension, device):
    table = torch.randn(10, 100, dtype=torch.bfloat16, device=device)  # rows not whole chunks
    w = torch.ones(100, dtype=torch.bfloat16, device=device)
    ids = torch.tensor([1, 2], device=device)
    assert not extension.embed_rmsnorm_supported(table, ids, w)
    with pytest.raises(RuntimeError, match="16-byte chunks"):
        extension.embed_rmsnorm(table, ids, w)
    assert not extension.embed_rmsnorm_supported(table[:, :96].contiguous(), ids.int(), w[:96])
    h, n = ops.embed_rmsnorm(table, ids, w, use_cuda=True)  # the lookup and rmsnorm instead
    assert torch.equal(h, table[ids]) and torch.equal(n, extension.rmsnorm(table[ids], w))


def test_add_rmsnorm_refusals_and_fallback(extension, device):
    x = torch.randn(4, 100, dtype=torch.bfloat16, device=device)  # 100 not a whole chunk count
    w = torch.ones(100, dtype=torch.bfloat16, device=device)
    assert not extension.add_rmsnorm_supported(x, x, w)
    with pytest.raises(RuntimeError, match="16-byte chunks"):
        extension.add_rmsnorm(x, x, w)
    h, n = ops.add_rmsnorm(x, x, w, use_cuda=True)  # the two ops instead
    assert torch.equal(h, x + x) and torch.equal(n, extension.rmsnorm(x + x, w))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(1, 16), (7, 48), (300, 3072)])
def test_swiglu_interleaved_is_split_then_swiglu(extension, device, dtype, rows, cols):
    """SwiGLU read straight off the 16-column gate/up interleave equals splitting it
    (torch_path.split_gate_up) and calling swiglu, bit for bit."""
    gen = torch.Generator().manual_seed(rows + cols)
    y = (torch.randn(rows, 2 * cols, generator=gen) * 3).to(dtype).to(device)
    gate, up = torch_path.split_gate_up(y)
    want = extension.swiglu(gate.contiguous(), up.contiguous())
    got = extension.swiglu_interleaved(y)
    assert got.shape == (rows, cols) and torch.equal(got, want)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        extension.swiglu_interleaved(y[:, : 2 * cols - 16])


def test_swiglu_misaligned_views(extension, device):
    g = torch.randn(1025, dtype=torch.bfloat16, device=device)[1:]
    u = torch.randn(1025, dtype=torch.bfloat16, device=device)[1:]
    assert torch.equal(extension.swiglu(g, u), torch_path.silu(g) * u)


def test_swiglu_refusals(extension, device):
    with pytest.raises(RuntimeError, match="must match"):
        extension.swiglu(torch.randn(4, device=device), torch.randn(5, device=device))
    with pytest.raises(RuntimeError, match="float64"):
        extension.swiglu(torch.randn(4, device=device).double(), torch.randn(4, device=device).double())


# ------------------------------------------------------------------ ops seam


def test_ops_route_elementwise_to_the_kernels(extension, device, monkeypatch):
    calls = []
    for name in ("rmsnorm", "rope", "swiglu"):
        original = getattr(extension, name)

        def spy(*a, _orig=original, _name=name, **k):
            calls.append(_name)
            return _orig(*a, **k)

        monkeypatch.setattr(extension, name, spy)
    x = torch.randn(4, 128, device=device)
    ops.rmsnorm(x, torch.ones(128, device=device), use_cuda=True)
    cos, sin = (t.to(device) for t in torch_path.rope_tables(128, 16))
    ops.rope(x[None, :, None], torch.arange(4, device=device), cos, sin, use_cuda=True)
    ops.swiglu(x, x, use_cuda=True)
    assert calls == ["rmsnorm", "rope", "swiglu"]


def test_hello_axpby(extension, device):
    x = torch.randn(1000, device=device)
    assert torch.allclose(extension.hello(x, 2.0, 3.0), 2.0 * x + 3.0)


# ---------------------------------------------------------------- qk_norm_rope


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [32, 64, 128, 256])
@pytest.mark.parametrize("pos_dtype", [torch.int64, torch.int32])
def test_qk_norm_rope_is_bitwise_the_unfused_kernels(extension, device, dtype, head_dim, pos_dtype):
    t, hq, hk = 37, 16, 8
    q = (torch.randn(t, hq, head_dim) * 2).to(dtype).to(device)
    k = (torch.randn(t, hk, head_dim) * 2).to(dtype).to(device)
    wq = (torch.rand(head_dim) + 0.5).to(dtype).to(device)
    wk = (torch.rand(head_dim) + 0.5).to(dtype).to(device)
    cos, sin = (x.to(device) for x in torch_path.rope_tables(head_dim, 512))
    pos = torch.randint(0, 512, (t,), dtype=pos_dtype).to(device)
    assert extension.qk_norm_rope_supported(dtype, head_dim)
    fq, fk = extension.qk_norm_rope(q, k, wq, wk, pos, cos, sin, 1e-6)
    uq = extension.rope(extension.rmsnorm(q, wq, 1e-6).unsqueeze(0), pos, cos, sin).squeeze(0)
    uk = extension.rope(extension.rmsnorm(k, wk, 1e-6).unsqueeze(0), pos, cos, sin).squeeze(0)
    torch.cuda.synchronize()
    for got, want in ((fq, uq), (fk, uk)):
        bad = (got != want).nonzero()
        assert bad.numel() == 0, [(tuple(i.tolist()), float(got[tuple(i)]), float(want[tuple(i)]))
                                  for i in bad[:6]]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("t,hq,hk", [(4096, 16, 8), (1500, 16, 8), (3000, 6, 2)])
def test_qk_norm_rope_row_groups_are_bitwise_the_unfused_kernels(extension, device, dtype, t, hq, hk):
    """Large calls, where one lane group takes 8, 4 or 2 heads of a token (the head
    counts and the token count pick it), bitwise the unfused kernels, including rows at
    out-of-range positions (NaN) among in-range ones."""
    d = 128
    gen = torch.Generator().manual_seed(t + hq)
    q = (torch.randn(t, hq, d, generator=gen) * 2).to(dtype).to(device)
    k = (torch.randn(t, hk, d, generator=gen) * 2).to(dtype).to(device)
    wq = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    wk = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    cos, sin = (x.to(device) for x in torch_path.rope_tables(d, 8192))
    pos = torch.randint(0, 8192, (t,), generator=gen)
    pos[::97] = 8192  # out of range: NaN rows
    pos = pos.to(device)
    fq, fk = extension.qk_norm_rope(q, k, wq, wk, pos, cos, sin, 1e-6)
    uq = extension.rope(extension.rmsnorm(q, wq, 1e-6).unsqueeze(0), pos, cos, sin).squeeze(0)
    uk = extension.rope(extension.rmsnorm(k, wk, 1e-6).unsqueeze(0), pos, cos, sin).squeeze(0)
    torch.cuda.synchronize()
    for got, want in ((fq, uq), (fk, uk)):
        assert torch.equal(torch.isnan(got), torch.isnan(want))
        assert torch.equal(got.nan_to_num(0.0), want.nan_to_num(0.0))
    assert torch.isnan(fq[97]).all() and torch.isfinite(fq[1]).all()


def test_qk_norm_rope_against_the_oracle(extension, device):
    """Within two storage ulps of the numpy oracle's rms_norm -> apply_rope (the norm's
    fp32 sum order may move one rounding by one ulp)."""
    t, hq, hk, d = 20, 4, 2, 128
    q = (torch.randn(t, hq, d) * 2).to(torch.bfloat16)
    k = (torch.randn(t, hk, d) * 2).to(torch.bfloat16)
    wq = (torch.rand(d) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(d) + 0.5).to(torch.bfloat16)
    cos, sin = torch_path.rope_tables(d, 64)
    pos = torch.randint(0, 64, (t,))
    fq, fk = extension.qk_norm_rope(q.to(device), k.to(device), wq.to(device), wk.to(device),
                                    pos.to(device), cos.to(device), sin.to(device), 1e-6)
    for x, w, got in ((q, wq, fq), (k, wk, fk)):
        n = ew.rms_norm(x.float().numpy(), w.float().numpy(), 1e-6, "bf16")
        want = ew.apply_rope(n[None], pos.numpy(), cos.numpy(), sin.numpy(), "bf16")[0]
        err = np.abs(got.float().cpu().numpy() - want)
        assert np.all(err <= np.maximum(np.abs(want), 2.0**-6) * 2.0**-7 * 2), err.max()


def test_qk_norm_rope_broadcast_positions_and_nan_for_out_of_range(extension, device):
    cos, sin = (x.to(device) for x in torch_path.rope_tables(64, 16))
    q = torch.randn(6, 2, 64, device=device)
    k = torch.randn(6, 1, 64, device=device)
    w = torch.ones(64, device=device)
    fq, fk = extension.qk_norm_rope(q, k, w, w, torch.tensor([3, 99, 5], device=device), cos, sin)
    torch.cuda.synchronize()
    assert torch.isnan(fq[1]).all() and torch.isnan(fq[4]).all() and torch.isnan(fk[1]).all()
    assert torch.isfinite(fq[[0, 2, 3, 5]]).all()
    uq = extension.rope(extension.rmsnorm(q, w).unsqueeze(0), torch.tensor([3, 99, 5], device=device), cos, sin)
    assert torch.equal(fq[0], uq[0, 0]) and torch.equal(fq[5], uq[0, 5])


def test_ops_qk_norm_rope_routes_and_refuses(extension, device):
    cos, sin = (x.to(device) for x in torch_path.rope_tables(128, 16))
    q = torch.randn(3, 4, 128, dtype=torch.bfloat16, device=device)
    k = torch.randn(3, 2, 128, dtype=torch.bfloat16, device=device)
    w = torch.ones(128, dtype=torch.bfloat16, device=device)
    pos = torch.arange(3, device=device)
    kq, kk = ops.qk_norm_rope(q, k, w, w, pos, cos, sin, use_cuda=True)
    tq, tk = ops.qk_norm_rope(q, k, w, w, pos, cos, sin, use_cuda=False)
    assert (kq.float() - tq.float()).abs().max() <= 2 ** -5
    with pytest.raises(RuntimeError, match="share a dtype"):
        extension.qk_norm_rope(q, k.float(), w, w, pos, cos, sin)
    with pytest.raises(RuntimeError, match="T x H_q x D"):
        extension.qk_norm_rope(q[0], k, w, w, pos, cos, sin)
