"""The op seam on the CPU: routing rules and the explicit PyTorch path."""

from __future__ import annotations

import pytest
import torch

from conftest import assert_max_abs
from mini_vllm import torch_path
from mini_vllm.kernels import ops
from mini_vllm.workloads import build_batch
from oracle import elementwise as ew
from oracle.paged_attention import paged_attention as oracle_paged


def test_use_cuda_true_on_cpu_tensors_falls_back_to_the_pytorch_path():
    """The reference's contract (ops.py:82-89, tests/test_qwen3_cached.py:335-350): the
    flag means "use kernels where they apply", so CPU tensors take the PyTorch path and
    give exactly its result; the decline is reported by dispatch_report."""
    ops.FALLBACKS.clear()
    b = build_batch([20], [1], num_q_heads=4, num_kv_heads=2, head_dim=32)
    assert torch.equal(ops.paged_attention(*b.args(), use_cuda=True),
                       ops.paged_attention(*b.args(), use_cuda=False))
    x, w = torch.randn(2, 8), torch.rand(8) + 0.5
    assert torch.equal(ops.rmsnorm(x, w, use_cuda=True), ops.rmsnorm(x, w))
    g, u = torch.randn(4), torch.randn(4)
    assert torch.equal(ops.swiglu(g, u, use_cuda=True), ops.swiglu(g, u))
    report = ops.dispatch_report(True)
    assert "declined calls" in report and "needs device tensors" in report
    assert ops.FALLBACKS["paged_attention"] and ops.FALLBACKS["rmsnorm"]


def test_strict_mode_raises_on_every_decline():
    b = build_batch([20], [1], num_q_heads=4, num_kv_heads=2, head_dim=32)
    with ops.strict_kernels():
        with pytest.raises(RuntimeError, match="use_cuda=True needs device tensors"):
            ops.paged_attention(*b.args(), use_cuda=True)
        with pytest.raises(RuntimeError, match="strict kernel mode"):
            ops.rmsnorm(torch.randn(2, 8), torch.ones(8), use_cuda=True)
        with pytest.raises(RuntimeError, match="needs device tensors"):
            ops.swiglu(torch.randn(4), torch.randn(4), use_cuda=True)
        # use_cuda=False is an explicit choice of the PyTorch path, never a decline
        ops.rmsnorm(torch.randn(2, 8), torch.ones(8), use_cuda=False)
    assert not ops.is_strict()


def test_paged_gate_reasons_follow_the_reference():
    """``_kernel_can_page`` (reference ops.py:257-275) plus this library's head dims:
    each unserved shape names its reason; a served one has none. Checked on
    meta tensors for the layout rules, device placement aside."""
    b = build_batch([20], [1], num_q_heads=4, num_kv_heads=2, head_dim=32)
    can = ops._kernel_can_page
    assert "device tensors" in can(b.q, b.key_pool, b.value_pool, b.block_tables)
    assert "T x H_q x D" in can(b.q.unsqueeze(0), b.key_pool, b.value_pool, b.block_tables)
    assert "float64" in can(b.q.double(), b.key_pool, b.value_pool, b.block_tables)
    assert "share a dtype" in can(b.q.half(), b.key_pool, b.value_pool, b.block_tables)
    q96 = torch.randn(1, 4, 96)
    pool96 = torch.randn(4, 16, 2, 96)
    assert "head dim 96" in can(q96, pool96, pool96, b.block_tables)
    assert "contiguous" in can(b.q, b.key_pool.transpose(1, 2), b.value_pool, b.block_tables)
    assert "int32" in can(b.q, b.key_pool, b.value_pool, b.block_tables.long())
    assert "int32" in can(b.q, b.key_pool, b.value_pool, b.block_tables,
                          (b.cu_seqlens_q.long(),))


def test_a_head_dim_the_kernels_do_not_serve_runs_the_pytorch_path():
    """Reference behaviour for D <= 256 outside this build's set: the PyTorch path."""
    b = build_batch([30, 5], [1, 5], num_q_heads=4, num_kv_heads=2, head_dim=48, seed=5)
    got = ops.paged_attention(*b.args(), use_cuda=True)
    want = oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale)
    assert_max_abs(got, want, 1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_torch_path_paged_attention_matches_the_oracle(dtype):
    b = build_batch([300, 1, 40, 64], [1, 1, 8, 64], dtype=dtype, num_q_heads=8,
                    num_kv_heads=2, head_dim=64, seed=3)
    got = ops.paged_attention(*b.args(), use_cuda=False)
    want = oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale)
    assert_max_abs(got, want, 1e-5 if dtype == torch.float32 else 3e-2)


def test_torch_path_fp8_pool():
    b = build_batch([100, 30], [1, 30], dtype=torch.bfloat16, kv_dtype=torch.float8_e4m3fn,
                    num_q_heads=8, num_kv_heads=2, head_dim=64, seed=2)
    got = ops.paged_attention(*b.args(), use_cuda=False, k_scale=b.k_scale, v_scale=b.v_scale)
    want = oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale, b.k_scale, b.v_scale)
    assert_max_abs(got, want, 3e-2)


def test_torch_path_elementwise_matches_the_oracle():
    x = torch.randn(6, 128).to(torch.bfloat16)
    w = (torch.rand(128) + 0.5).to(torch.bfloat16)
    got = ops.rmsnorm(x, w).float().numpy()
    want = ew.rms_norm(x.float().numpy(), w.float().numpy(), 1e-6, "bf16")
    assert (abs(got - want) <= abs(want) * 2**-7 + 1e-30).all()
    cos, sin = torch_path.rope_tables(64, 32)
    xr = torch.randn(1, 5, 3, 64)
    pos = torch.tensor([0, 3, 9, 31, 2])
    assert (ops.rope(xr, pos, cos, sin).numpy() ==
            ew.apply_rope(xr.numpy(), pos.numpy(), cos.numpy(), sin.numpy())).all()


def test_dispatch_report_names_every_op():
    on = ops.dispatch_report(True)
    off = ops.dispatch_report(False)
    for name in ops.CUDA_KERNELS:
        assert name in on and name in off
    assert "paged_attention    hip" in on
    assert "use_cuda is off" in off
    assert set(ops.cuda_kernel_names()) == {"rmsnorm", "rope", "swiglu", "paged_attention", "kv_write",
                                            "qk_norm_rope", "linear", "decode_attention",
                                            "flash_prefill", "argmax", "blas_linear"}
    assert not ops.NOT_YET_FASTER  # every kernel in the library is dispatched


def test_dense_attention_torch_path_decode_and_causal():
    q = torch.randn(2, 8, 1, 32)
    k = torch.randn(2, 4, 10, 32)
    v = torch.randn(2, 4, 10, 32)
    out = ops.attention(q, k, v)
    g = 2
    ref = torch.softmax((q.reshape(2, 4, g, 1, 32) @ k.unsqueeze(2).transpose(-1, -2)) / 32**0.5, -1)
    ref = (ref @ v.unsqueeze(2)).reshape(2, 8, 1, 32)
    assert torch.allclose(out, ref, atol=1e-6)
    assert torch.equal(ops.attention(q, k, v, use_cuda=True), out)
    with ops.strict_kernels(), pytest.raises(RuntimeError, match="device tensors"):
        ops.attention(q, k, v, use_cuda=True)


def test_dense_kernel_gate_follows_the_reference():
    """``_kernel_can_attend`` (reference ops.py:278-305): decode takes None or "causal",
    prefill only "causal"; explicit masks, fp64, S < L and a strided head dim go to the
    PyTorch path."""
    q1, qL = torch.randn(1, 4, 1, 32), torch.randn(1, 4, 6, 32)
    k = torch.randn(1, 2, 9, 32)
    can = ops._kernel_can_attend
    assert can(q1, k, k, None, True) and can(q1, k, k, "causal", True)
    assert not can(q1, k, k, torch.zeros(1, 9), True)
    assert can(qL, k, k, "causal", False) and not can(qL, k, k, None, False)
    assert not can(qL, k[:, :, :5], k[:, :, :5], "causal", False)  # S < L
    assert not can(q1.double(), k.double(), k.double(), None, True)
    strided = torch.randn(1, 2, 9, 64)[..., ::2]
    assert not can(q1, strided, strided, None, True)


def test_linear_torch_path_is_x_matmul_w_transposed():
    x = torch.randn(5, 64)
    w = torch.randn(7, 64)
    torch.testing.assert_close(ops.linear(x, w), x @ w.t())
    assert torch.equal(ops.linear(x, w, use_cuda=True), x @ w.t())
    with ops.strict_kernels(), pytest.raises(RuntimeError, match="device tensors"):
        ops.linear(x, w, use_cuda=True)


def test_gate_up_interleave_layout():
    """Rows 32j .. 32j+15 of the interleave are gate rows 16j .. 16j+15 and the next 16
    the same up rows; split_gate_up undoes it on the product's columns."""
    gate = torch.arange(48 * 3, dtype=torch.float32).view(48, 3)
    up = -gate - 1
    w = torch_path.interleave_gate_up(gate, up)
    assert w.shape == (96, 3)
    for j in range(3):
        assert torch.equal(w[32 * j:32 * j + 16], gate[16 * j:16 * j + 16])
        assert torch.equal(w[32 * j + 16:32 * j + 32], up[16 * j:16 * j + 16])
    x = torch.randn(5, 3)
    g, u = torch_path.split_gate_up(x @ w.t())
    torch.testing.assert_close(g, x @ gate.t(), rtol=0, atol=0)
    torch.testing.assert_close(u, x @ up.t(), rtol=0, atol=0)
    with pytest.raises(ValueError):
        torch_path.interleave_gate_up(gate[:40], up[:40])


def test_fused_projection_torch_paths():
    """The fused projections' PyTorch paths equal the unfused ops they replace."""
    x = torch.randn(6, 64)
    wq, wk, wv = torch.randn(64, 64), torch.randn(32, 64), torch.randn(32, 64)
    qkv = ops.pack_weight(torch.cat((wq, wk, wv)))
    assert qkv.packed is None  # no kernel on the PyTorch path
    q, k, v = ops.linear_split(x, qkv, (64, 32, 32))
    for got, w in ((q, wq), (k, wk), (v, wv)):
        assert got.is_contiguous()
        torch.testing.assert_close(got, x @ w.t())
    r = torch.randn(6, 48)
    wo = ops.pack_weight(torch.randn(48, 64))
    torch.testing.assert_close(ops.linear_residual(x, wo, r), r + x @ wo.dense.t())
    torch.testing.assert_close(ops.linear(x, wo), x @ wo.dense.t())
    gate, up = torch.randn(32, 64), torch.randn(32, 64)
    torch.testing.assert_close(
        ops.linear_swiglu(x, ops.pack_weight(torch_path.interleave_gate_up(gate, up))),
        ops.swiglu(x @ gate.t(), x @ up.t()))
    assert not ops.skinny(x, use_cuda=False)
    assert torch.equal(ops.linear_residual(x, wo, r, use_cuda=True), r + x @ wo.dense.t())
    with ops.strict_kernels(), pytest.raises(RuntimeError, match="device tensors"):
        ops.linear_residual(x, wo, r, use_cuda=True)


def test_pack_fragments_layout():
    """Piece (t, s, l = 32 h + r) of the packed weight is w[32 t + r, 16 s + 8 h : +8],
    rows past N zero; checked element by element against that definition."""
    n, k = 45, 64
    w = torch.arange(n * k, dtype=torch.float32).view(n, k) + 1
    packed = torch_path.pack_fragments(w).view(-1, 64, 8)
    steps = k // 16
    assert packed.shape[0] == 2 * steps
    for t in range(2):
        for s in range(steps):
            for l in range(64):
                r, h = 32 * t + l % 32, l // 32
                want = w[r, 16 * s + 8 * h:16 * s + 8 * h + 8] if r < n else torch.zeros(8)
                assert torch.equal(packed[t * steps + s, l], want), (t, s, l)


def test_add_rmsnorm_torch_path():
    x, r = torch.randn(3, 64), torch.randn(3, 64)
    w = torch.rand(64) + 0.5
    h, n = ops.add_rmsnorm(x, r, w)
    torch.testing.assert_close(h, r + x, rtol=0, atol=0)
    torch.testing.assert_close(n, ops.rmsnorm(r + x, w), rtol=0, atol=0)
    h2, n2 = ops.add_rmsnorm(x, r, w, use_cuda=True)
    assert torch.equal(h2, h) and torch.equal(n2, n)
    with ops.strict_kernels(), pytest.raises(RuntimeError, match="needs device tensors"):
        ops.add_rmsnorm(x, r, w, use_cuda=True)
