"""The allocation-free paged-attention entry (``mvllm_paged_attention_noalloc``) through
the C ABI: its output equals the workspace entry's (``mvllm_paged_attention``) bit for
bit on the same inputs and plan, on consecutive calls that share the library's static
scratch (the second smaller, so it starts on the first call's leftovers), and a plan
that needs more scratch than the library holds is refused before any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from mini_vllm.kernels.extension import DTYPE_CODES, make_plan_options
from mini_vllm.workloads import build_batch

pytestmark = pytest.mark.gpu


def _noalloc(ext, b, out, options=None):
    _, bs, hk, d = b.key_pool.shape
    opts = make_plan_options(options)
    stream = torch.cuda.current_stream().cuda_stream
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = ext.lib.mvllm_paged_attention_noalloc(
        out.data_ptr(), b.q.data_ptr(), b.key_pool.data_ptr(), b.value_pool.data_ptr(),
        ptr(b.k_scale), ptr(b.v_scale), b.block_tables.data_ptr(), b.cu_seqlens_q.data_ptr(),
        b.context_lens.data_ptr(), b.seq_lens.data_ptr(), b.q.shape[0], len(b.contexts),
        b.q.shape[1], hk, d, bs, b.key_pool.shape[0], b.block_tables.shape[1],
        b.max_query_len, b.max_context_len, b.scale, DTYPE_CODES[b.q.dtype],
        DTYPE_CODES[b.key_pool.dtype], None if opts is None else ctypes.byref(opts), stream)
    return rc


def _both(ext, b, options=None):
    want = ext.paged_attention(*b.args(), k_scale=b.k_scale, v_scale=b.v_scale,
                               plan_options=options)
    got = torch.full_like(want, float("nan"))
    rc = _noalloc(ext, b, got, options)
    assert rc == 0, ext.lib.mvllm_last_error().decode()
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("kv_dtype", [None, torch.float8_e4m3fn], ids=["bf16", "fp8"])
def test_noalloc_equals_the_workspace_entry_on_two_calls(extension, device, kv_dtype):
    big = build_batch([4096, 3000, 513, 17, 2048] * 6, [1] * 30, dtype=torch.bfloat16,
                      kv_dtype=kv_dtype, num_q_heads=16, num_kv_heads=8, head_dim=128, seed=21,
                      device=device)
    got, want = _both(extension, big)
    assert torch.equal(got, want)
    small = build_batch([700, 33, 90], [1, 1, 1], dtype=torch.bfloat16, kv_dtype=kv_dtype,
                        num_q_heads=16, num_kv_heads=8, head_dim=128, seed=22, device=device)
    got, want = _both(extension, small)
    assert torch.equal(got, want)


def test_noalloc_mixed_batch_with_the_grid_prefill(extension, device):
    """Decodes beside prefill chunks: the prefill on the grid schedule with every item
    whole (no scratch), the decode partials in the static array; then a smaller
    decode-only call. With the planner's defaults the workspace entry may cut long items
    into pieces whose partials do not fit the static scratch: the allocation-free entry
    then keeps its items whole, the same result as the workspace entry asked for whole
    items, and within the bf16 tolerance of the cut run."""
    b = build_batch([1500, 700, 64, 300], [1, 300, 64, 1], dtype=torch.bfloat16,
                    num_q_heads=16, num_kv_heads=8, head_dim=128, seed=23, device=device)
    whole = {"prefill_schedule": "grid", "prefill_pieces": 1}
    got, want = _both(extension, b, whole)
    assert torch.equal(got, want)
    cut = extension.paged_attention(*b.args(), plan_options={"prefill_schedule": "grid"})
    default = torch.full_like(cut, float("nan"))
    assert _noalloc(extension, b, default, {"prefill_schedule": "grid"}) == 0
    torch.cuda.synchronize()
    assert torch.equal(default, want)
    assert (cut.float() - want.float()).abs().max().item() <= 2e-2
    small = build_batch([40, 5], [1, 1], dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8,
                        head_dim=128, seed=24, device=device)
    got, want = _both(extension, small)
    assert torch.equal(got, want)


def test_noalloc_refuses_a_plan_larger_than_its_scratch(extension, device):
    b = build_batch([4000], [512], dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8,
                    head_dim=128, seed=25, device=device)
    plan = extension.paged_attention_plan(512, 1, 16, 8, 128, 16, 512, 4000, torch.bfloat16,
                                          torch.bfloat16, plan_options={"prefill_schedule": "stream"})
    assert plan["workspace_bytes"] > 16 << 20
    out = torch.zeros_like(b.q)
    rc = _noalloc(extension, b, out, {"prefill_schedule": "stream"})
    assert rc == 2 and "scratch" in extension.lib.mvllm_last_error().decode()
    torch.cuda.synchronize()
    assert not out.any()  # refused before any launch
