"""Decode attention that forms the step's new token itself
(``mvllm_paged_decode_qk_norm_rope``, ``csrc/paged_decode.hip``) on the MI355X (``-m gpu``).

The entry replaces, for a decode-only batch, the pair the model would otherwise call:
``qk_norm_rope_kv_write`` (positions ``context_lens - 1``, each sequence's slot from its
block table) and then ``paged_attention`` over the rotated q. Checked here:

* bitwise equality with that pair, the attention output and both pools (the new
  token's K and V at their slots, every other byte untouched), over the stream
  schedule's cases: a context of one key (the new token alone), page boundaries, one
  long sequence cut into many workgroup shares (the new token in the last), many short
  sequences sharing workgroups, every GQA chunking (one, two or four query heads per
  wave; two waves per kv head when a group has eight heads), f16 and bf16, column views
  of a fused projection output, more workgroups per CU;
* the oracle chain: ``oracle/elementwise.py`` rms_norm -> apply_rope for q and k, the K/V
  write by slot, then ``oracle/paged_attention.py``, at the attention tolerance;
* refusals (host-side, no launch) and the op seam's routing.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATTN_ATOL, assert_max_abs
from mini_vllm import torch_path
from mini_vllm.kernels import ops
from mini_vllm.workloads import build_batch
from oracle import elementwise as ew
from oracle.paged_attention import paged_attention as oracle_paged

pytestmark = pytest.mark.gpu

EPS = 1e-6
MAX_POS = 16384


def _slots(b) -> torch.Tensor:
    """Slot of each sequence's last position, from its block table."""
    ctx = b.context_lens.cpu().long()
    tables = b.block_tables.cpu().long()
    bs = b.key_pool.shape[1]
    pos = ctx - 1
    page = tables[torch.arange(len(ctx)), pos // bs]
    return (page * bs + pos % bs).to(torch.int32)


def _case(contexts, hq, hk, dtype, device, seed, views=True):
    b = build_batch(contexts, [1] * len(contexts), dtype=dtype, num_q_heads=hq,
                    num_kv_heads=hk, head_dim=128, seed=seed, device=device)
    s, d = len(contexts), 128
    gen = torch.Generator().manual_seed(seed + 1)
    proj = (torch.randn(s, (hq + 2 * hk) * d, generator=gen) * 3).to(dtype).to(device)
    q, k, v = proj.split([hq * d, hk * d, hk * d], dim=-1)
    q, k, v = q.view(s, hq, d), k.view(s, hk, d), v.view(s, hk, d)
    if not views:
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    wq = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    wk = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    return b, q, k, v, wq, wk


def _pair(ext, b, q, k, v, wq, wk, cos, sin, options=None):
    pk, pv = b.key_pool.clone(), b.value_pool.clone()
    pos = (b.context_lens - 1).long()
    q_rot = ext.qk_norm_rope_kv_write(q, k, v, wq, wk, pos, cos, sin, EPS, pk, pv,
                                      _slots(b).to(q.device))
    out = ext.paged_attention(q_rot, pk, pv, b.block_tables, b.cu_seqlens_q, b.context_lens,
                              b.seq_lens, 1, b.max_context_len, b.scale, plan_options=options)
    return out, pk, pv


def _fused(ext, b, q, k, v, wq, wk, cos, sin, options=None):
    pk, pv = b.key_pool.clone(), b.value_pool.clone()
    out = ext.paged_decode_qk_norm_rope(q, k, v, wq, wk, cos, sin, EPS, pk, pv, b.block_tables,
                                        b.cu_seqlens_q, b.context_lens, b.seq_lens,
                                        b.max_context_len, b.scale, plan_options=options)
    return out, pk, pv


CASES = {
    "one_key": [1],
    "boundaries": [1, 15, 16, 17, 63, 64, 65, 200],
    "config5_like": [900 + (37 * i) % 400 for i in range(32)],
    "one_long": [8192],
    "many_short": [1 + (13 * i) % 50 for i in range(300)],
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", list(CASES))
def test_is_bitwise_the_unfused_pair(extension, device, dtype, name):
    contexts = CASES[name]
    b, q, k, v, wq, wk = _case(contexts, 16, 8, dtype, device, seed=len(contexts) + 5)
    cos, sin = torch_path.rope_tables(128, MAX_POS, device=device)
    want, wk_pool, wv_pool = _pair(extension, b, q, k, v, wq, wk, cos, sin)
    got, gk_pool, gv_pool = _fused(extension, b, q, k, v, wq, wk, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got.float() - want.float()).abs().max().item()
    assert torch.equal(gk_pool, wk_pool) and torch.equal(gv_pool, wv_pool)
    assert not torch.equal(gk_pool, b.key_pool)  # the new keys were written


@pytest.mark.parametrize("hq,hk", [(8, 8), (16, 8), (32, 8), (32, 4), (6, 2)])
def test_every_query_head_chunking(extension, device, hq, hk):
    """One, two or four query heads per wave (groups of 1, 2, 4, 8 and 3); a group of
    eight heads runs two waves per kv head, of which one writes the pool."""
    contexts = [1 + (97 * i) % 700 for i in range(24)]
    b, q, k, v, wq, wk = _case(contexts, hq, hk, torch.bfloat16, device, seed=hq * hk)
    cos, sin = torch_path.rope_tables(128, MAX_POS, device=device)
    want, wk_pool, wv_pool = _pair(extension, b, q, k, v, wq, wk, cos, sin)
    got, gk_pool, gv_pool = _fused(extension, b, q, k, v, wq, wk, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(gk_pool, wk_pool) and torch.equal(gv_pool, wv_pool)


@pytest.mark.parametrize("wgs_per_cu", [1, 3])
def test_contiguous_inputs_and_more_workgroups(extension, device, wgs_per_cu):
    contexts = [1 + (211 * i) % 3000 for i in range(40)]
    b, q, k, v, wq, wk = _case(contexts, 16, 8, torch.bfloat16, device, seed=77, views=False)
    cos, sin = torch_path.rope_tables(128, MAX_POS, device=device)
    opts = {"decode_wgs_per_cu": wgs_per_cu}
    want, wk_pool, wv_pool = _pair(extension, b, q, k, v, wq, wk, cos, sin, opts)
    got, gk_pool, gv_pool = _fused(extension, b, q, k, v, wq, wk, cos, sin, opts)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(gk_pool, wk_pool) and torch.equal(gv_pool, wv_pool)


@pytest.mark.parametrize("name", ["boundaries", "config5_like"])
def test_against_the_oracle_chain(extension, device, name):
    """QK-norm + RoPE of q and k by the numpy oracle (bf16 rounding points), k and v
    written to a copy of the pool at the oracle's slots, then the fp32 paged oracle:
    the fused output within the bf16 attention tolerance, its pools within two storage
    ulps of the oracle's rows (the norm's fp32 sum order may move one rounding)."""
    contexts = CASES[name]
    b, q, k, v, wq, wk = _case(contexts, 16, 8, torch.bfloat16, device, seed=11)
    cos, sin = torch_path.rope_tables(128, MAX_POS, device=device)
    got, gk_pool, gv_pool = _fused(extension, b, q, k, v, wq, wk, cos, sin)
    torch.cuda.synchronize()

    pos = (b.context_lens - 1).long().cpu().numpy()
    cos_np, sin_np = cos.cpu().numpy(), sin.cpu().numpy()

    def norm_rope(x, w):
        n = ew.rms_norm(x.float().cpu().numpy(), w.float().cpu().numpy(), EPS, "bf16")
        return ew.apply_rope(n[None], pos, cos_np, sin_np, "bf16")[0]

    q_rot, k_rot = norm_rope(q, wq), norm_rope(k, wk)
    slots = _slots(b).long()
    bs, hk = b.key_pool.shape[1], b.key_pool.shape[2]
    kp = b.key_pool.float().cpu().reshape(-1, hk, 128).clone()
    vp = b.value_pool.float().cpu().reshape(-1, hk, 128).clone()
    kp[slots] = torch.from_numpy(k_rot).float()
    vp[slots] = v.float().cpu()
    want = oracle_paged(torch.from_numpy(q_rot).float(), kp.reshape(-1, bs, hk, 128),
                        vp.reshape(-1, bs, hk, 128), b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale)
    assert_max_abs(got, want, ATTN_ATOL[torch.bfloat16], name)
    written = gk_pool.float().cpu().reshape(-1, hk, 128)[slots].numpy()
    err = np.abs(written - k_rot)
    assert np.all(err <= np.maximum(np.abs(k_rot), 2.0**-6) * 2.0**-7 * 2), err.max()
    assert torch.equal(gv_pool.cpu().reshape(-1, hk, 128)[slots], v.cpu())


def test_refusals_before_launch(extension, device):
    contexts = [5, 40, 17]
    b, q, k, v, wq, wk = _case(contexts, 16, 8, torch.bfloat16, device, seed=3)
    cos, sin = torch_path.rope_tables(128, 512, device=device)
    before_k, before_v = b.key_pool.clone(), b.value_pool.clone()
    call = extension.paged_decode_qk_norm_rope
    args = (b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q, b.context_lens,
            b.seq_lens, b.max_context_len, b.scale)
    with pytest.raises(RuntimeError, match="grid schedule"):
        call(q, k, v, wq, wk, cos, sin, EPS, *args, plan_options={"decode_schedule": 2})
    with pytest.raises(RuntimeError, match="one token per sequence"):
        call(q[:2], k[:2], v[:2], wq, wk, cos, sin, EPS, *args)
    with pytest.raises(RuntimeError, match="cos/sin tables"):
        call(q, k, v, wq, wk, cos[:, :64], sin[:, :64], EPS, *args)
    with pytest.raises(RuntimeError, match="weights must be"):
        call(q, k, v, wq[:64], wk, cos, sin, EPS, *args)
    torch.cuda.synchronize()
    assert torch.equal(b.key_pool, before_k) and torch.equal(b.value_pool, before_v)


def test_op_seam_routes_and_declines(extension, device):
    """ops.paged_decode_qk_norm_rope runs the fused launch for a 16-bit pool (the same
    bits as the extension call) and returns None for what it does not serve: an fp8
    pool, another head dim, the PyTorch path."""
    contexts = [30, 300, 1]
    b, q, k, v, wq, wk = _case(contexts, 16, 8, torch.bfloat16, device, seed=9)
    cos, sin = torch_path.rope_tables(128, 1024, device=device)
    want, _, _ = _fused(extension, b, q, k, v, wq, wk, cos, sin)
    pk, pv = b.key_pool.clone(), b.value_pool.clone()
    got = ops.paged_decode_qk_norm_rope(q, k, v, wq, wk, cos, sin, EPS, pk, pv, b.block_tables,
                                        b.cu_seqlens_q, b.context_lens, b.seq_lens,
                                        b.max_context_len, b.scale, use_cuda=True)
    torch.cuda.synchronize()
    assert got is not None and torch.equal(got, want)
    fp8 = b.key_pool.to(torch.float8_e4m3fn)
    assert ops.paged_decode_qk_norm_rope(q, k, v, wq, wk, cos, sin, EPS, fp8, fp8.clone(),
                                         b.block_tables, b.cu_seqlens_q, b.context_lens,
                                         b.seq_lens, b.max_context_len, b.scale,
                                         use_cuda=True) is None
    assert ops.paged_decode_qk_norm_rope(q, k, v, wq, wk, cos, sin, EPS, pk, pv, b.block_tables,
                                         b.cu_seqlens_q, b.context_lens, b.seq_lens,
                                         b.max_context_len, b.scale, use_cuda=False) is None


@pytest.mark.parametrize("contexts", [[700], [64, 1000, 2500]], ids=["one", "three"])
def test_a_spike_on_the_new_token(extension, device, contexts):
    """The reference's late-spike known answer (tests/test_decode_attention_cuda.py:85-109)
    placed on the key formed inside the launch: each sequence's new k is its q's first
    head, norm weights of 8 make that score ~64 / sqrt(128) x 8 above the rest, so every
    accumulator is rescaled on the last key and the output is ~ that token's v. Bitwise
    the unfused pair, and within the bf16 tolerance of the oracle chain."""
    b, q, k, v, wq, wk = _case(contexts, 16, 8, torch.bfloat16, device, seed=5)
    k[:, :, :] = q[:, 0:1, :]  # the new key points along query head 0 (every kv head)
    wq = torch.full_like(wq, 8.0)
    wk = torch.full_like(wk, 8.0)
    cos, sin = torch_path.rope_tables(128, MAX_POS, device=device)
    want, wk_pool, wv_pool = _pair(extension, b, q, k, v, wq, wk, cos, sin)
    got, gk_pool, gv_pool = _fused(extension, b, q, k, v, wq, wk, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(gk_pool, wk_pool) and torch.equal(gv_pool, wv_pool)
    # query head 0 of each sequence attends (almost) only to the new token: its output
    # is that token's v row of kv head 0
    assert_max_abs(got[:, 0, :], v[:, 0, :].float(), 2e-2, "spike")
