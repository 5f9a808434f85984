"""Paged KV write kernel (``csrc/kv_write.hip``) on the MI355X, through the C ABI, against
the CPU oracle (oracle/kv_write.py): bit-exact bytes and scales (``-m gpu``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mini_vllm.kernels import ops
from oracle import kv_write as ow

pytestmark = pytest.mark.gpu


def _rand_slots(rng, num_blocks, bs, t, pad=0):
    s = rng.choice(num_blocks * bs, size=t, replace=False).astype(np.int32)
    s = np.concatenate([s, -np.ones(pad, dtype=np.int32)])
    rng.shuffle(s)
    return s


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hk,d", [(8, 128), (2, 64), (3, 20)])
def test_copy_is_the_reference_index_copy(extension, device, dtype, hk, d):
    """Same-dtype pools: bit-exact scatter, padding slots (-1) skipped; (3, 20) rows are
    not a multiple of 16 bytes in 16-bit types and take the per-element kernel."""
    rng = np.random.default_rng(hk * d)
    nb, bs, t = 40, 16, 300
    pool_k = torch.randn(nb, bs, hk, d).to(dtype)
    pool_v = torch.randn(nb, bs, hk, d).to(dtype)
    slots = _rand_slots(rng, nb, bs, t, pad=7)
    key = torch.randn(t + 7, hk, d).to(dtype)
    value = torch.randn(t + 7, hk, d).to(dtype)
    want_k = ow.kv_write_copy(pool_k.float().numpy(), slots, key.float().numpy())
    want_v = ow.kv_write_copy(pool_v.float().numpy(), slots, value.float().numpy())
    gk, gv = pool_k.to(device), pool_v.to(device)
    extension.kv_write(gk, gv, key.to(device), value.to(device), torch.from_numpy(slots).to(device))
    torch.cuda.synchronize()
    assert np.array_equal(gk.float().cpu().numpy(), want_k)
    assert np.array_equal(gv.float().cpu().numpy(), want_v)


def _scenario(rng, hk, d, bs):
    """A prefill chunk over 2.5 blocks of one sequence plus 5 rows of another, then decode
    steps (with a padding row) whose magnitudes grow, so scales grow and rows already in
    a block are re-encoded; the last step reopens a freed block at row 0."""
    seq_a = [5 * bs + i for i in range(bs)] + [9 * bs + i for i in range(bs)] + \
            [2 * bs + i for i in range(bs // 2)]
    seq_b = [11 * bs + i for i in range(min(5, bs))]
    steps = [np.array(seq_a + seq_b, np.int32)]
    for k in range(6):
        row_a = bs // 2 + k
        a = 2 * bs + row_a if row_a < bs else 3 * bs + row_a - bs
        row_b = min(5, bs) + k
        b = 11 * bs + row_b if row_b < bs else 12 * bs + row_b - bs
        steps.append(np.array([a, b, -1], np.int32))
    steps.append(np.array([9 * bs, 9 * bs + 1], np.int32))
    xs = [(rng.standard_normal((len(s), hk, d)) * (1.0 + 0.7 * i)).astype(np.float32)
          for i, s in enumerate(steps)]
    return steps, xs


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("hk,d,bs", [(8, 128, 16), (2, 64, 16), (4, 256, 4), (2, 128, 1), (2, 32, 16)])
def test_fp8_write_matches_the_oracle_bytes(extension, device, src, hk, d, bs):
    rng = np.random.default_rng(d + bs)
    nb = 16
    steps, xs = _scenario(rng, hk, d, bs) if bs > 1 else (
        [np.array([3, 4, 9, -1, 12], np.int32), np.array([5, 3], np.int32)],
        [rng.standard_normal((5, hk, d)).astype(np.float32),
         rng.standard_normal((2, hk, d)).astype(np.float32) * 3])
    codes_k = np.zeros((nb, bs, hk, d), np.uint8)
    scales_k = np.zeros((nb, hk), np.float32)
    codes_v, scales_v = codes_k.copy(), scales_k.copy()
    kp = torch.zeros(nb, bs, hk, d, dtype=torch.float8_e4m3fn, device=device)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(nb, hk, device=device)
    vs = torch.zeros(nb, hk, device=device)
    for sl, x in zip(steps, xs):
        key = torch.from_numpy(x).to(src)
        value = (torch.from_numpy(x) * 0.5 + 0.25).to(src)
        codes_k, scales_k = ow.kv_write_fp8(codes_k, scales_k, sl, key.float().numpy())
        codes_v, scales_v = ow.kv_write_fp8(codes_v, scales_v, sl, value.float().numpy())
        extension.kv_write(kp, vp, key.to(device), value.to(device),
                           torch.from_numpy(sl).to(device), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert np.array_equal(ks.cpu().numpy(), scales_k)
    assert np.array_equal(vs.cpu().numpy(), scales_v)
    assert np.array_equal(kp.view(torch.uint8).cpu().numpy(), codes_k)
    assert np.array_equal(vp.view(torch.uint8).cpu().numpy(), codes_v)


def _large_fp8_call(rng, nb, bs, t):
    """Slots of one large call: sequences of 1..300 tokens (single-token ones are decode
    steps) on consecutive rows of their own pages, each starting at the row its page's
    history ends on (or at row 0 of a fresh page), with -1 padding between some; and
    the history call that partly filled those pages."""
    pages = rng.permutation(nb).tolist()
    hist, slots = [], []
    while len(slots) < t:
        n = int(rng.integers(1, 4)) if rng.random() < 0.3 else int(rng.integers(5, 300))
        n = min(n, t - len(slots))
        need = -(-(n + bs) // bs)
        if len(pages) < need:
            break
        own = [pages.pop() for _ in range(need)]
        start = int(rng.integers(0, bs))  # rows already written by the history call
        hist += [own[0] * bs + r for r in range(start)]
        rows = [own[(start + i) // bs] * bs + (start + i) % bs for i in range(n)]
        slots += rows
        if rng.random() < 0.2 and len(slots) < t:
            slots.append(-1)
    slots = slots[:t] + [-1] * (t - len(slots[:t]))
    return np.array(hist, np.int32), np.array(slots, np.int32)


@pytest.mark.parametrize("t", [2048, 3000, 4096, 70000])
def test_fp8_write_large_calls_match_the_oracle_bytes(extension, device, t):
    """Calls large enough that a workgroup takes several tokens (8 at 2048, 11 at 3000,
    16 at 4096 and 70000; at 2048 and 4096 the grid is a multiple of 8 and the windows go
    to the XCDs in eighths): runs start anywhere in a workgroup's tokens and cross into
    the next one's, pages are
    continued mid-way under a grown or kept scale, decode-like single tokens sit among
    long chunks; bytes and scales equal the oracle's. The same call with padding slots
    replaced by slots past the pool leaves the same pool."""
    rng = np.random.default_rng(t)
    hk, d, bs = 2, 32, 16
    nb = t // bs * 3
    hist, slots = _large_fp8_call(rng, nb, bs, t)
    codes_k = np.zeros((nb, bs, hk, d), np.uint8)
    scales_k = np.zeros((nb, hk), np.float32)
    codes_v, scales_v = codes_k.copy(), scales_k.copy()
    kp = torch.zeros(nb, bs, hk, d, dtype=torch.float8_e4m3fn, device=device)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(nb, hk, device=device)
    vs = torch.zeros(nb, hk, device=device)
    for step, sl in enumerate((hist, slots)):
        x = (rng.standard_normal((len(sl), hk, d)) * (1.0 + step)).astype(np.float32)
        key = torch.from_numpy(x).to(torch.bfloat16)
        value = (torch.from_numpy(x) * 0.5 + 0.25).to(torch.bfloat16)
        codes_k, scales_k = ow.kv_write_fp8(codes_k, scales_k, sl, key.float().numpy())
        codes_v, scales_v = ow.kv_write_fp8(codes_v, scales_v, sl, value.float().numpy())
        if step == 1:
            before = [a.clone() for a in (kp, vp, ks, vs)]
        extension.kv_write(kp, vp, key.to(device), value.to(device),
                           torch.from_numpy(sl).to(device), k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert np.array_equal(ks.cpu().numpy(), scales_k)
    assert np.array_equal(vs.cpu().numpy(), scales_v)
    assert np.array_equal(kp.view(torch.uint8).cpu().numpy(), codes_k)
    assert np.array_equal(vp.view(torch.uint8).cpu().numpy(), codes_v)
    bad = slots.copy()
    bad[bad < 0] = nb * bs + np.arange((bad < 0).sum(), dtype=np.int32)
    kp2, vp2, ks2, vs2 = before
    extension.kv_write(kp2, vp2, key.to(device), value.to(device),
                       torch.from_numpy(bad).to(device), k_scale=ks2, v_scale=vs2)
    torch.cuda.synchronize()
    assert torch.equal(kp2.view(torch.uint8), kp.view(torch.uint8))
    assert torch.equal(vp2.view(torch.uint8), vp.view(torch.uint8))
    assert torch.equal(ks2, ks) and torch.equal(vs2, vs)


def test_fp8_encoding_is_round_to_nearest_even(extension, device):
    """Every e4m3 code's value and every midpoint between neighbours (ties go to the
    even code), written at scale 1 (a block whose max is 448 -> scale pow2ceil(1) = 1)."""
    from oracle.elementwise import fp8_e4m3_decode, fp8_e4m3_encode
    vals = fp8_e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    x = np.concatenate([vals, mids, -vals, -mids, [448.0]]).astype(np.float32)
    n = x.size
    d = 128
    rows = -(-n // d)
    flat = np.zeros(rows * d, np.float32)
    flat[:n] = x
    flat[n:] = 448.0
    data = flat.reshape(rows, 1, d)
    kp = torch.zeros(1, rows, 1, d, dtype=torch.float8_e4m3fn, device=device)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(1, 1, device=device)
    vs = torch.zeros(1, 1, device=device)
    xt = torch.from_numpy(data).to(device)
    extension.kv_write(kp, vp, xt, xt, torch.arange(rows, dtype=torch.int32, device=device),
                       k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert float(ks[0, 0]) == 1.0
    got = kp.view(torch.uint8).cpu().numpy().reshape(-1)[:n]
    want = fp8_e4m3_encode(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:8]]


def test_ops_route_kv_write_to_the_kernel(extension, device):
    pool = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16, device=device)
    pool_v = torch.zeros_like(pool)
    x = torch.randn(3, 2, 64, dtype=torch.bfloat16, device=device)
    slots = torch.tensor([17, 18, 40], dtype=torch.int32, device=device)
    ops.kv_write(pool, pool_v, x, x, slots, use_cuda=True)
    assert torch.equal(pool.view(-1, 2, 64)[17], x[0]) and torch.equal(pool.view(-1, 2, 64)[40], x[2])
    with pytest.raises(RuntimeError, match="device tensors"):
        ops.kv_write(pool.cpu(), pool_v.cpu(), x.cpu(), x.cpu(), slots.cpu(), use_cuda=True)


def test_kv_write_refusals(extension, device):
    pool = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16, device=device)
    x = torch.randn(3, 2, 64, dtype=torch.bfloat16, device=device)
    slots = torch.tensor([1, 2, 3], dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError, match="share the keys' dtype"):
        extension.kv_write(pool.half(), pool.half(), x, x, slots)
    with pytest.raises(RuntimeError, match="int32"):
        extension.kv_write(pool, pool.clone(), x, x, slots.long())
    with pytest.raises(RuntimeError, match="shaped"):
        extension.kv_write(pool, pool.clone(), x[:, :1], x[:, :1], slots)
    fp8 = pool.to(torch.float8_e4m3fn)
    with pytest.raises(RuntimeError, match="k_scale"):
        extension.kv_write(fp8, fp8.clone(), x, x, slots)
    with pytest.raises(RuntimeError, match="float8 pools only"):
        extension.kv_write(pool, pool.clone(), x, x, slots, k_scale=torch.zeros(4, 2, device=device))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hk,d,t", [(16, 8, 128, 200), (4, 2, 64, 200), (8, 1, 256, 200),
                                       (16, 8, 128, 3000), (6, 2, 128, 2500)])
def test_qk_norm_rope_kv_write_is_the_unfused_sequence(extension, device, dtype, hq, hk, d, t):
    """QK-norm + RoPE with the pool write in one launch: q bitwise the fused
    qk_norm_rope's, and both pools bitwise what qk_norm_rope then kv_write leave (the
    rotated k and the raw v at their slots, -1 slots and the rest of the pool untouched).
    The larger calls take several heads of a token per lane group."""
    from mini_vllm.torch_path import rope_tables

    rng = np.random.default_rng(hq * d + t)
    bs = 16
    nb = max(30, t // bs + 40)
    gen = torch.Generator().manual_seed(hq + d)
    q = torch.randn(t + 5, hq, d, generator=gen).to(dtype).to(device)
    k = torch.randn(t + 5, hk, d, generator=gen).to(dtype).to(device)
    v = torch.randn(t + 5, hk, d, generator=gen).to(dtype).to(device)
    wq = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    wk = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    cos, sin = rope_tables(d, 4096, device=device)
    pos = torch.from_numpy(rng.integers(0, 4096, size=t + 5)).to(device)
    slots = torch.from_numpy(_rand_slots(rng, nb, bs, t, pad=5)).to(device)
    pool_k = torch.randn(nb, bs, hk, d, generator=gen).to(dtype).to(device)
    pool_v = torch.randn(nb, bs, hk, d, generator=gen).to(dtype).to(device)
    want_k, want_v = pool_k.clone(), pool_v.clone()
    q_ref, k_ref = extension.qk_norm_rope(q, k, wq, wk, pos, cos, sin, 1e-6)
    extension.kv_write(want_k, want_v, k_ref, v, slots)
    q_got = extension.qk_norm_rope_kv_write(q, k, v, wq, wk, pos, cos, sin, 1e-6, pool_k, pool_v, slots)
    torch.cuda.synchronize()
    assert torch.equal(q_got, q_ref)
    assert torch.equal(pool_k, want_k) and torch.equal(pool_v, want_v)
    q_ops = ops.qk_norm_rope_kv_write(q, k, v, wq, wk, pos, cos, sin, 1e-6, pool_k, pool_v, slots,
                                      use_cuda=True)
    assert q_ops is not None and torch.equal(q_ops, q_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hq,hk,d", [(16, 8, 128), (6, 2, 64)])
def test_qk_norm_rope_kv_write_reads_column_views(extension, device, dtype, hq, hk, d):
    """q, k, v as column views of one fused q/k/v projection output (token stride the
    projection's width, the prefill path): every output bitwise the call on contiguous
    copies, with no copy made."""
    from mini_vllm.torch_path import rope_tables

    rng = np.random.default_rng(7 * hq + d)
    nb, bs, t = 20, 16, 150
    gen = torch.Generator().manual_seed(3 * hq + d)
    width = (hq + 2 * hk) * d
    fused = torch.randn(t, width, generator=gen).to(dtype).to(device)
    q, k, v = fused.split([hq * d, hk * d, hk * d], dim=-1)
    q, k, v = q.view(t, hq, d), k.view(t, hk, d), v.view(t, hk, d)
    assert not q.is_contiguous() and q.stride(0) == width
    wq = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    wk = (torch.rand(d, generator=gen) + 0.5).to(dtype).to(device)
    cos, sin = rope_tables(d, 2048, device=device)
    pos = torch.from_numpy(rng.integers(0, 2048, size=t)).to(device)
    slots = torch.from_numpy(_rand_slots(rng, nb, bs, t - 4, pad=4)).to(device)
    pool_k = torch.randn(nb, bs, hk, d, generator=gen).to(dtype).to(device)
    pool_v = torch.randn(nb, bs, hk, d, generator=gen).to(dtype).to(device)
    want_k, want_v = pool_k.clone(), pool_v.clone()
    q_want = extension.qk_norm_rope_kv_write(q.contiguous(), k.contiguous(), v.contiguous(), wq,
                                             wk, pos, cos, sin, 1e-6, want_k, want_v, slots)
    q_got = extension.qk_norm_rope_kv_write(q, k, v, wq, wk, pos, cos, sin, 1e-6, pool_k, pool_v,
                                            slots)
    torch.cuda.synchronize()
    assert torch.equal(q_got, q_want)
    assert torch.equal(pool_k, want_k) and torch.equal(pool_v, want_v)


def test_qk_norm_rope_kv_write_leaves_fp8_pools_to_the_two_ops(extension, device):
    """An fp8 pool (quantised with per-block scales) is not written by the fused launch:
    ops returns None and the caller runs qk_norm_rope then kv_write."""
    from mini_vllm.torch_path import rope_tables

    q = torch.randn(4, 16, 128, dtype=torch.bfloat16, device=device)
    k = torch.randn(4, 8, 128, dtype=torch.bfloat16, device=device)
    w = torch.ones(128, dtype=torch.bfloat16, device=device)
    cos, sin = rope_tables(128, 64, device=device)
    pool = torch.zeros(4, 16, 8, 128, dtype=torch.float8_e4m3fn, device=device)
    slots = torch.arange(4, dtype=torch.int32, device=device)
    pos = torch.arange(4, device=device)
    assert ops.qk_norm_rope_kv_write(q, k, k, w, w, pos, cos, sin, 1e-6, pool, pool, slots,
                                     use_cuda=True) is None


def test_qk_norm_rope_kv_write_refuses_mismatched_shapes_before_launch(extension, device):
    """The fused write takes q's token count for k, v and the slots and reads the tables
    at pos x D, so every shape it relies on is checked on the host (no launch)."""
    from mini_vllm.torch_path import rope_tables

    bf = dict(dtype=torch.bfloat16, device=device)
    q, k, v = (torch.randn(6, h, 128, **bf) for h in (16, 8, 8))
    w = torch.ones(128, **bf)
    cos, sin = rope_tables(128, 64, device=device)
    pool = torch.zeros(4, 16, 8, 128, **bf)
    slots = torch.arange(6, dtype=torch.int32, device=device)
    pos = torch.arange(6, device=device)
    before = pool.clone()
    call = extension.qk_norm_rope_kv_write
    with pytest.raises(RuntimeError, match="T x H_q x D"):
        call(q, k[:4], v[:4], w, w, pos, cos, sin, 1e-6, pool, pool.clone(), slots)
    with pytest.raises(RuntimeError, match="cos/sin tables"):
        call(q, k, v, w, w, pos, cos[:, :64], sin[:, :64], 1e-6, pool, pool.clone(), slots)
    with pytest.raises(RuntimeError, match="weights must be"):
        call(q, k, v, w[:64], w, pos, cos, sin, 1e-6, pool, pool.clone(), slots)
    with pytest.raises(RuntimeError, match="T x H_q x D"):
        call(q.view(6, 16 * 128), k, v, w, w, pos, cos, sin, 1e-6, pool, pool.clone(), slots)
    with pytest.raises(RuntimeError, match="slot_mapping"):
        call(q, k, v, w, w, pos, cos, sin, 1e-6, pool, pool.clone(), slots[:5])
    with pytest.raises(RuntimeError, match="matching k and v"):
        call(q, k, v[:, :4], w, w, pos, cos, sin, 1e-6, pool, pool.clone(), slots)
    torch.cuda.synchronize()
    assert torch.equal(pool, before)


@pytest.mark.parametrize("fused", [False, True])
def test_slots_outside_the_pool_are_skipped(extension, device, fused):
    """A slot at or past num_blocks x P writes nothing (as a negative one), in the plain
    KV write and in the fused QK-norm + RoPE write: the rest of the pool is exactly what
    the in-range tokens leave."""
    from mini_vllm.torch_path import rope_tables

    nb, bs, hk, d = 4, 16, 2, 64
    bf = dict(dtype=torch.bfloat16, device=device)
    k = torch.randn(5, hk, d, **bf)
    v = torch.randn(5, hk, d, **bf)
    good = torch.tensor([3, 17, -1, 40, 63], dtype=torch.int32, device=device)
    bad = torch.tensor([3, 17, nb * bs, 40, nb * bs + 1000], dtype=torch.int32, device=device)
    keep = torch.tensor([3, 17, -1, 40, -1], dtype=torch.int32, device=device)
    pools = []
    for slots in (bad, keep):
        pk, pv = torch.zeros(nb, bs, hk, d, **bf), torch.zeros(nb, bs, hk, d, **bf)
        if fused:
            q = torch.randn(5, 4, d, **bf)
            w = torch.ones(d, **bf)
            cos, sin = rope_tables(d, 64, device=device)
            extension.qk_norm_rope_kv_write(q, k, v, w, w, torch.arange(5, device=device), cos,
                                            sin, 1e-6, pk, pv, slots)
        else:
            extension.kv_write(pk, pv, k, v, slots)
        pools.append((pk, pv))
    torch.cuda.synchronize()
    assert torch.equal(pools[0][0], pools[1][0]) and torch.equal(pools[0][1], pools[1][1])
    assert pools[1][1].view(-1, hk, d)[17].equal(v[1]) and good.numel() == 5
