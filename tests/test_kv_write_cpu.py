"""Paged KV write on the CPU: the oracle (oracle/kv_write.py) pinned against the
reference's own operation and against closed forms, and the PyTorch path
(``ops.kv_write(use_cuda=False)``) against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mini_vllm import torch_path
from mini_vllm.block import PagedKvPool
from mini_vllm.workloads import quantize_fp8_per_block
from oracle import kv_write as ow
from oracle.elementwise import fp8_e4m3_decode


def _slots(rng, num_blocks, bs, t, pad=0):
    """t distinct random slots plus `pad` padding (-1) entries."""
    s = rng.choice(num_blocks * bs, size=t, replace=False).astype(np.int32)
    return np.concatenate([s, -np.ones(pad, dtype=np.int32)])


def test_copy_oracle_is_the_references_index_copy():
    """block/kv_pool.py:148-155: flat_pool.index_copy_(0, slot_mapping, x)."""
    rng = np.random.default_rng(0)
    pool = rng.standard_normal((12, 16, 2, 8)).astype(np.float32)
    slots = _slots(rng, 12, 16, 40)
    x = rng.standard_normal((40, 2, 8)).astype(np.float32)
    want = torch.from_numpy(pool.copy()).view(-1, 2, 8)
    want.index_copy_(0, torch.from_numpy(slots).long(), torch.from_numpy(x))
    assert np.array_equal(ow.kv_write_copy(pool, slots, x), want.view(12, 16, 2, 8).numpy())


def test_copy_skips_negative_slots_and_torch_path_agrees():
    rng = np.random.default_rng(1)
    pool = rng.standard_normal((6, 4, 2, 8)).astype(np.float32)
    slots = _slots(rng, 6, 4, 10, pad=3)
    x = rng.standard_normal((13, 2, 8)).astype(np.float32)
    want = ow.kv_write_copy(pool, slots, x)
    kp, vp = torch.from_numpy(pool.copy()), torch.from_numpy(pool.copy())
    xt = torch.from_numpy(x)
    torch_path.kv_write(kp, vp, xt, xt, torch.from_numpy(slots))
    assert np.array_equal(kp.numpy(), want) and np.array_equal(vp.numpy(), want)


def test_runs():
    assert ow.runs(np.array([44, 45, 46, 47, 48, 7, -1, 8, 9]), 16) == [(0, 4), (4, 1), (5, 1), (7, 2)]
    assert ow.runs(np.array([3, 5, 6]), 16) == [(0, 1), (1, 2)]


def _fp8_state(num_blocks, bs, hk, d):
    return np.zeros((num_blocks, bs, hk, d), np.uint8), np.zeros((num_blocks, hk), np.float32)


def test_pow2_ceil():
    t = np.array([0.0, 1.0, 1.5, 3.0, 0.75, 2.0**-130, 448.0 / 448], np.float32)
    want = np.array([0.0, 1.0, 2.0, 4.0, 1.0, 2.0**-126, 1.0], np.float32)
    assert np.array_equal(ow.pow2_ceil(t), want)
    r = np.random.default_rng(5).uniform(1e-6, 1e3, 1000).astype(np.float32)
    p = ow.pow2_ceil(r)
    assert np.all(p >= r) and np.all(p / 2 < r) and np.all(np.log2(p) == np.round(np.log2(p)))
    assert torch.equal(torch_path._pow2_ceil(torch.from_numpy(r)), torch.from_numpy(p))


def test_fp8_fresh_block_equals_the_per_block_quantiser():
    """One run filling a fresh block = the config-4 quantiser of that block, with the
    block's scale pow2ceil(amax / 448) in place of amax / 448."""
    rng = np.random.default_rng(2)
    bs, hk, d = 16, 2, 32
    x = rng.standard_normal((bs, hk, d)).astype(np.float32) * 3
    codes, scales = _fp8_state(4, bs, hk, d)
    codes, scales = ow.kv_write_fp8(codes, scales, np.arange(2 * bs, 3 * bs, dtype=np.int32), x)
    s = ow.pow2_ceil((np.abs(x).max(axis=(0, 2)) / np.float32(448)).astype(np.float32))
    assert np.array_equal(scales[2], s)
    xt = torch.from_numpy(x)
    q = (xt / torch.from_numpy(s)[None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert np.array_equal(codes[2], q.view(torch.uint8).numpy())
    _, s_static = quantize_fp8_per_block(xt[None])
    assert np.all(s >= s_static[0].numpy()) and np.all(s < 2 * s_static[0].numpy())


def test_fp8_token_by_token_scale_is_the_block_amax():
    """Appending rows one at a time (decode), the scale ends at pow2ceil(max|x| / 448)
    of the block, and every row decodes within half an e4m3 step of its source at the
    scale it was written with (re-encoding under grown scales is exact here)."""
    rng = np.random.default_rng(3)
    bs, hk, d = 16, 2, 32
    x = rng.standard_normal((bs, hk, d)).astype(np.float32) * np.linspace(0.1, 4, bs)[:, None, None].astype(np.float32)
    codes, scales = _fp8_state(3, bs, hk, d)
    written_at = []
    for t in range(bs):
        codes, scales = ow.kv_write_fp8(codes, scales, np.array([bs + t], np.int32), x[t:t + 1])
        written_at.append(scales[1].copy())
    amax = np.abs(x).max(axis=(0, 2)).astype(np.float32)
    assert np.array_equal(scales[1], ow.pow2_ceil((amax / np.float32(448)).astype(np.float32)))
    got = fp8_e4m3_decode(codes[1]) * scales[1][None, :, None]
    s_t = np.stack(written_at)[:, :, None]                 # scale of each row's write
    err = np.abs(got - x)
    # e4m3: 3 mantissa bits -> half step <= 2^-4 relative; subnormal step 2^-9 * scale
    assert np.all(err <= np.abs(x) * 2.0**-4 + s_t * 2.0**-10)


def _fp8_scenario(rng, hk=2, d=32, bs=16):
    """A prefill chunk over 2.5 blocks, then decode steps with growing magnitudes (so
    the scale grows and old rows are re-encoded), interleaved with another sequence."""
    steps = []
    a = [5 * bs + i for i in range(bs)] + [9 * bs + i for i in range(bs)] + [2 * bs + i for i in range(8)]
    b = [11 * bs + i for i in range(5)]
    steps.append(np.array(a + b, np.int32))
    for k in range(6):
        steps.append(np.array([2 * bs + 8 + k, 11 * bs + 5 + k, -1], np.int32))
    xs = []
    for i, sl in enumerate(steps):
        grow = 1.0 + 0.6 * i
        xs.append((rng.standard_normal((len(sl), hk, d)) * grow).astype(np.float32))
    return steps, xs


def test_fp8_torch_path_matches_the_oracle_bytes():
    rng = np.random.default_rng(4)
    steps, xs = _fp8_scenario(rng)
    codes, scales = _fp8_state(16, 16, 2, 32)
    kp = torch.zeros((16, 16, 2, 32), dtype=torch.float8_e4m3fn)
    vp = torch.zeros_like(kp)
    ks, vs = torch.zeros((16, 2)), torch.zeros((16, 2))
    for sl, x in zip(steps, xs):
        codes, scales = ow.kv_write_fp8(codes, scales, sl, x)
        xt = torch.from_numpy(x).to(torch.bfloat16).float()  # representable either way
        torch_path.kv_write(kp, vp, torch.from_numpy(x), torch.from_numpy(-x),
                            torch.from_numpy(sl), k_scale=ks, v_scale=vs)
    assert np.array_equal(kp.view(torch.uint8).numpy(), codes)
    assert np.array_equal(ks.numpy(), scales)
    assert np.array_equal(vs.numpy(), scales)  # -x has the same magnitudes
    assert np.array_equal(vp.view(torch.uint8).numpy(), codes ^ np.where(codes & 0x7F, 0x80, 0).astype(np.uint8))


def test_pool_write_routes_through_ops_and_holds_fp8_scales():
    pool = PagedKvPool(2, 8, 4, 2, 16, dtype=torch.float8_e4m3fn)
    assert pool.is_fp8 and pool.layer_scales(1)[0].shape == (8, 2)
    x = torch.randn(3, 2, 16)
    pool.write(1, torch.tensor([4, 5, 6], dtype=torch.int32), x, x)
    k_scale, _ = pool.layer_scales(1)
    assert torch.equal(k_scale[1], torch_path._pow2_ceil(x.abs().amax(dim=(0, 2)) / 448.0))
    assert pool.keys[0].view(torch.uint8).count_nonzero() == 0
    with pytest.raises(ValueError, match="shaped"):
        pool.write(0, torch.tensor([0], dtype=torch.int32), x, x)
