"""Pin the CPU oracle before trusting it (CPU only).

Every function of ``oracle/`` is checked here against something other than its own
formula: the golden fixtures (float64 brute force), the reference's known-answer
properties (tests/test_paged_attention_cuda.py:202-289, test_block_manager.py:297-486),
closed forms, and torch's own casts for the rounding helpers. Each check is chosen so
a plausible slip (wrong causal offset, transposed operand, dropped scale, wrong GQA
head mapping, wrong slot arithmetic) fails at least one of them.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from mini_vllm.workloads import build_batch, config_batch, quantize_fp8_per_block
from oracle import brute, elementwise as ew
from oracle.paged_attention import paged_attention as oracle_paged, slots_for

GOLDEN = __import__("pathlib").Path(__file__).parent / "golden"


def run_oracle(b, **kw):
    return oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale, b.k_scale, b.v_scale, **kw)


# ----------------------------------------------------------------- golden vectors


@pytest.mark.parametrize("name,make", [
    ("paged_cfg1", lambda: config_batch(1)),
    ("paged_mixed_small", lambda: build_batch([300, 1, 17, 50], [1, 1, 17, 8], num_q_heads=8,
                                              num_kv_heads=2, head_dim=64, seed=5)),
])
def test_oracle_matches_golden(name, make):
    gold = np.load(GOLDEN / f"{name}.npz")
    b = make()
    # The seeded inputs are the ones the fixture was made from.
    assert np.array_equal(gold["block_tables"], b.block_tables.numpy())
    assert gold["fp_keys"] == pytest.approx(b.key_pool.double().sum().item(), rel=1e-12)
    assert gold["fp_values"] == pytest.approx(b.value_pool.double().sum().item(), rel=1e-12)
    assert gold["fp_q"] == pytest.approx(b.q.double().sum().item(), rel=1e-12)
    got = run_oracle(b).double().numpy()
    assert np.abs(got - gold["out"]).max() < 2e-6
    # and the brute force reproduces its own fixture
    again = brute.paged_attention_f64(b.q, b.key_pool, b.value_pool, b.block_tables,
                                      b.cu_seqlens_q, b.context_lens, b.scale)
    assert np.abs(again - gold["out"]).max() < 1e-12


def test_config1_shape_is_the_baseline_one():
    b = config_batch(1)
    assert b.contexts == [37, 128, 511, 1000]
    assert tuple(b.key_pool.shape) == (512, 16, 8, 128)
    assert tuple(b.block_tables.shape) == (4, 63)
    assert b.kv_bytes() == 13_729_792  # 1676 keys x 8 heads x 128 x 4 B x 2


# ------------------------------------------------------ oracle vs brute force


@pytest.mark.parametrize("contexts,query_lens,hq,hk,d,p", [
    ([1, 15, 16, 17, 63, 64, 65], [1] * 7, 8, 4, 64, 16),
    ([40], [8], 8, 4, 64, 16),                # a chunk at the end of a context
    ([12, 300], [12, 1], 8, 8, 32, 1),        # block size 1, no GQA
    ([100, 9], [1, 9], 8, 1, 32, 64),         # block size 64, one kv head
    ([70, 33, 5], [3, 1, 5], 16, 8, 128, 2),
])
def test_oracle_matches_float64_brute_force(contexts, query_lens, hq, hk, d, p):
    b = build_batch(contexts, query_lens, num_q_heads=hq, num_kv_heads=hk, head_dim=d,
                    block_size=p, seed=sum(contexts))
    want = brute.paged_attention_f64(b.q, b.key_pool, b.value_pool, b.block_tables,
                                     b.cu_seqlens_q, b.context_lens, b.scale)
    got = run_oracle(b, compute_dtype=torch.float64).numpy()
    assert np.abs(got - want).max() < 1e-10


def test_fp8_oracle_matches_float64_brute_force():
    b = build_batch([100, 40], [1, 4], num_q_heads=8, num_kv_heads=2, head_dim=64,
                    dtype=torch.bfloat16, kv_dtype=torch.float8_e4m3fn, seed=3)
    want = brute.paged_attention_f64(b.q, b.key_pool, b.value_pool, b.block_tables,
                                     b.cu_seqlens_q, b.context_lens, b.scale, b.k_scale,
                                     b.v_scale)
    got = run_oracle(b, compute_dtype=torch.float64).numpy()
    assert np.abs(got - want).max() < 1e-6


# -------------------------------------------------------------- known answers


def test_one_visible_key_returns_that_value_exactly():
    """First query of a prompt sees only logical key 0 (test_paged_attention_cuda.py:202-214)."""
    b = build_batch([12], [12], num_q_heads=8, num_kv_heads=4, head_dim=64, seed=11)
    got = run_oracle(b)
    first_block = int(b.block_tables[0, 0])
    expected = b.value_pool[first_block, 0]  # H_k x D at logical position 0
    for h in range(8):
        assert torch.equal(got[0, h], expected[h // 2])


def test_two_keys_closed_form():
    """Decode over two keys: w = sigmoid(s0 - s1) by hand, per query head."""
    b = build_batch([2], [1], num_q_heads=4, num_kv_heads=2, head_dim=32, block_size=1, seed=2)
    got = run_oracle(b, compute_dtype=torch.float64)
    t = b.block_tables[0]
    for h in range(4):
        kvh = h // 2
        k0, k1 = b.key_pool[int(t[0]), 0, kvh].double(), b.key_pool[int(t[1]), 0, kvh].double()
        v0, v1 = b.value_pool[int(t[0]), 0, kvh].double(), b.value_pool[int(t[1]), 0, kvh].double()
        qv = b.q[0, h].double()
        s0, s1 = (qv @ k0) * b.scale, (qv @ k1) * b.scale
        w0 = 1.0 / (1.0 + math.exp(s1 - s0))
        assert torch.allclose(got[0, h], w0 * v0 + (1 - w0) * v1, atol=1e-12)


def test_physical_layout_does_not_change_the_answer():
    """Same logical keys under two physical layouts (test_paged_attention_cuda.py:272-289):
    move every block to a new id, remap the table, and the output must not move."""
    b = build_batch([200, 37], [1, 5], num_q_heads=8, num_kv_heads=4, head_dim=64, seed=4)
    n = b.key_pool.shape[0]
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(9))
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(n)
    moved_keys, moved_values = torch.empty_like(b.key_pool), torch.empty_like(b.value_pool)
    moved_keys[perm] = b.key_pool
    moved_values[perm] = b.value_pool
    table = b.block_tables.clone().long()
    table[table >= 0] = perm[table[table >= 0]]
    got = oracle_paged(b.q, moved_keys, moved_values, table.int(), b.cu_seqlens_q,
                       b.context_lens, b.scale)
    assert torch.allclose(got, run_oracle(b), atol=1e-6)


def test_each_sequence_of_a_mixed_batch_equals_its_run_alone():
    b = build_batch([300, 700, 50, 64], [300, 1, 50, 1], num_q_heads=8, num_kv_heads=4,
                    head_dim=64, seed=6)
    together = run_oracle(b)
    for s in range(4):
        lo, hi = int(b.cu_seqlens_q[s]), int(b.cu_seqlens_q[s + 1])
        alone = oracle_paged(b.q[lo:hi], b.key_pool, b.value_pool, b.block_tables[s:s + 1],
                             torch.tensor([0, hi - lo], dtype=torch.int32), b.context_lens[s:s + 1],
                             b.scale)
        assert torch.allclose(together[lo:hi], alone, atol=1e-6)


def test_prefill_row_equals_decode_at_its_position():
    """Row r of a chunk of L over S keys sees S - L + r + 1 keys: exactly a decode."""
    b = build_batch([40], [8], num_q_heads=8, num_kv_heads=4, head_dim=64, seed=8)
    chunk = run_oracle(b, compute_dtype=torch.float64)
    for r in range(8):
        single = oracle_paged(b.q[r:r + 1], b.key_pool, b.value_pool, b.block_tables,
                              torch.tensor([0, 1], dtype=torch.int32),
                              torch.tensor([40 - 8 + r + 1], dtype=torch.int32), b.scale,
                              compute_dtype=torch.float64)
        assert torch.allclose(chunk[r], single[0], atol=1e-12)


def test_padding_and_spare_blocks_are_never_read():
    b = build_batch([33, 5], [1, 1], num_q_heads=8, num_kv_heads=4, head_dim=64, seed=12,
                    spare_blocks=4)
    used = {int(x) for x in b.block_tables.flatten() if int(x) >= 0}
    keys, values = b.key_pool.clone(), b.value_pool.clone()
    for blk in range(keys.shape[0]):
        if blk not in used:
            keys[blk] = float("nan")
            values[blk] = float("nan")
    got = oracle_paged(b.q, keys, values, b.block_tables, b.cu_seqlens_q, b.context_lens, b.scale)
    assert torch.isfinite(got).all()


def test_reading_past_the_table_raises():
    b = build_batch([33, 5], [1, 1], num_q_heads=8, num_kv_heads=4, head_dim=64, seed=1)
    with pytest.raises(ValueError, match="padded"):   # row 1 is [id, -1, -1]
        oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                     torch.tensor([33, 40], dtype=torch.int32), b.scale)
    with pytest.raises(ValueError, match="past the end"):
        oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                     torch.tensor([80, 5], dtype=torch.int32), b.scale)


def test_convex_combination_of_visible_values():
    b = build_batch([64], [64], num_q_heads=8, num_kv_heads=4, head_dim=64, seed=13)
    got = run_oracle(b)
    visible = torch.stack([b.value_pool[int(x)] for x in b.block_tables[0]])
    assert got.min() >= visible.min() - 1e-5 and got.max() <= visible.max() + 1e-5


def test_slot_mapping_known_answer():
    """Slots for a 6-token sequence over tables [[0, 1]] at P=4 are 0..5
    (test_block_manager.py:475-486), and shuffled tables map block-wise."""
    assert slots_for(torch.tensor([0, 1]), 6, 4).tolist() == [0, 1, 2, 3, 4, 5]
    assert slots_for(torch.tensor([3, 0, -1]), 6, 4).tolist() == [12, 13, 14, 15, 0, 1]


# --------------------------------------------------------- elementwise oracle


def test_bf16_rounding_matches_torch_cast():
    x = torch.randn(1 << 16) * torch.logspace(-30, 30, 1 << 16)
    x[:4] = torch.tensor([0.0, -0.0, 1.00390625, 1.01171875])  # exact ties
    want = x.to(torch.bfloat16).float().numpy()
    assert np.array_equal(ew.round_bf16(x.numpy()), want)


def test_fp8_codec_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = ew.fp8_e4m3_decode(codes.numpy())
    finite = ~np.isnan(want)
    assert np.array_equal(np.isnan(got), ~finite)
    assert np.array_equal(got[finite], want[finite])
    assert ew.fp8_e4m3_decode(np.array([0x7E], dtype=np.uint8))[0] == 448.0
    x = torch.randn(4096) * 100
    assert np.array_equal(ew.fp8_e4m3_encode(x.numpy()),
                          x.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy())


def test_per_block_fp8_quantisation_scales():
    x = torch.randn(6, 16, 8, 128)
    q, s = quantize_fp8_per_block(x)
    assert torch.allclose(s, x.abs().amax(dim=(1, 3)) / 448.0)
    deq = q.float() * s[:, None, :, None]
    # e4m3 has a 3-bit mantissa: relative error <= 2^-4 on normal values
    assert ((deq - x).abs() <= x.abs() * 2**-4 + s[:, None, :, None] * 2**-9).all()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_rms_norm_unit_weight_has_unit_rms(dtype):
    x = np.random.default_rng(0).standard_normal((16, 1024)).astype(np.float32) * 3
    out = ew.rms_norm(ew.round_to(x, dtype), np.ones(1024, np.float32), dtype=dtype)
    rms = np.sqrt((out.astype(np.float64) ** 2).mean(axis=-1))
    assert np.allclose(rms, 1.0, atol=1e-2 if dtype != "f32" else 1e-5)


def test_rms_norm_rounds_before_the_weight_like_torch():
    x = torch.randn(32, 128).to(torch.bfloat16)
    w = (torch.rand(128) * 2).to(torch.bfloat16)
    x32 = x.float()
    want = w * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    got = ew.rms_norm(x.float().numpy(), w.float().numpy(), 1e-6, "bf16")
    diff = np.abs(got - want.float().numpy())
    ulp = np.abs(want.float().numpy()) * 2**-7 + 1e-30
    assert (diff <= ulp).all()
    assert (diff == 0).mean() > 0.99


def test_rope_tables_and_rotation_properties():
    cos, sin = ew.rope_tables(128, 64)
    t_cos = torch.outer(torch.arange(64, dtype=torch.float32),
                        1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128)))
    # float32 pow may differ by one ulp between numpy and torch; position 63 amplifies
    # that to a few 1e-6 in the angle. The kernels take the tables as inputs anyway.
    assert np.allclose(cos[:, :64], torch.cos(t_cos).numpy(), atol=1e-5)
    assert np.array_equal(cos[:, :64], cos[:, 64:])
    x = np.random.default_rng(1).standard_normal((5, 4, 128)).astype(np.float32)
    # position 0 is the identity
    assert np.array_equal(ew.apply_rope(x, np.zeros(5, np.int64), cos, sin), x)
    # rotation preserves each (i, i + D/2) pair's norm
    out = ew.apply_rope(x, np.arange(5), cos, sin)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = out[..., :64] ** 2 + out[..., 64:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)


def test_swiglu_matches_torch_cpu_within_a_rounding():
    g = torch.randn(8192) * 4
    u = torch.randn(8192)
    for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        gd, ud = g.to(dt), u.to(dt)
        want = (gd * torch.sigmoid(gd) * ud).float().numpy()
        got = ew.swiglu(gd.float().numpy(), ud.float().numpy(), name)
        tol = np.abs(want) * (2**-7 if name == "bf16" else 1e-6) + 1e-30
        assert (np.abs(got - want) <= tol).all()
    assert ew.swiglu(np.zeros(3, np.float32), np.ones(3, np.float32))[0] == 0.0


# -- dense-cache attention oracle (oracle/dense_attention.py)

def _as_pages(k: torch.Tensor, block: int = 16, seed: int = 0):
    """k ``B x H_k x S x D`` laid out as a shuffled paged pool ``nb x P x H_k x D`` with
    its block tables."""
    b, hk, s, d = k.shape
    pages = -(-s // block)
    perm = torch.randperm(b * pages, generator=torch.Generator().manual_seed(seed))
    pool = torch.zeros(b * pages, block, hk, d, dtype=k.dtype)
    tables = perm.view(b, pages).to(torch.int32)
    for i in range(b):
        for j in range(s):
            pool[tables[i, j // block], j % block] = k[i, :, j]
    return pool, tables


@pytest.mark.parametrize("L,S", [(1, 37), (5, 5), (7, 40)])
def test_dense_oracle_equals_the_paged_oracle(L, S):
    """The same keys as a dense cache and as shuffled pages give the same attention."""
    from oracle.dense_attention import dense_attention

    gen = torch.Generator().manual_seed(L * 100 + S)
    b, hq, hk, d = 3, 8, 2, 32
    q = torch.randn(b, hq, L, d, generator=gen)
    k = torch.randn(b, hk, S, d, generator=gen)
    v = torch.randn(b, hk, S, d, generator=gen)
    dense = dense_attention(q, k, v, causal=True)
    kp, tables = _as_pages(k)
    vp, _ = _as_pages(v)
    qt = q.transpose(1, 2).reshape(b * L, hq, d)
    cu = torch.arange(0, (b + 1) * L, L, dtype=torch.int32)
    ctx = torch.full((b,), S, dtype=torch.int32)
    paged = oracle_paged(qt, kp, vp, tables, cu, ctx, 1 / math.sqrt(d), compute_dtype=torch.float64)
    torch.testing.assert_close(dense.transpose(1, 2).reshape(b * L, hq, d), paged, rtol=0, atol=1e-12)


def test_dense_oracle_known_answers():
    """One visible key (S = 1) returns its value; q = 0 (equal scores) returns the mean
    of the visible values, per query row under the causal offset."""
    from oracle.dense_attention import dense_attention

    gen = torch.Generator().manual_seed(5)
    q = torch.randn(2, 4, 1, 16, generator=gen)
    k = torch.randn(2, 2, 1, 16, generator=gen)
    v = torch.randn(2, 2, 1, 16, generator=gen)
    out = dense_attention(q, k, v)
    assert torch.equal(out, v.double().repeat_interleave(2, dim=1))
    L, S = 3, 6
    v = torch.randn(1, 1, S, 8, generator=gen)
    out = dense_attention(torch.zeros(1, 2, L, 8), torch.randn(1, 1, S, 8, generator=gen), v)
    for i in range(L):
        want = v[0, 0, : S - L + i + 1].double().mean(0)
        torch.testing.assert_close(out[0, 1, i], want, rtol=0, atol=1e-12)


def test_dense_model_oracle_matches_transformers_qwen3():
    """oracle/qwen3_dense.py (and its KV-cached loop) against Hugging Face's Qwen3 in
    float64 on the tiny shape with non-unit norm weights (fixture made by
    tests/golden/make_qwen3_golden.py, transformers 5.15.0): the same greedy tokens and
    next-token logits to 1e-6 at every step (Hugging Face computes the RoPE frequencies
    and the RMSNorm statistics in float32 even in a float64 model: ~1e-7 here, against
    O(0.1) for any wiring mistake). This pins the layer wiring (norm order,
    QK-norm per head, rotate-half RoPE at theta 1e6, GQA, SwiGLU, tied embedding)
    independently of this repository's engine."""
    import sys

    from oracle.qwen3_dense import DenseQwen3, generate_greedy

    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    from make_qwen3_golden import golden_weights, weights_digest

    fx = np.load(Path(__file__).resolve().parent / "golden" / "qwen3_tiny_hf.npz")
    config, weights = golden_weights()
    assert weights_digest(weights) == str(fx["weights_sha256"]), "the weight generator changed"
    dense = DenseQwen3(config, weights)
    for i in range(int(fx["num_prompts"])):
        prompt = fx[f"prompt_{i}"].tolist()
        want_tokens, want_logits = fx[f"tokens_{i}"].tolist(), fx[f"step_logits_{i}"]
        for tokens, logits in (generate_greedy(config, weights, prompt, len(want_tokens)),
                               dense.generate(prompt, len(want_tokens))):
            assert tokens == want_tokens, f"prompt {i}"
            got = np.stack([l.numpy() for l in logits])
            assert np.abs(got - want_logits).max() < 1e-6, f"prompt {i}"


def test_fp8_pages_of_the_dense_oracle():
    """oracle/qwen3_dense.py's Fp8Pages: one write of a fresh sequence equals a direct
    per-(page, kv head) quantisation at scale pow2ceil(amax / 448) (the closed form of the
    write policy for one run); written token by token, every page ends at the scale of
    its whole contents and every value within half an e4m3 step of its source (re-encoding
    under a grown power-of-two scale being exact above the subnormals)."""
    from oracle.kv_write import pow2_ceil
    from oracle.qwen3_dense import Fp8Pages

    gen = torch.Generator().manual_seed(5)
    k = torch.randn(40, 2, 8, generator=gen, dtype=torch.float64) * 3
    v = torch.randn(40, 2, 8, generator=gen, dtype=torch.float64)
    pages = Fp8Pages(1, 2, 8)
    keys, vals = pages.write(0, 0, k, v)
    for x, got in ((k, keys), (v, vals)):
        padded = torch.zeros(48, 2, 8, dtype=torch.float64)
        padded[:40] = x
        blocks = padded.view(3, 16, 2, 8).float()
        amax = blocks.abs().amax(dim=(1, 3)).numpy()
        scale = torch.from_numpy(pow2_ceil(amax / np.float32(448.0)))
        codes = (blocks / scale[:, None, :, None]).to(torch.float8_e4m3fn)
        want = (codes.float() * scale[:, None, :, None]).view(48, 2, 8)[:40].double()
        assert torch.equal(got, want)
    step = Fp8Pages(1, 2, 8)
    for t in range(40):
        keys, vals = step.write(0, t, k[t:t + 1], v[t:t + 1])
    assert keys.shape == (40, 2, 8)
    for x, got, i in ((k, keys, 0), (v, vals, 1)):
        scales = step.scales[0][i]
        for b in range(3):
            rows = x[16 * b:16 * b + 16].float()
            want_s = pow2_ceil((rows.abs().amax(dim=(0, 2)) / 448.0).numpy())
            assert np.array_equal(scales[b], want_s), b
            s = torch.from_numpy(want_s).double()[None, :, None]
            mag = (rows.double() / s).abs()
            half_step = torch.where(mag < 2.0**-6, 2.0**-10, 2.0 ** (torch.floor(torch.log2(mag)) - 4))
            assert ((got[16 * b:16 * b + 16] - rows.double()).abs() <= half_step * s + 1e-12).all(), b


@pytest.mark.parametrize("kv_fp8", [False, True])
def test_teacher_forcing_the_greedy_tokens_gives_the_same_logits(kv_fp8):
    """DenseQwen3.forced fed the model's own greedy continuation returns exactly the
    logits its generate() saw (same cache path, one token a step), with and without
    the fp8 pages."""
    from engine_helpers import tiny_config
    from mini_vllm.model import random_weights
    from oracle.qwen3_dense import DenseQwen3

    config = tiny_config()
    dense = DenseQwen3(config, random_weights(config, seed=1, std=0.3), kv_fp8=kv_fp8)
    prompt = [5, 9, 100, 7, 300]
    tokens, logits = dense.generate(prompt, 6)
    forced = dense.forced(prompt, tokens)
    assert len(forced) == 6 and all(torch.equal(a, b) for a, b in zip(logits, forced))
