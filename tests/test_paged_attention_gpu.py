"""Paged attention on the MI355X against the CPU oracle (``-m gpu``).

The case list follows the reference's kernel tests
(tests/test_paged_attention_cuda.py:135-447): block/tile boundaries, the split path,
ragged batches with empty splits, every GQA group size, head dim and block size,
prefill lengths, the chunk's causal offset, known answers, mixed batches, the shuffle,
dtypes, refusals and dispatch. BASELINE configs 1-4 are checked at full size.

Tolerances (max-abs vs the fp32 oracle): fp32 2e-5, fp16 1e-2, bf16 2e-2, fp8 KV 6e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATTN_ATOL, assert_max_abs
from mini_vllm.kernels import ops
from mini_vllm.workloads import build_batch, config_batch, prefill_flops
from oracle.paged_attention import paged_attention as oracle_paged

pytestmark = pytest.mark.gpu

HQ, HK, D = 8, 4, 64


def oracle(b):
    return oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale, b.k_scale, b.v_scale)


def kernel(ext, b, options=None):
    out = ext.paged_attention(*b.args(), k_scale=b.k_scale, v_scale=b.v_scale,
                              plan_options=options)
    torch.cuda.synchronize()
    return out


def case(contexts, query_lens, device, **kw):
    kw.setdefault("num_q_heads", HQ)
    kw.setdefault("num_kv_heads", HK)
    kw.setdefault("head_dim", D)
    kw.setdefault("seed", sum(contexts) + len(contexts))
    return build_batch(contexts, query_lens, device=device, **kw)


def check(ext, b, dtype=None, msg="", options=None):
    dtype = dtype or b.key_pool.dtype
    got = kernel(ext, b, options)
    assert got.dtype == b.q.dtype
    assert_max_abs(got, oracle(b), ATTN_ATOL[dtype], msg)
    return got


# --------------------------------------------------------------------- decode


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("context", [1, 15, 16, 17, 63, 64, 65, 200, 1000])
def test_decode_matches_the_oracle_at_every_boundary(extension, device, context, dtype):
    check(extension, case([context], [1], device, dtype=dtype), msg=f"context {context}")


def test_decode_over_a_long_context_uses_the_split_path(extension, device):
    b = case([8192], [1], device)
    plan = extension.paged_attention_plan(1, 1, HQ, HK, D, 16, 1, 8192, b.q.dtype, b.q.dtype)
    assert plan["decode_mode"] == "stream" and plan["decode_workgroups"] > 1
    check(extension, b)


DECODE_SCHEDULES = {"stream": None, "grid": {"decode_schedule": "grid"}}


@pytest.mark.parametrize("schedule", sorted(DECODE_SCHEDULES))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_every_decode_schedule_agrees_with_the_oracle(extension, device, schedule, dtype):
    """The stream schedule (default) and the split grid (forced) on a ragged batch,
    including sequences shorter than one workgroup's share (or than its waves) and
    longer than many."""
    options = DECODE_SCHEDULES[schedule]
    b = case([8192, 33, 4096, 17, 1, 700, 2], [1] * 7, device, dtype=dtype)
    plan = extension.paged_attention_plan(7, 7, HQ, HK, D, 16, 1, 8192, dtype, dtype,
                                          plan_options=options)
    assert plan["decode_mode"] == schedule
    check(extension, b, options=options)


@pytest.mark.parametrize("schedule", sorted(DECODE_SCHEDULES))
@pytest.mark.parametrize("kv_dtype", [None, torch.float8_e4m3fn])
def test_decode_schedules_in_a_mixed_batch(extension, device, kv_dtype, schedule):
    """Prefill chunks beside decode rows: each decode schedule leaves the chunks to the
    prefill kernel; GQA groups of 2 and 4, fp8 pools with their scales."""
    for heads, kv_heads in ((16, 8), (16, 4)):
        b = case([900, 2500, 40, 700, 5], [1, 400, 1, 1, 5], device, dtype=torch.bfloat16,
                 kv_dtype=kv_dtype, num_q_heads=heads, num_kv_heads=kv_heads, head_dim=128)
        check(extension, b, dtype=kv_dtype or torch.bfloat16, options=DECODE_SCHEDULES[schedule])


@pytest.mark.parametrize("wgs_per_cu", ["1", "4"])
def test_stream_schedule_with_more_workgroups_than_keys(extension, device, wgs_per_cu):
    """Tiny batches leave most stream workgroups with empty shares; the merge must skip
    their slots."""
    b = case([3, 5, 2], [1, 1, 1], device, dtype=torch.bfloat16, block_size=1)
    check(extension, b, options={"decode_wgs_per_cu": wgs_per_cu})


def test_a_ragged_decode_batch_with_empty_splits(extension, device):
    """Short sequences beside a long one get fewer splits than the grid holds."""
    b = case([8192, 33, 4096, 17], [1, 1, 1, 1], device)
    check(extension, b)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("wgs_per_cu", ["1", "3"])
def test_stream_decode_merge_of_cut_sequences(extension, device, kv_dtype, wgs_per_cu):
    """Sequences cut between stream workgroups are merged by the merge kernel after the
    decode launch: sequences of one piece, of two and of dozens, with prefill rows beside
    them, on calls in a row that give the same bits."""
    b = case([12000, 700, 33, 4096, 1, 2500, 300], [1, 1, 1, 1, 1, 1, 64], device,
             dtype=torch.bfloat16, kv_dtype=kv_dtype, num_q_heads=16, num_kv_heads=8,
             head_dim=128)
    want = oracle(b)
    runs = []
    for _ in range(3):
        got = kernel(extension, b, {"decode_wgs_per_cu": wgs_per_cu})
        assert_max_abs(got, want, ATTN_ATOL[kv_dtype], "stream decode + merge")
        runs.append(got)
    for got in runs[1:]:
        assert torch.equal(got, runs[0])


@pytest.mark.parametrize("split_tokens", ["64", "1024"])
def test_forced_split_sizes_agree(extension, device, split_tokens):
    check(extension, case([3000, 129, 64, 1], [1, 1, 1, 1], device, dtype=torch.bfloat16),
          options={"decode_schedule": "grid", "decode_split_tokens": split_tokens})


@pytest.mark.parametrize("kv_heads", [1, 2, 8])
def test_every_group_size(extension, device, kv_heads):
    check(extension, case([100], [1], device, num_q_heads=8, num_kv_heads=kv_heads))


@pytest.mark.parametrize("heads,kv_heads", [(16, 1), (12, 4), (6, 2)])
def test_wide_and_odd_groups(extension, device, heads, kv_heads):
    check(extension, case([300, 7], [1, 1], device, num_q_heads=heads, num_kv_heads=kv_heads))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [32, 64, 128, 256])
def test_every_head_dimension(extension, device, head_dim, dtype):
    check(extension, case([100, 250], [1, 1], device, head_dim=head_dim, dtype=dtype))


@pytest.mark.parametrize("block_size", [1, 2, 16, 64])
def test_every_block_size(extension, device, block_size):
    check(extension, case([100, 1100], [1, 1], device, block_size=block_size))


# -------------------------------------------------------------------- prefill


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("length", [2, 8, 9, 16, 17, 64, 300])
def test_prefill_matches_the_oracle(extension, device, length, dtype):
    check(extension, case([length], [length], device, dtype=dtype), msg=f"length {length}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_a_chunk_sees_its_prefix_and_not_its_future(extension, device, dtype):
    check(extension, case([40], [8], device, dtype=dtype))


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("heads,kv_heads", [(16, 8), (8, 8), (16, 2), (12, 4)])
def test_mfma_prefill_shapes(extension, device, head_dim, heads, kv_heads):
    b = case([700, 130, 97], [200, 130, 33], device, dtype=torch.bfloat16, head_dim=head_dim,
             num_q_heads=heads, num_kv_heads=kv_heads)
    check(extension, b)


def _prefill_schedule(schedule):
    return {"prefill_schedule": schedule}


@pytest.mark.parametrize("schedule", ["stream", "grid"])
@pytest.mark.parametrize("heads,kv_heads", [(16, 8), (6, 2), (3, 3)])
def test_prefill_schedules_on_a_ragged_batch(extension, device, schedule, heads, kv_heads):
    """Balanced stream shares cut long items between workgroups (merged afterwards);
    the grid runs every item whole. Prefixes from 0 to several thousand keys; GQA
    pairs (two heads per work item, a wave each) and odd groups (one head)."""
    options = _prefill_schedule(schedule)
    b = case([4000, 520, 17, 1300, 64], [512, 520, 9, 300, 2], device, dtype=torch.bfloat16,
             num_q_heads=heads, num_kv_heads=kv_heads, head_dim=128)
    plan = extension.paged_attention_plan(b.q.shape[0], 5, heads, kv_heads, 128, 16, 520, 4000,
                                          torch.bfloat16, torch.bfloat16, plan_options=options)
    assert plan["prefill_mfma"] == 1
    assert (plan["prefill_workgroups"] > 0) == (schedule == "stream")
    check(extension, b, options=options)


@pytest.mark.parametrize("decodes", [27, 66])
def test_prefill_stream_beside_many_decode_rows(extension, device, decodes):
    """Chunks cut between stream workgroups in batches of fewer and of more than 64
    sequences (the merge finds an item's sequence by a one-wave ballot below 64 and by
    a binary search above)."""
    gen = torch.Generator().manual_seed(decodes)
    contexts = torch.randint(1, 2300, (decodes,), generator=gen).tolist()
    b = case(contexts + [1600, 512, 900], [1] * decodes + [512, 512, 77], device,
             dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8, head_dim=128)
    check(extension, b, options={"prefill_schedule": "stream"})


@pytest.mark.parametrize("wgs_per_cu", ["1", "3"])
def test_prefill_stream_with_more_workgroups_than_tiles(extension, device, wgs_per_cu):
    """A two-tile prefill over hundreds of workgroups: most workgroups idle, and with
    one-tile shares each tile of an item sits in a different workgroup."""
    b = case([70, 3], [70, 3], device, dtype=torch.bfloat16, num_q_heads=4, num_kv_heads=2,
             head_dim=64)
    for tiles in ("1", "4"):
        check(extension, b, options={"prefill_wgs_per_cu": wgs_per_cu, "prefill_schedule": "stream",
                                     "prefill_share_tiles": tiles})


@pytest.mark.parametrize("tiles", ["1", "3", "64"])
def test_prefill_stream_share_sizes(extension, device, tiles):
    """Shares of one tile (every item cut into many pieces), of a few, and so large that
    the quarter-grid floor sets their number: the same attention."""
    b = case([2000, 700, 1300, 64], [512, 300, 512, 64], device, dtype=torch.bfloat16)
    check(extension, b, options={"prefill_schedule": "stream", "prefill_share_tiles": tiles})


@pytest.mark.parametrize("schedule", ["stream", "grid"])
def test_prefill_schedules_in_a_mixed_fp8_batch(extension, device, schedule):
    b = case([900, 2500, 40, 700], [1, 400, 40, 1], device, dtype=torch.bfloat16,
             kv_dtype=torch.float8_e4m3fn, num_q_heads=16, num_kv_heads=8, head_dim=128)
    check(extension, b, dtype=torch.float8_e4m3fn, options=_prefill_schedule(schedule))


@pytest.mark.parametrize("block_size", [16, 32, 64])
def test_fp8_prefill_on_the_pipelined_grid_kernel(extension, device, block_size):
    """fp8 pools on the grid schedule take the pipelined kernel (codes staged straight
    into LDS, dequantised there with each page's scale): ragged prefixes, partial last
    tiles, a decode row, pages of 16 to 64 keys."""
    b = case([1500, 700, 130, 65, 3000], [512, 300, 130, 1, 200], device, dtype=torch.bfloat16,
             kv_dtype=torch.float8_e4m3fn, num_q_heads=16, num_kv_heads=8, head_dim=128,
             block_size=block_size)
    check(extension, b, dtype=torch.float8_e4m3fn, options={"prefill_schedule": "grid"})


def _split(pieces, share_tiles=1):
    return {"prefill_schedule": "grid", "prefill_pieces": pieces,
            "prefill_share_tiles": share_tiles}


@pytest.mark.parametrize("pieces", [2, 3, 16])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_split_grid_cuts_long_items(extension, device, pieces, kv_dtype):
    """The grid cuts items longer than ~1.2x the mean work per CU into key ranges run by
    workgroups of their own in the same launch, the last piece to finish merging the
    others: a 6000-key prefix beside short chunks (its items cut into up to 5 pieces),
    ragged chunk ends, a decode row, an fp8 pool."""
    b = case([6000, 700, 130, 65, 3000], [512, 300, 130, 1, 200], device, dtype=torch.bfloat16,
             kv_dtype=kv_dtype, num_q_heads=16, num_kv_heads=8, head_dim=128)
    plan = extension.paged_attention_plan(b.q.shape[0], 5, 16, 8, 128, 16, 512, 6000,
                                          torch.bfloat16, kv_dtype, plan_options=_split(pieces))
    assert plan["prefill_pieces"] == pieces and plan["workspace_bytes"] > 0
    check(extension, b, dtype=kv_dtype, options=_split(pieces))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_grid_one_long_prompt(extension, device, dtype):
    """One sequence alone: every item long against the mean, so each is cut (up to 7
    pieces of ~13 tiles); whichever piece finishes last folds them in piece order, so
    three calls in a row give the same bits (and each finds the arrival counters left
    at zero by the one before)."""
    b = case([6100], [512], device, dtype=dtype, num_q_heads=16, num_kv_heads=8, head_dim=128)
    want = oracle(b)
    first = None
    for _ in range(3):
        got = kernel(extension, b, _split(16))
        assert_max_abs(got, want, ATTN_ATOL[dtype], "split, one long prompt")
        first = got if first is None else first
        assert torch.equal(got, first)


def test_split_grid_matches_the_whole_item_grid(extension, device):
    """Config 3's shape on the split grid (the default) and with every item whole: both
    within tolerance of the oracle and of each other."""
    b = config_batch(3, device=device)
    whole = kernel(extension, b, {"prefill_schedule": "grid", "prefill_pieces": 1})
    split = kernel(extension, b, {"prefill_schedule": "grid"})
    assert_max_abs(split.float(), whole.float(), 2 * ATTN_ATOL[torch.bfloat16], "split vs whole")


def test_split_grid_piece_lengths_and_bounds(extension, device):
    """Pieces at the floor of one tile and of many tiles, beside decode rows and a batch
    of 64 items (the most the split schedule takes), and of 65 (items stay whole)."""
    b = case([2000, 900, 64, 3000, 17], [512, 1, 64, 512, 1], device, dtype=torch.bfloat16,
             num_q_heads=16, num_kv_heads=8, head_dim=128)
    for tiles in (1, 8, 64):
        check(extension, b, options=_split(4, tiles))
    for seqs in (64, 65):
        gen = torch.Generator().manual_seed(seqs)
        ctx = torch.randint(40, 1500, (seqs,), generator=gen).tolist()
        lens = [min(c, 100) for c in ctx]
        bb = case(ctx, lens, device, dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8,
                  head_dim=128)
        plan = extension.paged_attention_plan(bb.q.shape[0], seqs, 16, 8, 128, 16, max(lens),
                                              max(ctx), torch.bfloat16, torch.bfloat16,
                                              plan_options=_split(4))
        assert (plan["prefill_pieces"] > 1) == (seqs <= 64)
        check(extension, bb, options=_split(4))


@pytest.mark.parametrize("schedule", ["stream", "grid"])
@pytest.mark.parametrize("scale", [-0.3, 0.0, 2.0])
def test_prefill_with_unusual_scales(extension, device, scale, schedule):
    """The softmax runs on raw scores with |scale| folded into the exponent and the sign
    of a negative scale moved into Q; zero gives uniform weights."""
    b = case([300, 90], [150, 90], device, dtype=torch.bfloat16, num_q_heads=16,
             num_kv_heads=8, head_dim=128)
    b.scale = scale
    check(extension, b, options=_prefill_schedule(schedule))


def test_prefill_schedule_choice(extension):
    """Grid when the items fill the CUs; stream for a chunk of a long prompt."""
    bf = torch.bfloat16
    many = extension.paged_attention_plan(4096, 8, 16, 8, 128, 16, 512, 2048, bf, bf)
    assert many["prefill_mfma"] == 1 and many["prefill_workgroups"] == 0
    chunk = extension.paged_attention_plan(543, 32, 16, 8, 128, 16, 512, 8192, bf, bf)
    assert chunk["prefill_mfma"] == 1 and chunk["prefill_workgroups"] > 0


@pytest.mark.parametrize("block_size", [1, 2, 64])
def test_mfma_prefill_block_sizes(extension, device, block_size):
    check(extension, case([180, 70], [100, 70], device, dtype=torch.bfloat16,
                          block_size=block_size, num_q_heads=16, num_kv_heads=8, head_dim=128))


def test_the_first_query_of_a_prompt_returns_its_own_value(extension, device):
    for dtype in (torch.float32, torch.bfloat16):
        b = case([12], [12], device, dtype=dtype)
        got = kernel(extension, b)
        first = b.value_pool[int(b.block_tables[0, 0]), 0]
        for h in range(HQ):
            assert torch.equal(got[0, h], first[h // (HQ // HK)]), f"{dtype} head {h}"


def test_output_is_a_convex_combination_of_visible_values(extension, device):
    b = case([64], [64], device)
    got = kernel(extension, b)
    visible = torch.stack([b.value_pool[int(x)] for x in b.block_tables[0]])
    assert got.min() >= visible.min() - 1e-4 and got.max() <= visible.max() + 1e-4


# ---------------------------------------------------------------- mixed batch


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_a_mixed_batch_gives_each_sequence_what_it_gets_alone(extension, device, dtype):
    contexts, lens = [300, 700, 4096, 50], [300, 1, 1, 50]
    b = case(contexts, lens, device, dtype=dtype)
    together = kernel(extension, b)
    for s in range(4):
        lo, hi = int(b.cu_seqlens_q[s]), int(b.cu_seqlens_q[s + 1])
        alone = extension.paged_attention(
            b.q[lo:hi].contiguous(), b.key_pool, b.value_pool, b.block_tables[s:s + 1].contiguous(),
            torch.tensor([0, hi - lo], dtype=torch.int32, device=device), b.context_lens[s:s + 1],
            b.seq_lens[s:s + 1], hi - lo, contexts[s], b.scale)
        torch.cuda.synchronize()
        assert_max_abs(together[lo:hi], alone, 1e-6 if dtype == torch.float32 else 1e-2,
                       f"sequence {s} changed in the batch")
    assert_max_abs(together, oracle(b), ATTN_ATOL[dtype])


def test_the_shuffle_is_what_is_being_tested(extension, device):
    ordered = case([200], [1], device, shuffle=False, spare_blocks=0)
    shuffled = case([200], [1], device, shuffle=True, spare_blocks=0)
    assert not torch.equal(ordered.block_tables, shuffled.block_tables)
    assert torch.equal(ordered.q, shuffled.q)
    check(extension, ordered)
    check(extension, shuffled)


def test_padding_and_spare_blocks_are_never_read(extension, device):
    b = case([33, 5, 100], [1, 1, 20], device, dtype=torch.bfloat16, spare_blocks=5)
    used = {int(x) for x in b.block_tables.flatten().cpu() if int(x) >= 0}
    for blk in range(b.key_pool.shape[0]):
        if blk not in used:
            b.key_pool[blk] = float("nan")
            b.value_pool[blk] = float("nan")
    assert torch.isfinite(kernel(extension, b)).all()


# -------------------------------------------------------------------- dtypes / fp8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_stays_within_tolerance(extension, device, dtype):
    check(extension, case([512, 77], [1, 1], device, dtype=dtype))


@pytest.mark.parametrize("lens", [([100, 2048, 17], [1, 1, 1]), ([300, 64], [100, 64])])
def test_fp8_kv_cache(extension, device, lens):
    b = case(*lens, device, dtype=torch.bfloat16, kv_dtype=torch.float8_e4m3fn,
             num_q_heads=16, num_kv_heads=8, head_dim=128)
    check(extension, b, dtype=torch.float8_e4m3fn)


def test_fp8_dequantisation_is_exact_for_one_visible_key(extension, device):
    """With one visible key the output is that key's dequantised value, rounded once."""
    b = case([12], [12], device, dtype=torch.bfloat16, kv_dtype=torch.float8_e4m3fn,
             num_q_heads=16, num_kv_heads=8, head_dim=128)
    got = kernel(extension, b)
    blk = int(b.block_tables[0, 0])
    want = (b.value_pool[blk, 0].float() * b.v_scale[blk][:, None]).to(torch.bfloat16)
    for h in range(16):
        assert torch.equal(got[0, h], want[h // 2])


@pytest.mark.parametrize("query_len", [1, 12])
def test_fp8_decodes_every_finite_code_exactly(extension, device, query_len):
    """Key 0's values cover all 254 finite e4m3fn codes with scale 1; a query that sees
    only key 0 (a decode over one key, or the first row of a prefill chunk) returns
    them decoded exactly (both representable in bf16)."""
    b = case([query_len], [query_len], device, dtype=torch.bfloat16,
             kv_dtype=torch.float8_e4m3fn, num_q_heads=16, num_kv_heads=8, head_dim=128)
    codes = torch.tensor([c for c in range(256) if c & 0x7F != 0x7F], dtype=torch.uint8)
    blk = int(b.block_tables[0, 0])
    row = codes.repeat(5)[: 8 * 128].reshape(8, 128).to(device)
    b.value_pool.view(torch.uint8)[blk, 0] = row
    b.v_scale[blk] = 1.0
    got = kernel(extension, b)
    want = row.view(torch.float8_e4m3fn).float().to(torch.bfloat16)
    for h in range(16):
        assert torch.equal(got[0, h], want[h // 2]), f"head {h}"


# ------------------------------------------------------------------- configs


def test_config1_fp32_matches_golden_and_oracle(extension, device):
    b = config_batch(1, device=device)
    gold = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "paged_cfg1.npz")
    got = kernel(extension, b)
    assert_max_abs(got, torch.from_numpy(gold["out"]), 2e-5, "config 1 vs golden")
    assert_max_abs(got, oracle(b), 2e-5, "config 1 vs oracle")


@pytest.mark.slow
def test_config2_bf16_decode_full_size(extension, device):
    b = config_batch(2, device=device)
    check(extension, b, msg="config 2")


@pytest.mark.slow
def test_config3_chunked_prefill_full_size(extension, device):
    b = config_batch(3, device=device)
    assert prefill_flops(b) > 1e10
    check(extension, b, msg="config 3")


@pytest.mark.slow
def test_config3_chunked_prefill_over_an_fp8_pool_full_size(extension, device):
    """Config 3's shape (8 x 512-token chunks after prefixes U[0,1536]) over an fp8 pool
    quantised per (block, kv head), every row against the oracle's dequantise-then-dense
    path at the fp8 tolerance."""
    b = config_batch(3, device=device, kv_dtype=torch.float8_e4m3fn)
    assert b.key_pool.dtype == torch.float8_e4m3fn and prefill_flops(b) > 1e10
    check(extension, b, msg="config 3, fp8 pool")


@pytest.mark.slow
def test_config4_fp8_decode_full_size(extension, device):
    """The full config-4 batch (128 sequences of 2048-8192 fp8 keys) on the GPU, every
    row checked against the CPU oracle, 32 sequences per oracle call (sequences are
    independent, so the groups together are the whole check)."""
    b = config_batch(4, device=device)
    got = kernel(extension, b).cpu()
    pools = (b.key_pool.cpu(), b.value_pool.cpu(), b.k_scale.cpu(), b.v_scale.cpu())
    for lo in range(0, 128, 32):
        picks = list(range(lo, lo + 32))
        rows = torch.tensor([int(b.cu_seqlens_q[s]) for s in picks])
        sub = oracle_paged(b.q[rows].cpu(), pools[0], pools[1], b.block_tables[picks].cpu(),
                           torch.arange(len(picks) + 1, dtype=torch.int32),
                           b.context_lens[picks].cpu(), b.scale, pools[2], pools[3])
        assert_max_abs(got[rows], sub, ATTN_ATOL[torch.float8_e4m3fn], f"config 4 rows {lo}+")


def test_repeated_calls_are_deterministic(extension, device):
    b = case([3000, 40], [1, 40], device, dtype=torch.bfloat16, num_q_heads=16, num_kv_heads=8,
             head_dim=128)
    first = kernel(extension, b)
    for _ in range(3):
        assert torch.equal(kernel(extension, b), first)


# ------------------------------------------------------------------- refusals


def _call(ext, b, **over):
    args = dict(q=b.q, key_pool=b.key_pool, value_pool=b.value_pool,
                block_tables=b.block_tables, cu_seqlens_q=b.cu_seqlens_q,
                context_lens=b.context_lens, seq_lens=b.seq_lens, max_query_len=1,
                max_context_len=64, scale=b.scale)
    args.update(over)
    return ext.paged_attention(*args.values())


@pytest.mark.parametrize("mutate,message", [
    (lambda b: dict(key_pool=b.key_pool.narrow(0, 0, b.key_pool.shape[0] - 1)[::2],
                    value_pool=b.key_pool.narrow(0, 0, b.key_pool.shape[0] - 1)[::2]), "contiguous"),
    (lambda b: dict(key_pool=b.key_pool.repeat(1, 3, 1, 1)[:, :3].contiguous(),
                    value_pool=b.key_pool.repeat(1, 3, 1, 1)[:, :3].contiguous()), "power of two"),
    (lambda b: dict(block_tables=b.block_tables.long()), "int32"),
    (lambda b: dict(q=b.q.unsqueeze(0)), "T x H_q x D"),
    (lambda b: dict(max_query_len=8, max_context_len=4), "at least max_query_len"),
    (lambda b: dict(q=b.q.double(), key_pool=b.key_pool.double(), value_pool=b.value_pool.double()),
     "float64"),
    (lambda b: dict(q=b.q.to(torch.bfloat16)), "must share a dtype"),
])
def test_refusals(extension, device, mutate, message):
    b = case([64], [1], device)
    with pytest.raises(RuntimeError, match=message):
        _call(extension, b, **mutate(b))


def test_fp8_pool_without_scales_is_refused(extension, device):
    b = case([64], [1], device, dtype=torch.bfloat16, kv_dtype=torch.float8_e4m3fn)
    with pytest.raises(RuntimeError, match="k_scale"):
        extension.paged_attention(*b.args())


# ------------------------------------------------------------------- dispatch


def test_the_op_routes_to_the_kernel(extension, device, monkeypatch):
    b = case([256], [1], device)
    calls = []
    original = extension.paged_attention

    def spy(*args, **kwargs):
        calls.append(args)
        return original(*args, **kwargs)

    monkeypatch.setattr(extension, "paged_attention", spy)
    got = ops.paged_attention(*b.args(), use_cuda=True)
    torch.cuda.synchronize()
    assert len(calls) == 1, "use_cuda=True did not reach the kernel"
    assert_max_abs(got, oracle(b), ATTN_ATOL[torch.float32])


def test_strict_mode_refuses_what_the_kernel_cannot_serve(extension, device):
    b = case([64], [1], device)
    with pytest.raises(RuntimeError, match="contiguous"):
        ops.paged_attention(b.q, b.key_pool[::2], b.value_pool[::2], *b.args()[3:],
                            use_cuda=True)


def test_declined_calls_fall_back_to_the_pytorch_path_on_device(extension, device):
    """Outside strict mode a call the kernel cannot serve (a strided pool, a head dim
    outside 32/64/128/256) runs the PyTorch path on the device, as the reference's
    ``_kernel_can_page`` routes it (ops.py:257-275), and is reported."""
    ops.FALLBACKS.clear()
    with ops.strict_kernels(False):
        b = case([64, 9], [1, 9], device)

        def strided(pool):  # the same pool as a non-contiguous view
            wide = torch.zeros(*pool.shape[:-1], 2 * pool.shape[-1], dtype=pool.dtype,
                               device=pool.device)
            wide[..., :pool.shape[-1]] = pool
            return wide[..., :pool.shape[-1]]

        kp, vp = strided(b.key_pool), strided(b.value_pool)
        got = ops.paged_attention(b.q, kp, vp, *b.args()[3:], use_cuda=True)
        want = ops.paged_attention(b.q, kp, vp, *b.args()[3:], use_cuda=False)
        assert torch.equal(got, want)
        assert_max_abs(got, oracle(b), ATTN_ATOL[torch.float32])
        b48 = case([40, 7], [1, 7], device, head_dim=48)
        assert_max_abs(ops.paged_attention(*b48.args(), use_cuda=True), oracle(b48), 1e-5)
    assert "contiguous" in ops.dispatch_report(True) and "head dim 48" in ops.dispatch_report(True)


def test_the_torch_path_runs_on_device_without_cuda_requested(extension, device):
    b = case([256, 30], [1, 30], device)
    got = ops.paged_attention(*b.args(), use_cuda=False)
    assert_max_abs(got, oracle(b), 1e-5)


def test_a_captured_split_prefill_runs_items_whole(extension, device):
    """A split-grid prefill captured into a graph must not name its stream's arrival
    counters (a replay on another stream could overlap a launch on the capture stream):
    captured, it runs every item whole - counted by split_stats - and each replay, also
    on another stream, matches the oracle and the eager whole-item call's bits."""
    b = case([6000, 700], [512, 300], device, dtype=torch.bfloat16, num_q_heads=16,
             num_kv_heads=8, head_dim=128)
    opts = _split(8)
    whole = kernel(extension, b, {"prefill_schedule": "grid", "prefill_pieces": 1})
    kernel(extension, b, opts)  # eager warm-up: the workspace exists before capture
    before = extension.split_stats()["whole_capturing"]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out = extension.paged_attention(*b.args(), plan_options=opts)
    assert extension.split_stats()["whole_capturing"] > before
    want = oracle(b)
    other = torch.cuda.Stream()
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        if i == 2:
            with torch.cuda.stream(other):
                graph.replay()
        else:
            graph.replay()
        torch.cuda.synchronize()
        assert_max_abs(out, want, ATTN_ATOL[torch.bfloat16], f"replay {i}")
        assert torch.equal(out, whole)
