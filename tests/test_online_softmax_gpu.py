"""The online-softmax recurrence under directed inputs, on every HIP attention path
(``-m gpu``).

The reference pins its rescale with known answers (tests/test_decode_attention_cuda.py:
85-175): a late spike, which every accumulator must be rescaled by; an early spike, on
which a correction of the wrong sign is still right (so the two go together); a spike in
the last split, which the merge must rescale the earlier splits by; scores near the
exponential's overflow. Random N(0, 1) inputs at scale 1/sqrt(D) keep every score O(1)
and leave these paths idle, so here they are driven on purpose:

* decode: the stream schedule (a sequence cut into many shares, merged by the merge
  kernel) with the spike in its first, a middle and its last share, and the grid
  schedule (splits of 64-1024 keys, its own merge);
* prefill: the item grid, the split grid (long items cut into key-range pieces in one
  launch, the last piece folding the others), the stream schedule (shares of all key
  tiles, cut items merged after), the register-staged kernel, and fp32 rows (the
  decode kernel run by row);
* the prefill kernels' lazy rescale: the running max is raised only when a tile's max
  exceeds it by more than 8 log2 units, so a staircase of scores with steps just below
  and just above that slack, placed in different tiles, split pieces and stream shares,
  takes both branches several times within one item;
* the dense-cache entries (decode and causal prefill on virtual pages);
* 16-bit and fp8-e4m3 pools (per-(page, kv head) scales).

Every case is compared with the fp32 oracle (oracle/paged_attention.py,
oracle/dense_attention.py) at the north-star tolerances (max-abs fp32 2e-5, fp16 1e-2,
bf16 2e-2, fp8 KV 6e-2); the spike cases also check the known answer itself (the
output is the spike key's value within 1%, as the reference's
``assert_relative_error_below`` does), so a kernel that dropped the spike fails too.
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import ATTN_ATOL, assert_max_abs
from mini_vllm.workloads import build_batch, quantize_fp8_per_block
from oracle.dense_attention import dense_attention as dense_oracle
from oracle.paged_attention import paged_attention as oracle_paged

pytestmark = pytest.mark.gpu

HQ, HK, D, P = 16, 8, 128, 16


def directed(contexts, query_lens, *, dtype, kv_dtype=None, scores=(), base=0.0,
             q_fill=1.0, hq=HQ, hk=HK, d=D, block_size=P, seed=0):
    """A paged batch whose queries are all ``q_fill`` and whose keys are all ``base``
    except ``scores``: (sequence, key position, score) entries whose key is set so that
    every query's score against it (q . k x scale, natural log units) is ``score``.
    Values stay N(0, 1). The pool is edited in fp32 and then cast to ``dtype`` or
    quantised per (page, kv head) for an fp8 pool, so the oracle sees the stored keys."""
    b = build_batch(contexts, query_lens, dtype=torch.float32, num_q_heads=hq,
                    num_kv_heads=hk, head_dim=d, block_size=block_size, seed=seed)
    b.key_pool.fill_(base)
    b.q.fill_(q_fill)
    per_unit = q_fill * d * b.scale  # score of a key whose elements are all 1
    for seq, pos, score in scores:
        blk = int(b.block_tables[seq, pos // block_size])
        b.key_pool[blk, pos % block_size] = score / per_unit
    kv_dtype = kv_dtype or dtype
    if kv_dtype == torch.float8_e4m3fn:
        b.key_pool, b.k_scale = quantize_fp8_per_block(b.key_pool)
        b.value_pool, b.v_scale = quantize_fp8_per_block(b.value_pool)
    else:
        b.key_pool, b.value_pool = b.key_pool.to(kv_dtype), b.value_pool.to(kv_dtype)
    b.q = b.q.to(dtype)
    return b.to("cuda")


def run(ext, b, options=None):
    out = ext.paged_attention(*b.args(), k_scale=b.k_scale, v_scale=b.v_scale,
                              plan_options=options)
    torch.cuda.synchronize()
    return out


def oracle(b):
    return oracle_paged(b.q, b.key_pool, b.value_pool, b.block_tables, b.cu_seqlens_q,
                        b.context_lens, b.scale, b.k_scale, b.v_scale)


def value_of(b, seq, pos):
    """The stored value rows of a key (``H_k x D``), dequantised for an fp8 pool."""
    blk = int(b.block_tables[seq, pos // P])
    v = b.value_pool[blk, pos % P].float()
    if b.v_scale is not None:
        v = v * b.v_scale[blk][:, None]
    return v


def assert_answer(got_rows, want_kv_rows, rel, msg):
    """Each query head's output is its kv head's ``want`` within relative error
    ``rel`` (in norm), as the reference's known-answer checks do."""
    got = got_rows.float().cpu()                        # rows x H_q x D
    want = want_kv_rows.float().cpu().repeat_interleave(got.shape[1] // want_kv_rows.shape[0], 0)
    err = ((got - want).norm(dim=-1) / want.norm(dim=-1)).max().item()
    assert err <= rel, f"{msg}: relative error {err:.3e} > {rel}"


def tol(dtype, kv_dtype=None):
    return ATTN_ATOL[kv_dtype or dtype]


KV_POOLS = [None, torch.float8_e4m3fn]
KV_IDS = ["16-bit", "fp8"]

# ---------------------------------------------------------------------- decode

DECODE_PATHS = {
    "stream": None,                                   # default: shares + merge kernel
    "grid": {"decode_schedule": "grid"},              # splits + grid merge kernel
    "grid-64": {"decode_schedule": "grid", "decode_split_tokens": 64},
}


@pytest.mark.parametrize("path", sorted(DECODE_PATHS))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_late_spike(extension, device, path, dtype):
    """The reference's late spike (``test_survives_a_late_spike``): keys 0.01, the last
    of 200 aligned with the query (score ~22.6 against ~0.11); the output is its value."""
    b = directed([200], [1], dtype=dtype, base=0.01, scores=[(0, 199, 22.6)])
    got = run(extension, b, DECODE_PATHS[path])
    assert_max_abs(got, oracle(b), tol(dtype), f"{path} late spike")
    assert_answer(got, value_of(b, 0, 199), 0.01, f"{path} late spike")


@pytest.mark.parametrize("path", sorted(DECODE_PATHS))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_early_spike(extension, device, path, dtype):
    """The mirror image (``test_survives_an_early_spike``): the maximum comes first, so
    every later correction is 1; a correction of the wrong sign passes this one and
    fails the late spike."""
    b = directed([200], [1], dtype=dtype, base=0.01, scores=[(0, 0, 11.3)])
    got = run(extension, b, DECODE_PATHS[path])
    assert_max_abs(got, oracle(b), tol(dtype), f"{path} early spike")


@pytest.mark.parametrize("kv_dtype", KV_POOLS, ids=KV_IDS)
@pytest.mark.parametrize("where", ["first", "middle", "last"])
@pytest.mark.parametrize("path", sorted(DECODE_PATHS))
def test_decode_spike_in_each_piece(extension, device, path, where, kv_dtype):
    """``test_the_merge_rescales_across_splits`` and its neighbours: one 8192-key
    sequence is cut into dozens of stream shares (or grid splits); the spike sits in the
    first, a middle or the last piece, so the merge must rescale every other piece by
    it. A second sequence shares the launch (its shares sit between)."""
    pos = {"first": 3, "middle": 4133, "last": 8191}[where]
    b = directed([8192, 3000], [1, 1], dtype=torch.bfloat16, kv_dtype=kv_dtype, base=0.01,
                 scores=[(0, pos, 22.6), (1, 2999, 22.6)])
    plan = extension.paged_attention_plan(2, 2, HQ, HK, D, P, 1, 8192, torch.bfloat16,
                                          kv_dtype or torch.bfloat16,
                                          plan_options=DECODE_PATHS[path])
    assert plan["decode_workgroups"] > 8, plan  # the sequence really is cut
    got = run(extension, b, DECODE_PATHS[path])
    assert_max_abs(got, oracle(b), tol(torch.bfloat16, kv_dtype), f"{path} spike {where}")
    assert_answer(got[:1], value_of(b, 0, pos), 0.01, f"{path} spike {where}")
    assert_answer(got[1:], value_of(b, 1, 2999), 0.01, f"{path} second sequence")


@pytest.mark.parametrize("kv_dtype", KV_POOLS, ids=KV_IDS)
@pytest.mark.parametrize("path", sorted(DECODE_PATHS))
def test_decode_staircase_across_pieces(extension, device, path, kv_dtype):
    """Scores rising in steps of 6 (natural log units) from piece to piece, so the
    merge's running maximum moves at every piece, beside sequences of one piece; no
    step dominates the sum so much that a missed rescale would hide (each step's weight
    is e^6 times the last, a missed rescale overweights the earlier ones by as much)."""
    steps = [(0, 500 * i + 7, 6.0 * i) for i in range(1, 16)]
    b = directed([8000, 40, 900], [1, 1, 1], dtype=torch.bfloat16, kv_dtype=kv_dtype,
                 scores=steps + [(2, 5, 4.0), (2, 800, 10.0)])
    got = run(extension, b, DECODE_PATHS[path])
    assert_max_abs(got, oracle(b), tol(torch.bfloat16, kv_dtype), f"{path} staircase")


@pytest.mark.parametrize("dtype,kv_dtype", [(torch.float32, None), (torch.bfloat16, None),
                                            (torch.bfloat16, torch.float8_e4m3fn)],
                         ids=["fp32", "bf16", "bf16-fp8"])
@pytest.mark.parametrize("path", sorted(DECODE_PATHS))
def test_decode_logits_that_would_overflow(extension, device, path, dtype, kv_dtype):
    """``test_handles_logits_that_would_overflow``: q = k = 30, so every score is
    30 * 30 * 128 / sqrt(128) ~ 10182, far past exp's range; subtracting the running max
    makes every weight 1 and the output the mean of the values. One short sequence and
    one cut into many pieces."""
    b = directed([100, 5000], [1, 1], dtype=dtype, kv_dtype=kv_dtype, base=30.0, q_fill=30.0)
    got = run(extension, b, DECODE_PATHS[path])
    assert torch.isfinite(got).all(), "the running max is not being subtracted"
    assert_max_abs(got, oracle(b), tol(dtype, kv_dtype), f"{path} overflow")


# --------------------------------------------------------------------- prefill

PREFILL_PATHS = {
    "item-grid": {"prefill_schedule": "grid", "prefill_pieces": 1},
    "split-grid": {"prefill_schedule": "grid", "prefill_pieces": 16},
    "stream": {"prefill_schedule": "stream"},
    "stream-1-tile": {"prefill_schedule": "stream", "prefill_share_tiles": 1},
    "register-staged": {"prefill_schedule": "grid", "prefill_staging": 1},
}

# A staircase over a 3000-key prefix: steps of +3 (4.3 log2 units: under the kernels'
# 8-unit slack, so the running max is left alone and the exponentials grow to 2^4.3)
# and of +6 (8.7 units: the max is raised and O and l rescaled), in tiles 1, 10, 23,
# 34 and 46 of the 64-key walk; one more spike inside the 512-token chunk, seen only by
# the rows after it.
PREFIX = 3000
STAIRCASE = [(100, 3.0), (700, 9.0), (1500, 12.0), (2200, 18.0), (2990, 21.0),
             (PREFIX + 200, 24.0)]


def _staircase_batch(dtype, kv_dtype, extra=()):
    scores = [(0, pos, s) for pos, s in STAIRCASE] + list(extra)
    return directed([PREFIX + 512, 900, 130], [512, 300, 1], dtype=dtype, kv_dtype=kv_dtype,
                    scores=scores + [(1, 650, 14.0), (1, 20, 7.0)])


@pytest.mark.parametrize("kv_dtype", KV_POOLS, ids=KV_IDS)
@pytest.mark.parametrize("path", sorted(PREFILL_PATHS))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_lazy_rescale_staircase(extension, device, path, dtype, kv_dtype):
    """Both branches of the lazy rescale within one item, with steps landing in
    different key tiles, split pieces and stream shares; rows before the chunk's spike
    must not see it (the causal mask), rows after it are dominated by it."""
    b = _staircase_batch(dtype, kv_dtype)
    plan = extension.paged_attention_plan(b.q.shape[0], 3, HQ, HK, D, P, 512, PREFIX + 512,
                                          dtype, kv_dtype or dtype,
                                          plan_options=PREFILL_PATHS[path])
    assert plan["prefill_mfma"] == 1
    if path == "split-grid":
        assert plan["prefill_pieces"] > 1
    got = run(extension, b, PREFILL_PATHS[path])
    assert_max_abs(got, oracle(b), tol(dtype, kv_dtype), f"{path} staircase")
    # the chunk's spike (score 24, e^3 above the prefix's best) carries > 95% of the
    # weight of every row that sees it
    rows = got[300:512]
    assert_answer(rows, value_of(b, 0, PREFIX + 200), 0.1, f"{path} rows after the spike")


@pytest.mark.parametrize("kv_dtype", KV_POOLS, ids=KV_IDS)
@pytest.mark.parametrize("path", sorted(PREFILL_PATHS))
def test_prefill_late_and_early_spikes(extension, device, path, kv_dtype):
    """The reference's late and early spikes for every row of a chunk: one key at the
    end of a long prefix (the last tile every row walks before the chunk) and one at its
    start, in separate sequences; every row's output is that key's value."""
    late, early = 2047, 0
    b = directed([2048 + 256, 2048 + 256], [256, 256], dtype=torch.bfloat16,
                 kv_dtype=kv_dtype, base=0.01, scores=[(0, late, 22.6), (1, early, 22.6)])
    got = run(extension, b, PREFILL_PATHS[path])
    assert_max_abs(got, oracle(b), tol(torch.bfloat16, kv_dtype), f"{path} spikes")
    assert_answer(got[:256], value_of(b, 0, late), 0.01, f"{path} late spike")
    assert_answer(got[256:], value_of(b, 1, early), 0.01, f"{path} early spike")


@pytest.mark.parametrize("kv_dtype", KV_POOLS, ids=KV_IDS)
@pytest.mark.parametrize("path", sorted(PREFILL_PATHS))
def test_prefill_logits_that_would_overflow(extension, device, path, kv_dtype):
    """q = k = 30 for every row of a chunk after a prefix: all visible scores ~10182,
    every weight 1, row r's output the mean of the values it sees (the causal mask
    still applies at that scale)."""
    b = directed([1700, 300], [600, 300], dtype=torch.bfloat16, kv_dtype=kv_dtype,
                 base=30.0, q_fill=30.0)
    got = run(extension, b, PREFILL_PATHS[path])
    assert torch.isfinite(got).all(), "the running max is not being subtracted"
    assert_max_abs(got, oracle(b), tol(torch.bfloat16, kv_dtype), f"{path} overflow")


@pytest.mark.parametrize("path", ["stream", "item-grid", "split-grid"])
def test_prefill_one_long_prompt_spike_in_each_piece(extension, device, path):
    """One 512-query chunk after a 6000-key prefix, whose items the split grid cuts into
    up to 16 pieces and the stream schedule into shares: a staircase of +6 steps every
    400 keys moves the maximum in nearly every piece, and the merge of the pieces must
    rescale them all."""
    steps = [(0, 400 * i + 13, 6.0 * i) for i in range(1, 16)]
    b = directed([6512], [512], dtype=torch.bfloat16, scores=steps)
    got = run(extension, b, PREFILL_PATHS[path])
    assert_max_abs(got, oracle(b), tol(torch.bfloat16), f"{path} pieces")


@pytest.mark.parametrize("scores", [[(0, 40, 22.6)], [(0, 0, 11.3), (0, 70, 3.0)]],
                         ids=["late", "early"])
def test_fp32_prefill_rows_spikes(extension, device, scores):
    """fp32 prefill rows run on the decode kernel by row (no MFMA for fp32): the late
    and early spikes and the overflow case for every row of a chunk."""
    b = directed([80, 9], [60, 9], dtype=torch.float32, base=0.01, scores=scores)
    assert_max_abs(run(extension, b), oracle(b), tol(torch.float32), "fp32 rows")
    b = directed([80, 9], [60, 9], dtype=torch.float32, base=30.0, q_fill=30.0)
    got = run(extension, b)
    assert torch.isfinite(got).all()
    assert_max_abs(got, oracle(b), tol(torch.float32), "fp32 rows overflow")


# ----------------------------------------------------------------------- dense


def _dense(b, hq, hk, L, S, d, dtype, base, q_fill, scores):
    q = torch.full((b, hq, L, d), q_fill)
    k = torch.full((b, hk, S, d), base)
    gen = torch.Generator().manual_seed(S + L)
    v = torch.randn(b, hk, S, d, generator=gen)
    per_unit = q_fill * d / math.sqrt(d)
    for batch, pos, score in scores:
        k[batch, :, pos] = score / per_unit
    return q.to(dtype).cuda(), k.to(dtype).cuda(), v.to(dtype).cuda()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", ["late", "early", "staircase", "overflow"])
def test_dense_decode_and_prefill(extension, device, case, dtype):
    """The dense-cache entries (the paged kernels over virtual pages): decode over a
    4097-key cache (cut into pieces) and causal prefill of 300 rows after 1800 keys."""
    spec = {
        "late": dict(base=0.01, q_fill=1.0, scores=[(0, 4096, 22.6), (1, 1799, 22.6)]),
        "early": dict(base=0.01, q_fill=1.0, scores=[(0, 0, 11.3), (1, 0, 11.3)]),
        "staircase": dict(base=0.0, q_fill=1.0,
                          scores=[(0, 250 * i + 3, 6.0 * i) for i in range(1, 8)] +
                                 [(1, 230 * i + 3, 3.0 * i) for i in range(1, 8)]),
        "overflow": dict(base=30.0, q_fill=30.0, scores=[]),
    }[case]
    d = 128
    q, k, v = _dense(2, 16, 8, 1, 4097, d, dtype, **spec)
    got = extension.decode_attention(q, k, v, d ** -0.5)
    assert torch.isfinite(got).all()
    assert_max_abs(got, dense_oracle(q, k, v), ATTN_ATOL[dtype], f"dense decode {case}")
    scores = [(bb, p, s) for bb, p, s in spec["scores"] if p < 2100]
    q, k, v = _dense(2, 16, 8, 300, 2100, d, dtype, spec["base"], spec["q_fill"], scores)
    got = extension.flash_prefill(q, k, v, d ** -0.5)
    assert torch.isfinite(got).all()
    assert_max_abs(got, dense_oracle(q, k, v), ATTN_ATOL[dtype], f"dense prefill {case}")
