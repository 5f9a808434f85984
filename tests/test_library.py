"""The C-ABI library on the CPU: it loads, exports every declared symbol, and refuses
bad arguments with the reference's messages before touching a GPU."""

from __future__ import annotations

import ctypes
import re

import pytest
import torch

from mini_vllm.kernels import extension
from mini_vllm.kernels.extension import EXPORTED_SYMBOLS, INCLUDE_DIR, open_library

HEADER = INCLUDE_DIR / "minivllm_hip.h"


@pytest.fixture(scope="module")
def lib():
    if not extension.LIB_PATH.exists():
        extension.build_library()
    return open_library()


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(mvllm_\w+)\s*\(", text, re.M))


def test_every_declared_symbol_is_exported(lib):
    declared = declared_functions()
    assert declared == set(EXPORTED_SYMBOLS), declared ^ set(EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), f"{name} is declared in {HEADER.name} but not exported"


def test_abi_version(lib):
    assert lib.mvllm_abi_version() == extension.ABI_VERSION
    assert lib.mvllm_last_error() == b""


def _paged(lib, **over):
    args = dict(out=1, q=1, key_pool=1, value_pool=1, k_scales=None, v_scales=None,
                block_tables=1, cu=1, ctx=1, seq=1, num_tokens=4, num_seqs=4, hq=16, hk=8,
                d=128, p=16, num_blocks=512, max_blocks=63, max_q=1, max_ctx=1000, scale=0.088,
                q_dtype=0, kv_dtype=0, options=None, ws=None, ws_bytes=0, stream=None)
    args.update(over)
    return lib.mvllm_paged_attention(*args.values())


@pytest.mark.parametrize("over,code,message", [
    (dict(p=3), 1, "power of two"),
    (dict(hq=12), 1, "must be a multiple of H_k"),
    (dict(max_q=8, max_ctx=4), 1, "at least max_query_len"),
    (dict(max_q=0), 1, "max_query_len must be >= 1"),
    (dict(d=96), 2, "head dim 96 is not supported"),
    (dict(q_dtype=5), 1, "float64 is not supported"),
    (dict(q_dtype=2, kv_dtype=0), 1, "must share a dtype"),
    (dict(q_dtype=2, kv_dtype=3), 1, "k_scales and v_scales"),
    (dict(out=None), 1, "NULL"),
])
def test_paged_attention_refusals(lib, over, code, message):
    assert _paged(lib, **over) == code
    assert message in lib.mvllm_last_error().decode()


def test_blas_linear_takes_the_callers_workspace(lib):
    """The hipBLASLt entry allocates nothing: a missing, short or misaligned workspace is
    refused before any HIP call."""
    need = lib.mvllm_blas_workspace_bytes()
    assert need >= 1 << 20
    for ws, nbytes in ((None, need), (4096, need - 1), (4096 + 16, need)):
        assert lib.mvllm_blas_linear(256, 512, 768, 64, 128, 128, 2, ws, nbytes, None) == 1
        assert "workspace" in lib.mvllm_last_error().decode()


def test_split_workspace_is_required_when_planned(lib):
    """Decode needs its partials workspace; a missing one is refused, not faulted."""
    assert _paged(lib, num_tokens=1, num_seqs=1, max_ctx=8192) == 4
    assert "workspace" in lib.mvllm_last_error().decode()


def _plan(lib, *args, options=None):
    plan = extension._Plan()
    opts = extension.make_plan_options(options)
    assert lib.mvllm_paged_attention_plan(*args, None if opts is None else ctypes.byref(opts),
                                          ctypes.byref(plan)) == 0
    return plan


SLOT_BYTES = 8 * 64 * 66 * 4  # one piece's (m, l, O) partial: 8 waves x 64 lanes


def test_prefill_grid_schedule_workspace(lib):
    """Enough 128-query items to fill the CUs: the grid schedule. Where the pipelined
    kernel runs it (D 128, GQA pairs, 16-bit or fp8 pools, <= 64 items) it may cut long
    items into pieces, whose partial slots are the only workspace it needs; with
    prefill_pieces = 1 (or where the pipelined kernel does not run) it needs none."""
    plan = _plan(lib, 4096, 8, 16, 8, 128, 16, 512, 2048, 2, 2)
    assert plan.prefill_mfma == 1 and plan.prefill_workgroups == 0
    assert plan.prefill_pieces == 8
    # at most 2 * ceil(100 cus / (150 cols)) slots per column, 8 columns (256 CUs without
    # a GPU)
    assert 0 < plan.workspace_bytes <= 2 * 22 * 8 * SLOT_BYTES + 256
    whole = _plan(lib, 4096, 8, 16, 8, 128, 16, 512, 2048, 2, 2, options={"prefill_pieces": 1})
    assert whole.prefill_pieces == 0 and whole.workspace_bytes == 0
    fp8 = _plan(lib, 4096, 8, 16, 8, 128, 16, 512, 2048, 2, 3)
    assert fp8.prefill_pieces == 8
    for args in [(4096, 8, 16, 8, 64, 16, 512, 2048, 2, 2),    # D 64: the item kernel
                 (4096, 8, 12, 4, 128, 16, 512, 2048, 2, 2),   # groups of 3: one head a wave
                 (4096, 8, 16, 8, 128, 8, 512, 2048, 2, 2),    # pages of 8 keys
                 (8192, 128, 16, 8, 128, 16, 64, 2048, 2, 2)]:  # 128 items > 64
        other = _plan(lib, *args)
        assert other.prefill_pieces == 0 and other.workspace_bytes == 0, args
    plan = _plan(lib, 512, 1, 16, 8, 128, 16, 512, 8192, 2, 2,
                 options={"prefill_schedule": "grid", "prefill_pieces": 1})
    assert plan.prefill_workgroups == 0 and plan.workspace_bytes == 0
    plan = _plan(lib, 4096, 8, 16, 8, 128, 16, 512, 2048, 2, 2,
                 options={"prefill_schedule": "stream"})
    assert plan.prefill_workgroups > 0 and plan.prefill_pieces == 0


def test_plan_options_are_explicit_and_checked(lib, monkeypatch):
    """The schedule depends on the sizes and the options only: no environment knob."""
    monkeypatch.setenv("MVLLM_DECODE_SCHEDULE", "2")
    monkeypatch.setenv("MVLLM_PREFILL_SCHEDULE", "1")
    assert _plan(lib, 64, 64, 16, 8, 128, 16, 1, 4096, 2, 2).decode_mode == 1
    assert _plan(lib, 4096, 8, 16, 8, 128, 16, 512, 2048, 2, 2).prefill_workgroups == 0
    grid = _plan(lib, 64, 64, 16, 8, 128, 16, 1, 4096, 2, 2,
                 options={"decode_schedule": "grid", "decode_split_tokens": 1024})
    assert grid.decode_mode == 2 and grid.split_tokens == 1024
    bad = extension.make_plan_options({"prefill_staging": 2})
    plan = extension._Plan()
    assert lib.mvllm_paged_attention_plan(64, 64, 16, 8, 128, 16, 1, 4096, 2, 2,
                                          ctypes.byref(bad), ctypes.byref(plan)) == 1
    assert "plan options" in lib.mvllm_last_error().decode()
    with pytest.raises(ValueError, match="unknown plan options"):
        extension.make_plan_options({"decode_sched": 1})


def test_only_the_stream_and_grid_decode_schedules_can_be_forced(lib):
    """By-row is the planner's own choice for prefill rows without an MFMA kernel, not a
    schedule one can force; codes past the grid are refused."""
    for bad in ({"decode_schedule": 3}, {"decode_schedule": 4}):
        opts = extension.make_plan_options(bad)
        assert lib.mvllm_paged_attention_plan(32, 32, 16, 8, 128, 16, 1, 4096, 2, 2,
                                              ctypes.byref(opts), ctypes.byref(extension._Plan())) == 1
        assert "plan options" in lib.mvllm_last_error().decode()


def test_the_library_carries_the_id_of_its_sources(lib):
    assert lib.mvllm_build_id().decode() == extension.source_hash()


def test_plan_is_host_only_and_consistent(lib):
    # pure decode: the stream schedule, partial slots for (workgroups + sequences) x H_q
    plan = _plan(lib, 64, 64, 16, 8, 128, 16, 1, 4096, 2, 2)
    assert plan.decode_mode == 1 and plan.prefill_mfma == 0
    assert 1 <= plan.decode_workgroups
    entries = (plan.decode_workgroups + 64) * 16
    assert plan.workspace_bytes >= entries * (128 + 2) * 4 + 65 * 4
    # one prefill chunk in bf16 (fewer 128-query items than CUs): no decode launch,
    # MFMA prefill on the stream schedule, whose partial slots (two per workgroup,
    # 2 heads x 128 rows each) and per-sequence prefix make up the workspace
    plan = _plan(lib, 512, 1, 16, 8, 128, 16, 512, 8192, 2, 2)
    assert plan.decode_mode == 0 and plan.prefill_mfma == 1 and plan.prefill_workgroups >= 1
    rows = 2 * plan.prefill_workgroups * 2 * 128
    assert plan.workspace_bytes >= rows * (128 + 2) * 4 + 2 * 4
    # mixed bf16 batch: stream decode + MFMA prefill, both workspaces
    plan = _plan(lib, 101, 2, 16, 8, 128, 16, 100, 2048, 2, 2)
    assert plan.decode_mode == 1 and plan.prefill_mfma == 1 and plan.prefill_workgroups >= 1
    decode_part = (plan.decode_workgroups + 2) * 16 * (128 + 2) * 4
    assert plan.workspace_bytes >= decode_part + 2 * plan.prefill_workgroups * 2 * 128 * 130 * 4
    # fp32 prefill has no MFMA kernel: the decode kernel serves every row
    plan = _plan(lib, 100, 4, 16, 8, 128, 16, 40, 2048, 0, 0)
    assert plan.decode_mode == 3 and plan.prefill_mfma == 0
    assert 64 <= plan.split_tokens <= 1024 and plan.split_tokens % 16 == 0
    # more (kv head, head chunk) units than one workgroup's 8 waves: the split grid
    plan = _plan(lib, 4, 4, 64, 8, 128, 16, 1, 4096, 2, 2)
    assert plan.decode_mode == 2
    assert plan.decode_workgroups == -(-4096 // plan.split_tokens)


@pytest.mark.parametrize("fn,args,message", [
    ("mvllm_rmsnorm", (1, 1, 1, 4, 8, 1e-6, 7, None), "float64 is not supported"),
    ("mvllm_rope", (1, 1, 1, 8, 1, 1, 4, 2, 7, 2, 16, 0, None), "must be even"),
    ("mvllm_rope", (1, 1, 1, 8, 1, 1, 6, 2, 8, 2, 16, 0, None), "cannot broadcast"),
    ("mvllm_rope", (1, 1, 1, 2, 1, 1, 4, 2, 8, 2, 16, 0, None), "int32 or int64"),
    ("mvllm_swiglu", (1, 1, 1, 8, 9, None), "float64 is not supported"),
    ("mvllm_swiglu_interleaved", (16, 16, 4, 40, 2, None), "multiple of 16"),
    ("mvllm_add_rmsnorm", (16, 16, 16, 16, 16, 4, 100, 1e-6, 2, None), "is not served"),
    # a q token stride shorter than the token's heads (16 x 128)
    ("mvllm_qk_norm_rope_kv_write", (16,) * 9 + (4, 16, 16, 16, 64, 4, 16, 8, 128, 4, 64, 1e-6,
                                     100, 0, 2, None), "token strides"),
    # a k/v token stride that breaks 16-byte alignment (bf16: a multiple of 8 elements)
    ("mvllm_qk_norm_rope_kv_write", (16,) * 9 + (4, 16, 16, 16, 64, 4, 16, 8, 128, 4, 64, 1e-6,
                                     0, 1028, 2, None), "16-byte aligned"),
])
def test_elementwise_refusals(lib, fn, args, message):
    assert getattr(lib, fn)(*args) != 0
    assert message in lib.mvllm_last_error().decode()


def test_empty_inputs_are_no_ops(lib):
    assert lib.mvllm_rmsnorm(None, None, None, 0, 128, 1e-6, 2, None) == 0
    assert lib.mvllm_swiglu(None, None, None, 0, 2, None) == 0
    assert _paged(lib, num_tokens=0, num_seqs=0, out=None) == 0


def test_load_extension_refuses_without_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(extension.ToolchainError, match="no GPU"):
        extension.load_extension()


def test_read_probe_refusals(lib):
    """The bandwidth probe checks its sizes before any launch."""
    assert lib.mvllm_read_probe(None, 1 << 20, None, 4, 32768, 8, 256, 2048, None) == 1
    assert lib.mvllm_read_probe(256, 1 << 20, None, 4, 3000, 8, 256, 2048, None) == 2
    assert "page_bytes" in lib.mvllm_last_error().decode()
    assert lib.mvllm_read_probe(256, 1 << 16, None, 4, 32768, 8, 256, 2048, None) == 1
    assert "fewer pages" in lib.mvllm_last_error().decode()
    assert lib.mvllm_read_probe(256, 1 << 20, None, 4, 32768, 8, 256, 100, None) == 1
    assert "sink" in lib.mvllm_last_error().decode()
