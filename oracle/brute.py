"""ctypes loader for the float64 brute-force oracle in brute.c (test infrastructure only)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle_brute.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        p = ctypes.c_void_p
        i32 = ctypes.c_int32
        lib.oracle_paged_attention_f64.restype = ctypes.c_int
        lib.oracle_paged_attention_f64.argtypes = [p] * 6 + [i32] * 6 + [ctypes.c_double, p]
        _lib = lib
    return _lib


def _f32(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().to(torch.float32).numpy())


def _i32(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().to(torch.int32).numpy())


def paged_attention_f64(q, key_pool, value_pool, block_tables, cu_seqlens_q, context_lens,
                        scale: float, k_scale=None, v_scale=None) -> np.ndarray:
    """float64 ``T x H_q x D`` reference output. fp8 pools are dequantised in float64."""
    if key_pool.dtype == torch.float8_e4m3fn:
        kp = key_pool.cpu().to(torch.float64) * k_scale.cpu().to(torch.float64)[:, None, :, None]
        vp = value_pool.cpu().to(torch.float64) * v_scale.cpu().to(torch.float64)[:, None, :, None]
        # The C code reads fp32; a float64 -> float32 rounding of value*scale is within
        # 2^-24 relative, far below every tolerance this oracle is used at.
        key_pool, value_pool = kp.to(torch.float32), vp.to(torch.float32)
    qa, ka, va = _f32(q), _f32(key_pool), _f32(value_pool)
    bt, cu, ctx = _i32(block_tables), _i32(cu_seqlens_q), _i32(context_lens)
    out = np.zeros(qa.shape, dtype=np.float64)
    _, num_q_heads, head_dim = qa.shape
    _, block_size, num_kv_heads, _ = ka.shape
    rc = _load().oracle_paged_attention_f64(
        qa.ctypes.data, ka.ctypes.data, va.ctypes.data, bt.ctypes.data, cu.ctypes.data,
        ctx.ctypes.data, len(ctx), num_q_heads, num_kv_heads, head_dim, block_size,
        bt.shape[1], float(scale), out.ctypes.data,
    )
    if rc == -1:
        raise ValueError("a sequence computes more tokens than it attends over")
    if rc == -2:
        raise ValueError("a key position falls on a padded (-1) table entry")
    if rc != 0:
        raise RuntimeError(f"brute-force oracle failed with {rc}")
    return out
