"""numpy restatements of the elementwise ops, with the reference's rounding points.

Test infrastructure only. Each function takes and returns float32 numpy arrays that
hold values of the storage dtype (``dtype`` in {"f32", "f16", "bf16"}), and rounds
exactly where the reference's PyTorch expression rounds:

  rms_norm    weight * T(x * rsqrt(mean(x^2) + eps))          layer_norm.py:40-46
  apply_rope  T(x*cos[pos] + rotate_half(x)*sin[pos]), fp32   positional_encoding.py:36-62
  rope_tables fp32 cos/sin of pos * theta^(-2i/D), halves duplicated
                                                              positional_encoding.py:97-110
  swiglu      T(T(g * T(sigmoid(g))) * u)                     basics.py:39-41, ops.py:163

Rounding helpers are written from the IEEE definitions (round to nearest, ties to
even), independent of torch. Pinned in tests/test_oracle.py against torch's own casts
and by closed forms (unit-weight RMS is 1, position 0 is the identity, rotation
preserves pair norms, silu(0) = 0).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "apply_rope",
    "fp8_e4m3_decode",
    "fp8_e4m3_encode",
    "rms_norm",
    "round_bf16",
    "round_to",
    "rope_tables",
    "swiglu",
]


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    raise ValueError(dtype)


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6, dtype: str = "f32") -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    mean_square = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(mean_square + eps)).astype(np.float32)
    normalized = round_to(x * inv, dtype)
    return round_to(normalized * np.asarray(weight, dtype=np.float32), dtype)


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 1_000_000.0):
    exponents = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv_freq = (np.float32(1.0) / (np.float32(theta) ** exponents)).astype(np.float32)
    angles = np.outer(np.arange(max_seq_len, dtype=np.float32), inv_freq).astype(np.float32)
    angles = np.concatenate([angles, angles], axis=-1)
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def apply_rope(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray,
               dtype: str = "f32") -> np.ndarray:
    """x: ``N.. x H x D``; positions broadcast over the token axes (``t % len``)."""
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    half = d // 2
    flat = x.reshape(-1, x.shape[-2], d)
    pos = np.asarray(positions).reshape(-1).astype(np.int64)
    tok = np.arange(flat.shape[0]) % pos.shape[0]
    c = cos[pos[tok]][:, None, :]
    s = sin[pos[tok]][:, None, :]
    rotated = np.concatenate([-flat[..., half:], flat[..., :half]], axis=-1)
    out = (flat * c).astype(np.float32) + (rotated * s).astype(np.float32)
    return round_to(out.astype(np.float32), dtype).reshape(x.shape)


def swiglu(gate: np.ndarray, up: np.ndarray, dtype: str = "f32") -> np.ndarray:
    g = np.asarray(gate, dtype=np.float32)
    sig = round_to((np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32), dtype)
    act = round_to((g * sig).astype(np.float32), dtype)
    return round_to((act * np.asarray(up, dtype=np.float32)).astype(np.float32), dtype)


# OCP float8 e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no infinities,
# 0x7f / 0xff are NaN, largest finite 448.
def fp8_e4m3_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    exp = (c >> 3) & 0xF
    man = c & 0x7
    value = np.where(exp == 0, man / 8.0 * 2.0**-6, (1.0 + man / 8.0) * 2.0 ** (exp - 7))
    value = np.where((c & 0x7F) == 0x7F, np.nan, value)
    return (sign * value).astype(np.float32)


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even encode with saturation to +-448 (finite inputs); the sign
    bit is kept, so -0.0 encodes as 0x80 (as torch's cast and the GPU conversion do)."""
    table = fp8_e4m3_decode(np.arange(256, dtype=np.uint8))
    finite = np.array([i for i in range(128) if not np.isnan(table[i])])  # positive codes
    mags = table[finite].astype(np.float64)
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), 448.0)
    idx = np.searchsorted(mags, a)
    idx = np.clip(idx, 1, len(mags) - 1)
    lo, hi = mags[idx - 1], mags[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & (finite[idx] % 2 == 0))
    code = np.where(pick_hi, finite[idx], finite[idx - 1])
    code = np.where(a == mags[idx - 1], finite[idx - 1], code)
    return (code | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)
