"""Bit-level numeric helpers for the oracle (test infrastructure only).

FP8 here is OCP ``float8_e4m3fn`` (bias 7, no infinities, 0x7F/0xFF = NaN,
max finite 448).  The reference stores K/V into FP8 arenas through Triton's
implicit store cast (compact_kv.py:243-252, compact_attention.py:186-209),
which rounds to nearest-even and saturates to +-448, and through torch's
``.to(torch.float8_e4m3fn)`` (compact_kv.py:1085-1087), which rounds to
nearest-even but maps |x| > 464 to NaN.  The two agree on |x| <= 464; the
oracle fixes the saturating form (clamp to +-448, then RNE), the one both
agree with on every finite value a model produces below 464.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = 448.0

# dtype codes shared with the C-ABI (include/fastdms_amd.h)
DT_F32, DT_F16, DT_BF16, DT_FP8 = 0, 1, 2, 3


def e4m3fn_encode(x) -> np.ndarray:
    """float32 values -> uint8 e4m3fn bits, clamp to +-448 then RNE.

    Pinned against torch's CPU cast on every |x| <= 448 in
    tests/test_oracle_numerics.py (a library routine).
    """
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    nan = np.isnan(x)
    sign = np.signbit(x)
    a = np.minimum(np.abs(np.where(nan, 0.0, x)), FP8_MAX)
    _, e = np.frexp(a)
    exp = np.where(a > 0, e - 1, -6)
    exp = np.maximum(exp, -6)
    step = np.ldexp(1.0, exp - 3)
    q = np.rint(a / step)  # numpy rint is round-half-to-even
    bits = ((exp + 6) * 8 + q).astype(np.int64)
    bits = np.where(nan, 0x7F, bits)
    bits = bits | np.where(sign, 0x80, 0)
    return bits.astype(np.uint8)


def e4m3fn_decode(bits) -> np.ndarray:
    """uint8 e4m3fn bits -> float32 values (exact)."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    exp = (b >> 3) & 0xF
    man = b & 0x7
    val = np.where(exp == 0, man * 2.0 ** -9, (8 + man) * np.ldexp(1.0, exp - 10))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (sign * val).astype(np.float32)


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest-even bfloat16 value, returned as float32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    bias = 0x7FFF + ((u >> 16) & 1)
    r = ((u + bias) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def bf16_bits(x) -> np.ndarray:
    """float32 (already bf16-representable) -> uint16 bits."""
    x = np.ascontiguousarray(bf16_round(x))
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def cast(x, dtype_code: int) -> np.ndarray:
    """Round float32 values to ``dtype_code`` and return them as float32 values."""
    x = np.asarray(x, dtype=np.float32)
    if dtype_code == DT_F32:
        return x.copy()
    if dtype_code == DT_F16:
        return x.astype(np.float16).astype(np.float32)
    if dtype_code == DT_BF16:
        return bf16_round(x)
    if dtype_code == DT_FP8:
        return e4m3fn_decode(e4m3fn_encode(x))
    raise ValueError(f"unknown dtype code {dtype_code}")


def to_storage(x, dtype_code: int) -> np.ndarray:
    """Round float32 values to ``dtype_code`` and return the storage array
    (float32 / float16 / uint16 bf16 bits / uint8 e4m3 bits)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype_code == DT_F32:
        return x.copy()
    if dtype_code == DT_F16:
        return x.astype(np.float16)
    if dtype_code == DT_BF16:
        return bf16_bits(x)
    if dtype_code == DT_FP8:
        return e4m3fn_encode(x)
    raise ValueError(f"unknown dtype code {dtype_code}")


def from_storage(s, dtype_code: int) -> np.ndarray:
    if dtype_code == DT_F32:
        return np.asarray(s, dtype=np.float32)
    if dtype_code == DT_F16:
        return np.asarray(s, dtype=np.float16).astype(np.float32)
    if dtype_code == DT_BF16:
        return bf16_from_bits(s)
    if dtype_code == DT_FP8:
        return e4m3fn_decode(s)
    raise ValueError(f"unknown dtype code {dtype_code}")


def storage_dtype(dtype_code: int):
    return {DT_F32: np.float32, DT_F16: np.float16, DT_BF16: np.uint16, DT_FP8: np.uint8}[dtype_code]
