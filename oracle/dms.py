"""DMS decision oracle (test infrastructure only).

Restates fastdms/engine/dms.py of the reference.
"""
from __future__ import annotations

import numpy as np


def dms_threshold(alpha_scale: float, alpha_offset: float) -> np.float32:
    """Threshold for the positive-scale branch.

    dms.py:37-38 / 224-225: ``evict = v > alpha_offset / alpha_scale`` with the
    Python-float quotient compared against an fp32 value, which torch and Triton
    both perform in fp32 (the scalar is rounded to fp32 first).  Pinned by the
    reference test's nextafter(0.05) edge cases (test_compact_kv.py:441-483).
    """
    return np.float32(float(alpha_offset) / float(alpha_scale))


def dms_decide(values, alpha_scale: float, alpha_offset: float) -> np.ndarray:
    """evict flag from fp32 decision values (dms.py:37-40, 224-227)."""
    v = np.asarray(values, dtype=np.float32)
    if alpha_scale > 0:
        return v > dms_threshold(alpha_scale, alpha_offset)
    prod = (v * np.float32(alpha_scale)).astype(np.float32)
    return (prod - np.float32(alpha_offset)).astype(np.float32) > np.float32(0.0)


def extract_dms_eviction_decisions(q, *, num_kv_heads: int, num_qo_heads: int, head_dim: int,
                                   alpha_scale: float, alpha_offset: float):
    """dms.py:152-232.

    ``q`` is float32 values shaped [T, Hq, D] or [T, Hq*D].  Returns
    ``(q_clean, evict)``: q with channel D-1 of head ``h*G`` zeroed for every
    kv head h, and evict [T, Hkv] bool.
    """
    if num_qo_heads % num_kv_heads != 0:
        raise ValueError("num_qo_heads must be divisible by num_kv_heads")
    q = np.array(q, dtype=np.float32, copy=True)
    shape = q.shape
    qv = q.reshape(shape[0], num_qo_heads, head_dim)
    g = num_qo_heads // num_kv_heads
    vals = qv[:, 0::g, head_dim - 1].copy()
    evict = dms_decide(vals, alpha_scale, alpha_offset)
    qv[:, 0::g, head_dim - 1] = 0.0
    return qv.reshape(shape), evict


def build_dms_live_mask(evict_mask, *, current_position: int, window_size: int, positions=None):
    """dms.py:235-262: live = ~evict | (current - pos <= window)."""
    evict_mask = np.asarray(evict_mask, dtype=bool)
    if evict_mask.ndim not in (2, 3):
        raise ValueError("expected evict_mask rank 2 or 3")
    if window_size < 0:
        raise ValueError("window_size must be non-negative")
    tokens = evict_mask.shape[-1]
    pos = np.arange(tokens, dtype=np.int64) if positions is None else np.asarray(positions, dtype=np.int64)
    inside = (int(current_position) - pos) <= int(window_size)
    return (~evict_mask) | inside.reshape((1,) * (evict_mask.ndim - 1) + (tokens,))
