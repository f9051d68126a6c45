"""FP8 / INT4 linear-layer oracle (test infrastructure only).

Restates fastdms/layers/linear.py (weight quantisation and the row-1 / small-M
FP8 paths) and embed_head.py (FP8 LM-head GEMV fused with argmax).  FP8 is
OCP e4m3fn (numerics.e4m3fn_encode).  Products of two FP8 values are exact in
float32; the oracle accumulates in float64, so kernel-vs-oracle differences
are accumulation-order only and are compared with the reference tests'
tolerances (test_compact_kv.py:505, 529, 582, 620).
"""
from __future__ import annotations

import numpy as np

from . import numerics

FP8_MAX = np.float32(448.0)


def amax_to_scale(amax, torch_form: bool = True) -> np.ndarray:
    """448/amax in fp32, 1 where amax == 0.

    torch_form: the reference's tensor expression ``_FP8_MAX / amax``
    (linear.py:386-388) evaluates as torch's ``__rtruediv__``, i.e.
    reciprocal(amax) * 448 with two fp32 roundings.  The Triton kernels
    (linear.py:514-523, 683-694) divide in fp32 directly (torch_form=False).
    """
    a = np.asarray(amax, dtype=np.float32)
    safe = np.where(a > 0, a, np.float32(1.0)).astype(np.float32)
    if torch_form:
        q = ((np.float32(1.0) / safe).astype(np.float32) * FP8_MAX).astype(np.float32)
    else:
        q = (FP8_MAX / safe).astype(np.float32)
    return np.where(a > 0, q, np.float32(1.0)).astype(np.float32)


def quantize_weight_to_fp8(weight):
    """linear.py:813-823: per output channel scale (torch form); W8^T [K, N]
    e4m3 bits and scale_inv [1, N] = reciprocal(scale) in fp32."""
    w = np.asarray(weight, dtype=np.float32)             # [N, K]
    scale = amax_to_scale(np.abs(w).max(axis=1))         # [N]
    w8_t = numerics.e4m3fn_encode((w.T * scale[None, :]).astype(np.float32))  # [K, N]
    scale_inv = (np.float32(1.0) / scale).astype(np.float32).reshape(1, -1)
    return w8_t, scale_inv


def quantize_rows_fp8(x, torch_form: bool = False):
    """Per-row dynamic activation quantisation: x_scale = 448/amax(row), xq =
    e4m3(x * x_scale).  torch_form=False: the row-1 / small-M Triton kernels
    (linear.py:514-523, 683-694); True: _fp8_linear (652-654).  Returns (xq bits, x_scale)."""
    x = np.asarray(x, dtype=np.float32)
    x_scale = amax_to_scale(np.abs(x).max(axis=-1), torch_form=torch_form)
    xq = numerics.e4m3fn_encode((x * x_scale[..., None]).astype(np.float32))
    return xq, x_scale


def fp8_linear(x, w8_t, scale_inv, quantize_x: bool = True, torch_form: bool = False, w_decoded=None):
    """y[m, n] = sum_k xq[m,k] w8[k,n] * (1/x_scale[m]) * scale_inv[n].

    Covers the row-1 (linear.py:492-578), small-M (665-719) and _scaled_mm
    (635-662, torch_form=True) paths, which share this closed form; with
    quantize_x=False the activation is used unquantised (linear.py:509-527
    QUANTIZE_X=False).  Returns float64 [M, N].  w_decoded: the float64
    decode of w8_t, when the caller keeps it across calls.
    """
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    w = numerics.e4m3fn_decode(w8_t).astype(np.float64) if w_decoded is None else w_decoded
    if quantize_x:
        xq, xs = quantize_rows_fp8(x, torch_form=torch_form)
        xv = numerics.e4m3fn_decode(xq).astype(np.float64)
        inv = (np.float32(1.0) / xs).astype(np.float64)
    else:
        xv = x.astype(np.float64)
        inv = np.ones(x.shape[0])
    return (xv @ w) * inv[:, None] * np.asarray(scale_inv, np.float64).reshape(1, -1)


def fp8_row1_argmax(x, w8_t, scale_inv) -> int:
    """embed_head.py:96-211: FP8 GEMV scores, argmax with ties to the lowest
    index (block_idx = min index attaining the max, embed_head.py:142, 160)."""
    s = fp8_linear(np.asarray(x, np.float32).reshape(1, -1), w8_t, scale_inv, quantize_x=True)[0]
    return int(np.flatnonzero(s == s.max())[0])


def fp8_rerank_topk(x, candidates, w8_t, scale_inv) -> int:
    """embed_head.py:214-262: FP8 scores (row-1 activation quantisation) of
    the candidate ids only; the best one, the lowest id on ties; ids outside
    [0, N) score -inf."""
    n = np.asarray(w8_t).shape[1]
    cand = np.asarray(candidates, np.int64).reshape(-1)
    ok = (cand >= 0) & (cand < n)
    s = np.full(cand.shape, -np.inf)
    if ok.any():
        sinv = np.asarray(scale_inv, np.float32).reshape(-1)
        sc = fp8_linear(np.asarray(x, np.float32).reshape(1, -1), np.asarray(w8_t)[:, cand[ok]], sinv[cand[ok]])[0]
        s[ok] = sc
    best = s.max()
    return int(cand[s == best].min())


def argmax_lowest(scores) -> np.ndarray:
    """Row-wise argmax, lowest index on ties."""
    s = np.asarray(scores)
    return np.array([int(np.flatnonzero(r == r.max())[0]) for r in s.reshape(-1, s.shape[-1])])


def _div_scalar(a, d: float, device_form: bool) -> np.ndarray:
    """fp32 ``tensor / python_float``.  On the GPU torch evaluates it as
    a * fp32(1/d) (its CUDA true-divide kernel multiplies by the reciprocal of
    a CPU scalar); on the CPU it divides.  The reference quantises on the GPU."""
    a = np.asarray(a, np.float32)
    if device_form:
        return (a * (np.float32(1.0) / np.float32(d))).astype(np.float32)
    return (a / np.float32(d)).astype(np.float32)


def quantize_weight_int4(weight, group_size: int, mode: str = "symmetric", device_form: bool = True):
    """linear.py:414-459 quantisation math (the packing is this build's own).

    Returns q [N, K] uint8 in 0..15, scale [N, K/gs] and zero [N, K/gs], both
    rounded to bf16 (the reference stores scale_zeros in bf16, linear.py:456-458);
    the codes use the fp32 scale / zero before that rounding.
    Dequant: (q - 8) * scale + zero.  device_form: amax / 7.0 and span / 15.0
    as torch computes them on the GPU (see _div_scalar).
    """
    w = np.asarray(weight, dtype=np.float32)
    n, k = w.shape
    g = w.reshape(n, k // group_size, group_size)
    mode = mode.strip().lower()
    if mode in {"sym", "symmetric"}:
        amax = np.abs(g).max(axis=2)
        scale = np.where(amax > 0, _div_scalar(amax, 7.0, device_form), np.float32(1.0))
        zero = np.zeros_like(scale)
        qs = np.clip(np.rint(g / scale[..., None]), -8, 7)
        q = (qs + 8).astype(np.uint8)
    elif mode in {"asym", "asymmetric", "affine"}:
        wmin, wmax = g.min(axis=2), g.max(axis=2)
        span = (wmax - wmin).astype(np.float32)
        nz = span > 0
        scale = np.where(nz, _div_scalar(span, 15.0, device_form), np.float32(1.0)).astype(np.float32)
        zero = np.where(nz, (wmin + np.float32(8.0) * scale).astype(np.float32), wmin).astype(np.float32)
        q = np.clip(np.rint((g - zero[..., None]) / scale[..., None] + 8.0), 0, 15).astype(np.uint8)
    else:
        raise ValueError("int4 quant_mode must be symmetric or asymmetric")
    return q.reshape(n, k), numerics.bf16_round(scale), numerics.bf16_round(zero)


def int4_dequant(q, scale, zero, group_size: int) -> np.ndarray:
    q = np.asarray(q, np.float64)
    n, k = q.shape
    s = np.repeat(np.asarray(scale, np.float64), group_size, axis=1)
    z = np.repeat(np.asarray(zero, np.float64), group_size, axis=1)
    return (q - 8.0) * s + z


def int4_linear(x, q, scale, zero, group_size: int) -> np.ndarray:
    """W4A16: y = x @ dequant(W)^T (linear.py:462-478 semantics), float64."""
    return np.atleast_2d(np.asarray(x, np.float64)) @ int4_dequant(q, scale, zero, group_size).T
