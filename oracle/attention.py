"""Attention-side oracle (test infrastructure only).

Restates the reference's RoPE (fastdms/layers/rotary_embedding.py), the fused
decode DMS + RoPE + compact append (compact_attention.py:67-209), compact
decode attention (compact_attention.py:1339-1364, the reference's own torch
reference) and the dense causal prefill attention that flash-attn computes
for the reference (attention.py:85-92).

Float work uses numpy float32 with one rounding per operation (no fused
multiply-add), or float64 where the reference is compared by tolerance.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import numerics
from .dms import dms_decide


def rope_inv_freq(head_dim: int, base: float, rope_scaling: dict | None = None) -> np.ndarray:
    """rotary_embedding.py:52-67 (default, linear and llama3 scaling), fp32."""
    import torch  # the reference builds the table with torch fp32 ops
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    if rope_scaling is not None:
        rt = rope_scaling.get("rope_type") or rope_scaling.get("type")
        if rt == "llama3":
            factor = float(rope_scaling["factor"])
            lo = float(rope_scaling.get("low_freq_factor", 1.0))
            hi = float(rope_scaling.get("high_freq_factor", 4.0))
            omax = int(rope_scaling["original_max_position_embeddings"])
            lo_wl, hi_wl = omax / lo, omax / hi
            wl = 2 * math.pi / inv
            inv_low = inv / factor
            smooth = (omax / wl - lo) / (hi - lo)
            smooth_f = (1.0 - smooth) * inv_low + smooth * inv
            out = torch.where(wl < hi_wl, inv, smooth_f)
            inv = torch.where(wl > lo_wl, inv_low, out)
        elif rt == "linear":
            inv = inv / float(rope_scaling.get("factor", 1.0))
        elif rt not in (None, "default"):
            raise NotImplementedError(rt)
    return inv.numpy()


def rope_cos_sin_cache(head_dim: int, max_position: int, base: float, rope_scaling=None) -> np.ndarray:
    """rotary_embedding.py:68-73: cat(cos, sin) fp32 shaped [max_pos, 1, D]."""
    import torch
    inv = torch.from_numpy(rope_inv_freq(head_dim, base, rope_scaling))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze(1).numpy()


def rotate(x1, x2, cos, sin):
    """(x1*cos - x2*sin, x2*cos + x1*sin), each product and sum rounded to fp32
    (rotary_embedding.py:12-14; compact_attention.py:149-150, 179-180)."""
    f = np.float32
    x1 = np.asarray(x1, f)
    x2 = np.asarray(x2, f)
    y1 = (x1 * cos).astype(f) - (x2 * sin).astype(f)
    y2 = (x2 * cos).astype(f) + (x1 * sin).astype(f)
    return y1.astype(f), y2.astype(f)


def apply_rotary_emb(x, cos, sin, out_dtype_code: int):
    """rotary_embedding.py:7-15, result cast back to the input dtype."""
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    y1, y2 = rotate(x[..., :half], x[..., half:], cos, sin)
    return numerics.cast(np.concatenate([y1, y2], axis=-1), out_dtype_code)


def fused_dms_rope_store_compact_decode(*, q, k, v, cos_sin_cache, compact_k, compact_v, slot_mapping,
                                        positions, num_kv_heads, alpha_scale, alpha_offset, q_dtype_code,
                                        k_dtype_code, compact_dtype_code, store_q=True, store_transient_k=True,
                                        k_scale=None, v_scale=None):
    """compact_attention.py:67-209, in place on numpy arrays; returns evict [B, Hkv].

    q [B, Hq, D], k/v [B, Hkv, D] float32 values; compact_* storage arrays;
    the decision lane (g=0, d=D-1) is zeroed before q's RoPE; RoPE(k) is
    stored into the arena straight from fp32; v is stored from its own dtype.
    """
    q = np.asarray(q)
    b, hq, d = q.shape
    g = hq // num_kv_heads
    half = d // 2
    evict = np.zeros((b, num_kv_heads), dtype=bool)
    for bi in range(b):
        cs = cos_sin_cache[int(positions[bi]), 0]
        cos, sin = cs[:half].astype(np.float32), cs[half:].astype(np.float32)
        for h in range(num_kv_heads):
            evict[bi, h] = dms_decide(np.float32(q[bi, h * g, d - 1]), alpha_scale, alpha_offset)
            if store_q:
                for gi in range(g):
                    qh = q[bi, h * g + gi].astype(np.float32)
                    q2 = qh[half:].copy()
                    if gi == 0:
                        q2[half - 1] = 0.0
                    y1, y2 = rotate(qh[:half], q2, cos, sin)
                    q[bi, h * g + gi] = numerics.cast(np.concatenate([y1, y2]), q_dtype_code)
            kh = np.asarray(k[bi, h], dtype=np.float32)
            y1, y2 = rotate(kh[:half], kh[half:], cos, sin)
            krot = np.concatenate([y1, y2])
            if store_transient_k:
                k[bi, h] = numerics.cast(krot, k_dtype_code)
            slot = int(slot_mapping[bi, h])
            if slot >= 0:
                vrow = np.asarray(v[bi, h], np.float32)
                if k_scale is not None:  # per-kv-head FP8 scale: stored = x * fp32(1 / scale)
                    krot = (krot * (np.float32(1.0) / np.float32(k_scale[h]))).astype(np.float32)
                if v_scale is not None:
                    vrow = (vrow * (np.float32(1.0) / np.float32(v_scale[h]))).astype(np.float32)
                compact_k[slot] = numerics.to_storage(krot, compact_dtype_code)
                compact_v[slot] = numerics.to_storage(vrow, compact_dtype_code)
    return evict


def store_compact_kvcache(key, value, compact_k, compact_v, slot_mapping, compact_dtype_code):
    """compact_attention.py:212-246 / 968-1007: compact[slot] = k/v if slot >= 0."""
    b, h, _ = np.asarray(key).shape
    for bi in range(b):
        for hi in range(h):
            s = int(slot_mapping[bi, hi])
            if s >= 0:
                compact_k[s] = numerics.to_storage(np.asarray(key[bi, hi], np.float32), compact_dtype_code)
                compact_v[s] = numerics.to_storage(np.asarray(value[bi, hi], np.float32), compact_dtype_code)


def _attend(q, keys, values, scale):
    s = keys @ q * scale
    m = s.max()
    p = np.exp(s - m)
    return (p @ values) / p.sum()


def compact_decode_attention(q, compact_k, compact_v, base_offsets, live_counts, scale=None, k_scale=None,
                             v_scale=None):
    """compact_attention.py:1339-1364 in float64.

    q [B, Hq, D] float values; compact_* float values [slots, D];
    base_offsets/live_counts [B, Hkv].  Returns float64 [B, Hq, D].
    k_scale / v_scale [Hkv]: per-kv-head dequant of stored FP8 values
    (K = stored * k_scale; no reference counterpart).
    """
    q = np.asarray(q, dtype=np.float64)
    b, hq, d = q.shape
    hkv = np.asarray(base_offsets).shape[1]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    ck = np.asarray(compact_k, dtype=np.float64)
    cv = np.asarray(compact_v, dtype=np.float64)
    out = np.zeros((b, hq, d), dtype=np.float64)
    ksc = np.ones(hkv) if k_scale is None else np.asarray(k_scale, np.float64)
    vsc = np.ones(hkv) if v_scale is None else np.asarray(v_scale, np.float64)
    for bi in range(b):
        for qh in range(hq):
            h = qh // g
            base, live = int(base_offsets[bi, h]), int(live_counts[bi, h])
            out[bi, qh] = _attend(q[bi, qh], ck[base:base + live] * ksc[h], cv[base:base + live] * vsc[h], scale)
    return out


def compact_decode_attention_storage(q, ck_storage, cv_storage, dtype_code, base_offsets, live_counts, scale=None,
                                     k_scale=None, v_scale=None):
    """compact_decode_attention over arena *storage* arrays, decoding only the
    live span of each (b, kv head)."""
    q = np.asarray(q, dtype=np.float64)
    b, hq, d = q.shape
    hkv = np.asarray(base_offsets).shape[1]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    out = np.zeros((b, hq, d), dtype=np.float64)
    for bi in range(b):
        for h in range(hkv):
            base, live = int(base_offsets[bi, h]), int(live_counts[bi, h])
            keys = numerics.from_storage(ck_storage[base:base + live], dtype_code).astype(np.float64)
            vals = numerics.from_storage(cv_storage[base:base + live], dtype_code).astype(np.float64)
            if k_scale is not None:
                keys = keys * float(k_scale[h])
            if v_scale is not None:
                vals = vals * float(v_scale[h])
            s = q[bi, h * g:(h + 1) * g] @ keys.T * scale
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[bi, h * g:(h + 1) * g] = (p @ vals) / p.sum(axis=1, keepdims=True)
    return out


def paged_rows(block_table_row, live: int, page_size: int) -> np.ndarray:
    """Physical slot of every rank r < live: table[r // P] * P + r % P."""
    r = np.arange(live)
    return np.asarray(block_table_row, dtype=np.int64)[r // page_size] * page_size + r % page_size


def compact_decode_attention_paged(q, kv_k, kv_v, block_tables, live_counts, page_size, scale=None, k_scale=None,
                                   v_scale=None):
    """Same math as compact_decode_attention, K/V addressed through a
    block table [B, Hkv, max_pages] of page_size-token pages."""
    q = np.asarray(q, dtype=np.float64)
    b, hq, d = q.shape
    hkv = np.asarray(live_counts).shape[1]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    ck = np.asarray(kv_k, dtype=np.float64)
    cv = np.asarray(kv_v, dtype=np.float64)
    out = np.zeros((b, hq, d), dtype=np.float64)
    for bi in range(b):
        for qh in range(hq):
            h = qh // g
            rows = paged_rows(block_tables[bi, h], int(live_counts[bi, h]), page_size)
            ks = 1.0 if k_scale is None else float(k_scale[h])
            vs = 1.0 if v_scale is None else float(v_scale[h])
            out[bi, qh] = _attend(q[bi, qh], ck[rows] * ks, cv[rows] * vs, scale)
    return out


def causal_prefill_attention(q, k, v, cu_seqlens, scale=None, cu_seqlens_k=None):
    """Dense causal softmax attention per sequence (attention.py:85-92;
    flash_attn_varlen_func semantics with causal=True).

    q [T, Hq, D], k/v [Tk, Hkv, D] float values; returns float64 [T, Hq, D].
    With cu_seqlens_k the sequence's queries are the last of its keys
    (flash-attn's bottom-right alignment: query i of n sees keys 0 ..
    klen - n + i); without it q_len == k_len and cu_seqlens_k = cu_seqlens.
    Evaluated in float64 with torch CPU matmuls (multi-threaded), 512 query
    rows of one KV head's query group at a time.
    """
    q = torch.from_numpy(np.ascontiguousarray(q, np.float64))
    k = torch.from_numpy(np.ascontiguousarray(k, np.float64))
    v = torch.from_numpy(np.ascontiguousarray(v, np.float64))
    hq, d = q.shape[1], q.shape[2]
    hkv = k.shape[1]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    out = torch.zeros_like(q)
    cq = [int(x) for x in cu_seqlens]
    ck = cq if cu_seqlens_k is None else [int(x) for x in cu_seqlens_k]
    for i in range(len(cq) - 1):
        s0, s1, k0, k1 = cq[i], cq[i + 1], ck[i], ck[i + 1]
        n, nk = s1 - s0, k1 - k0
        if nk < n:
            raise ValueError("a sequence has fewer keys than queries")
        for r0 in range(0, n, 512):
            r1 = min(n, r0 + 512)
            # query row r sees keys 0 .. nk - n + r
            qi = torch.arange(r0, r1).unsqueeze(1) + (nk - n)
            mask = torch.arange(nk).unsqueeze(0) <= qi
            for h in range(hkv):
                qs = q[s0 + r0:s0 + r1, h * g:(h + 1) * g].transpose(0, 1)  # [g, rows, d]
                sc = (qs @ k[k0:k1, h].T) * scale
                sc = sc.masked_fill(~mask, -float("inf"))
                sc = sc - sc.amax(dim=-1, keepdim=True)
                p = torch.exp(sc)
                o = (p @ v[k0:k1, h]) / p.sum(dim=-1, keepdim=True)
                out[s0 + r0:s0 + r1, h * g:(h + 1) * g] = o.transpose(0, 1)
    return out.numpy()
