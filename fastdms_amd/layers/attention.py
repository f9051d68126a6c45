"""Attention dispatch (mirror of fastdms/layers/attention.py:50-151).

Prefill: dense causal attention over the whole prompt (HIP MFMA kernel
``fdms_prefill_attention``; the reference uses flash_attn_varlen_func).
Decode with compact KV: per-layer slice of the [layers, batch, kv_heads]
metadata, optional unfused append, then ``compact_decode_attention``.
The dense paged decode path of the reference is not part of this build.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as nat
from ..utils.context import get_context
from .compact_attention import (compact_decode_attention, compact_decode_attention_paged,
                                fused_decode_attention_planned,
                                fused_dms_rope_store_compact_decode_attention, store_compact_kvcache)

PAGE_SIZE = 16  # rows per page of the paged compact layout (engine.paged_kv)


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                      max_seqlen: int, scale: float, out: torch.Tensor | None = None,
                      cu_seqlens_k: torch.Tensor | None = None) -> torch.Tensor:
    """Causal varlen attention: q [T, Hq, D], k/v [Tk, Hkv, D] bf16 -> [T, Hq, D].
    With ``cu_seqlens_k`` a sequence's queries are the last of its keys
    (bottom-right causal alignment, flash_attn_varlen_func's): a prompt chunk
    attending to the retained earlier chunks and itself."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("prefill attention expects bf16 q/k/v")
    t, hq, d = q.shape
    hkv = k.shape[1]
    if d not in (64, 128):
        raise ValueError(f"prefill attention supports head_dim 64 or 128, got {d}")
    for x in (q, k, v):
        if x.stride(2) != 1 or (x.stride(0) * 2) % 16 or (x.stride(1) * 2) % 16 or x.data_ptr() % 16:
            raise ValueError("prefill attention needs 16-byte aligned rows with a contiguous head_dim")
    if out is None:
        out = torch.empty((t, hq, d), device=q.device, dtype=q.dtype)
    cu = cu_seqlens.to(torch.int32)
    if cu_seqlens_k is None:
        nat.call("fdms_prefill_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
                 k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                 cu.data_ptr(), cu.numel() - 1, int(max_seqlen), hq, hkv, d, float(scale), nat.stream())
        return out
    cuk = cu_seqlens_k.to(torch.int32)
    if cuk.numel() != cu.numel():
        raise ValueError("cu_seqlens and cu_seqlens_k must describe the same sequences")
    nat.call("fdms_prefill_attention_varlen", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
             k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
             cu.data_ptr(), cuk.data_ptr(), cu.numel() - 1, int(max_seqlen), hq, hkv, d, float(scale), nat.stream())
    return out


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.compact_k_cache = self.compact_v_cache = torch.tensor([])
        # per-kv-head FP8 scales of this layer's arenas ([Hkv] fp32 views) or None
        self.compact_k_scale = self.compact_v_scale = None
        self.layer_id = -1

    def forward(self, q, k, v, *, compact_append_stored: bool = False, compact_q_rope: bool = False,
                positions: torch.Tensor | None = None, cos_sin_cache: torch.Tensor | None = None, out=None):
        ctx = get_context()
        if ctx.is_prefill:
            return prefill_attention(q, k, v, ctx.cu_seqlens_q, ctx.max_seqlen_q, self.scale, out=out)
        if not ctx.compact_kv_enabled:
            raise RuntimeError("dense paged decode is not part of this build; enable compact KV")
        base, bt, live, slot = self._layer_metadata(ctx)
        if slot is not None and not compact_append_stored:
            store_compact_kvcache(k, v, self.compact_k_cache, self.compact_v_cache, slot,
                                  k_scale=self.compact_k_scale, v_scale=self.compact_v_scale)
        rope = dict(q_rope_positions=positions if compact_q_rope else None,
                    q_rope_cos_sin_cache=cos_sin_cache if compact_q_rope else None)
        if bt is not None:
            return compact_decode_attention_paged(q, self.compact_k_cache, self.compact_v_cache, bt, live, PAGE_SIZE,
                                                  scale=self.scale, max_live_count=ctx.compact_max_live_count,
                                                  k_scale=self.compact_k_scale, v_scale=self.compact_v_scale, **rope)
        return compact_decode_attention(q, self.compact_k_cache, self.compact_v_cache, base, live, scale=self.scale,
                                        max_live_count=ctx.compact_max_live_count, k_scale=self.compact_k_scale,
                                        v_scale=self.compact_v_scale, **rope)

    def _layer_metadata(self, ctx):
        """This layer's (base offsets or None, block tables or None, live
        counts, append slots) from the step's [layers, batch, kv heads] context
        (block tables: the paged layout, [layers, batch, kv heads, pages])."""
        base, bt, live, slot = (ctx.compact_base_offsets, ctx.block_tables, ctx.compact_live_counts,
                                ctx.compact_slot_mapping)
        if live is None or (base is None and bt is None):
            raise RuntimeError("compact KV decode requires live counts and base offsets or block tables")
        if live.ndim == 3:
            live = live[self.layer_id]
            slot = None if slot is None else slot[self.layer_id]
            base = None if base is None else base[self.layer_id]
            bt = None if bt is None else bt[self.layer_id]
        return base, bt, live, slot

    def forward_fused_decode(self, q, k, v, positions, cos_sin_cache, evict_out, alpha_scale, alpha_offset,
                             q_norm=None, k_norm=None):
        """Decode step of this layer in one launch: DMS decision, RoPE, FP8
        append of k / v and compact attention (q / k / v raw from qkv_proj;
        q_norm / k_norm: Qwen3's per-head RMSNorm modules, applied in the
        kernel)."""
        ctx = get_context()
        norms = {}
        if q_norm is not None or k_norm is not None:
            norms = dict(q_norm_weight=None if q_norm is None else q_norm.weight,
                         k_norm_weight=None if k_norm is None else k_norm.weight,
                         norm_eps=(q_norm if q_norm is not None else k_norm).eps)
        if ctx.compact_plan is not None:  # the step's work plan (paged layout)
            return fused_decode_attention_planned(
                q, k, v, cos_sin_cache, self.compact_k_cache, self.compact_v_cache, evict_out, positions,
                ctx.compact_plan, self.layer_id, num_kv_heads=self.num_kv_heads, alpha_scale=alpha_scale, alpha_offset=alpha_offset,
                scale=self.scale, k_scale=self.compact_k_scale, v_scale=self.compact_v_scale, **norms)
        base, bt, live, slot = self._layer_metadata(ctx)
        return fused_dms_rope_store_compact_decode_attention(
            q, k, v, cos_sin_cache, self.compact_k_cache, self.compact_v_cache, slot, evict_out, positions, base,
            live, num_kv_heads=self.num_kv_heads, alpha_scale=alpha_scale, alpha_offset=alpha_offset,
            scale=self.scale, max_live_count=get_context().compact_max_live_count, k_scale=self.compact_k_scale,
            v_scale=self.compact_v_scale, block_tables=bt, page_size=PAGE_SIZE, **norms)
