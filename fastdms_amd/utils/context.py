"""Per-step metadata channel (mirror of fastdms/utils/context.py:5-85).

A process-global ``Context`` that the model runner sets before each forward
and the attention glue reads.  Not thread-safe, like the reference's.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    compact_kv_enabled: bool = False
    compact_base_offsets: torch.Tensor | None = None
    compact_live_counts: torch.Tensor | None = None
    compact_slot_mapping: torch.Tensor | None = None
    compact_max_live_count: int = 0
    dms_capture_enabled: bool = False
    dms_alpha_scale: float = 100.0
    dms_alpha_offset: float = 5.0
    dms_layer_evictions: dict | None = None
    dms_layer_evictions_buffer: torch.Tensor | None = None
    streaming_pack_manager: object | None = None
    streaming_pack_seq_ids: list | None = None
    streaming_pack_window_size: int = 0
    # host copy of cu_seqlens_q (saves a device sync in the streaming pack)
    cu_seqlens_q_host: list | None = None
    # a chunk of a long prompt in this prefill batch (engine.chunked_prefill.ChunkPlan)
    prefill_chunk: object | None = None
    # the decode step's attention work plan (layers.compact_attention.DecodePlan), or None
    compact_plan: object | None = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, compact_kv_enabled=False,
                compact_base_offsets=None, compact_live_counts=None, compact_slot_mapping=None,
                compact_max_live_count=0, dms_capture_enabled=False, dms_alpha_scale=100.0, dms_alpha_offset=5.0,
                dms_layer_evictions=None, dms_layer_evictions_buffer=None, streaming_pack_manager=None,
                streaming_pack_seq_ids=None, streaming_pack_window_size=0, cu_seqlens_q_host=None,
                prefill_chunk=None, compact_plan=None) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping,
                       context_lens, block_tables, compact_kv_enabled, compact_base_offsets, compact_live_counts,
                       compact_slot_mapping, compact_max_live_count, dms_capture_enabled, dms_alpha_scale,
                       dms_alpha_offset, dms_layer_evictions, dms_layer_evictions_buffer, streaming_pack_manager,
                       streaming_pack_seq_ids, streaming_pack_window_size, cu_seqlens_q_host, prefill_chunk,
                       compact_plan)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
