"""Chunked prefill over a dense-retained prompt (a build extension).

The reference never chunks a compact DMS prefill: its streaming mode keeps
no dense KV (model_runner.py:252-260, 309-311) and packs only sequences whose
prefill completes in the step (model_runner.py:652-659), so a chunk could
only attend to itself.  Its prefill semantics are dense causal attention over
the whole prompt with evictions applied at pack time (attention.py:85-92;
llama.py:177-192).  This keeps those semantics for a prompt longer than the
step's token budget: each chunk's post-RoPE K/V rows and DMS decisions go
into a dense per-prompt stage, the chunk attends to the staged earlier
chunks plus itself (queries aligned to the end of the keys), and the chunk
that completes the prompt packs the whole staged prompt into its compact
spans, exactly what an unchunked prefill would pack.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


class PromptStage:
    """Dense post-RoPE K/V [layers, tokens, kv heads, head dim] (bf16) and DMS
    decisions [layers, tokens, kv heads] of a prompt's prefilled chunks;
    ``filled`` tokens are valid."""

    def __init__(self, num_layers: int, total: int, num_kv_heads: int, head_dim: int, device):
        self.total = total
        self.filled = 0
        self.k = torch.empty((num_layers, total, num_kv_heads, head_dim), device=device, dtype=torch.bfloat16)
        self.v = torch.empty_like(self.k)
        self.evict = torch.empty((num_layers, total, num_kv_heads), device=device, dtype=torch.bool)


@dataclass
class ChunkPlan:
    """The chunked sequence of a prefill batch: its chunk is batch rows
    0 .. rows-1, at prompt positions start .. start + rows - 1; the rest of
    the batch (rows rows .. end) are whole prompts."""
    seq_id: int
    stage: PromptStage
    start: int
    rows: int
    final: bool
    cu_chunk_q: torch.Tensor   # [0, rows]
    cu_chunk_k: torch.Tensor   # [0, start + rows]
    rest_ids: list             # the other sequences' ids (packed from the batch rows)
    cu_rest: torch.Tensor | None
    cu_rest_host: list | None
    max_rest: int

    @property
    def end(self) -> int:
        return self.start + self.rows


def attend_and_pack(attn, layer_id: int, q, k, v, evict_mask, ctx, scale: float):
    """One layer's prefill attention and streaming pack for a batch holding a
    chunk: stage the chunk's rows, attend (the chunk over the staged prefix +
    itself; the other prompts over themselves), pack the completed prompt from
    the stage and the other prompts from the batch rows."""
    from ..layers.attention import prefill_attention
    ch = ctx.prefill_chunk
    n, s0, e = ch.rows, ch.start, ch.end
    st = ch.stage
    st.k[layer_id, s0:e].copy_(k[:n])
    st.v[layer_id, s0:e].copy_(v[:n])
    if evict_mask is not None:
        st.evict[layer_id, s0:e].copy_(evict_mask[:n])
    mgr = ctx.streaming_pack_manager
    if mgr is not None and ctx.dms_capture_enabled:
        if ch.final:
            mgr.streaming_pack_layer(layer_id=layer_id, k=st.k[layer_id, :e], v=st.v[layer_id, :e],
                                     evict_mask=st.evict[layer_id, :e], cu_seqlens_q=ch.cu_chunk_k,
                                     seq_ids=[ch.seq_id], window_size=ctx.streaming_pack_window_size,
                                     cu_seqlens_host=[0, e])
        if ch.rest_ids:
            mgr.streaming_pack_layer(layer_id=layer_id, k=k[n:], v=v[n:], evict_mask=evict_mask[n:],
                                     cu_seqlens_q=ch.cu_rest, seq_ids=ch.rest_ids,
                                     window_size=ctx.streaming_pack_window_size, cu_seqlens_host=ch.cu_rest_host)
    out = torch.empty((q.shape[0], q.shape[1], q.shape[2]), device=q.device, dtype=q.dtype)
    prefill_attention(q[:n], st.k[layer_id, :e], st.v[layer_id, :e], ch.cu_chunk_q, n, scale, out=out[:n],
                      cu_seqlens_k=ch.cu_chunk_k)
    if q.shape[0] > n:
        prefill_attention(q[n:], k[n:], v[n:], ch.cu_rest, ch.max_rest, scale, out=out[n:])
    return out
