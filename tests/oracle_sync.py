"""Hand the engine's compact state to the model oracle (test helper).

The oracle keeps the reference's flat spans.  For the span layout the GPU's
arenas and span metadata are copied as they are; for the paged layout each
(layer, seq, kv head) span is gathered from its pages in rank order into a
fresh flat arena (spans laid out one after another, each with room for the
sequence's metadata capacity), so the oracle's next decode step starts from
the same K/V rows, live counts, positions and decisions either way.
"""
from __future__ import annotations

import numpy as np
import torch

PAGE = 16


def sync_oracle_state(orc, mgr, seq_ids) -> None:
    from oracle import compact_kv as ock
    om = orc.mgr
    if not getattr(mgr, "paged", False):
        om.free_ranges_per_layer = [list(r) for r in mgr.free_ranges_per_layer]
        om.compact_k_per_layer = [t.view(torch.uint8).cpu().numpy().copy() for t in mgr.compact_k_per_layer]
        om.compact_v_per_layer = [t.view(torch.uint8).cpu().numpy().copy() for t in mgr.compact_v_per_layer]
        for sid in seq_ids:
            st = mgr.seq_states[sid]
            om.seq_states[sid] = ock.SeqState(
                sid, st.base_offsets.cpu().numpy().copy(), st.range_capacity.cpu().numpy().copy(),
                st.live_counts.cpu().numpy().copy(), st.token_positions.cpu().numpy().copy(),
                st.evict_mask.cpu().numpy().copy(), st.max_capacity_per_lh, st.decode_headroom,
                st.dms_initial_expiry_done, st.last_dms_expiry_position)
        return
    L, H = mgr.num_layers, mgr.num_kv_heads
    live_all = mgr.layer_major_live_counts.cpu().numpy()
    slots = [mgr.seq_states[sid].active_slot for sid in seq_ids]
    caps = [mgr.seq_states[sid].max_capacity_per_lh for sid in seq_ids]
    new_k, new_v, bases = ock.spans_from_pages(
        [t.view(torch.uint8).cpu().numpy() for t in mgr.compact_k_per_layer],
        [t.view(torch.uint8).cpu().numpy() for t in mgr.compact_v_per_layer], mgr.block_tables.cpu().numpy(),
        live_all, slots, caps, PAGE)
    for sid, slot, cap, base in zip(seq_ids, slots, caps, bases):
        st = mgr.seq_states[sid]
        om.seq_states[sid] = ock.SeqState(
            sid, base, np.full((L, H), cap, np.int32), live_all[:, slot].copy(),
            st.token_positions.cpu().numpy().copy(), st.evict_mask.cpu().numpy().copy(), cap, st.decode_headroom,
            st.dms_initial_expiry_done, st.last_dms_expiry_position)
    om.compact_k_per_layer, om.compact_v_per_layer = new_k, new_v
    om.free_ranges_per_layer = [[] for _ in range(L)]
