"""Block-table invariants of the paged compact-KV layout (test helper).

The reference has no block tables (it stores flat spans), so the tables are
pinned by invariants instead of vectors:
  * every span (layer, slot, kv head) holds exactly ceil(live / 16) pages,
    listed in table[0 .. held) with -1 after them;
  * within a layer, no page id appears twice across the spans, and the spans'
    pages plus the free stack page_stack[l, 0 .. top) are exactly 0 .. P-1;
  * slots without a sequence hold nothing and have live count 0.
"""
from __future__ import annotations

import numpy as np

PAGE = 16


def check_page_invariants(mgr, *, active_slots=None) -> dict:
    """Assert the invariants over the whole pool; returns per-layer counts."""
    bt = mgr.block_tables.cpu().numpy()
    held = mgr.pages_held.cpu().numpy()
    live = mgr.layer_major_live_counts.cpu().numpy()
    stack = mgr.page_stack.cpu().numpy()
    top = mgr.page_top.cpu().numpy()
    L, S, H, P = bt.shape
    if active_slots is None:
        active_slots = {st.active_slot for st in mgr.seq_states.values()}
    used = []
    for l in range(L):
        pages = []
        for s in range(S):
            for h in range(H):
                n = int(held[l, s, h])
                if s not in active_slots:
                    assert n == 0 and live[l, s, h] == 0, f"free slot {s} holds pages (layer {l}, head {h})"
                assert n == -(-int(live[l, s, h]) // PAGE), \
                    f"span (l={l}, s={s}, h={h}) holds {n} pages for live {live[l, s, h]}"
                row = bt[l, s, h]
                assert (row[:n] >= 0).all() and (row[:n] < mgr.num_pages).all(), f"bad page id in span {(l, s, h)}"
                assert (row[n:] == -1).all(), f"stale table entries after held in span {(l, s, h)}"
                pages.extend(row[:n].tolist())
        assert len(pages) == len(set(pages)), f"layer {l}: a page is held by two spans"
        free = stack[l, :int(top[l])].tolist()
        assert len(free) == len(set(free)), f"layer {l}: a page is on the free stack twice"
        assert not set(free) & set(pages), f"layer {l}: a held page is also free"
        assert sorted(free + pages) == list(range(mgr.num_pages)), f"layer {l}: pages lost or invented"
        used.append(len(pages))
    return {"pages_used": used}


def gather_span_rows(mgr, layer_id: int, slot: int, head: int, arena_rows: np.ndarray) -> np.ndarray:
    """Rows [live, ...] of one span in rank order from a host copy of the
    layer's arena."""
    n = int(mgr.layer_major_live_counts[layer_id, slot, head])
    table = mgr.block_tables[layer_id, slot, head].cpu().numpy()
    r = np.arange(n)
    return arena_rows[table[r // PAGE] * PAGE + r % PAGE]
