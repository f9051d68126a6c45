"""Compact-KV oracle (test infrastructure only).

Restates fastdms/engine/compact_kv.py of the reference with numpy: the
streaming prefill pack (count -> exclusive scan -> rank scatter), decode
append-slot metadata, decision recording, the exact / incremental expiry
compactions and the first-fit per-layer range allocator, plus the
``apply_dms_evictions`` policy that decides which of them runs on a step.

Compact storage is modelled as numpy *storage* arrays (uint8 e4m3fn bits,
uint16 bf16 bits, float16 or float32) shaped [slots, head_dim].  K/V sources
are float32 arrays holding values of their own dtype (every dtype here is
exactly representable in float32); the store cast to the arena dtype is
``numerics.to_storage`` (RNE, FP8 saturating).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import numerics

PACK_BLOCK_T = 256  # compact_kv.py:276, 318 — the chunk the rank scan runs over


# ---------------------------------------------------------------------------
# streaming prefill pack (A2, A4, A5, A6)
# ---------------------------------------------------------------------------

def prefill_keep(seq_evict, seq_len: int, window_size: int) -> np.ndarray:
    """Prefill keep rule, compact_kv.py:156-163 / 209-217 / 971-974.

    keep[t, h] = (t < seq_len) & (~evict[t, h] | t >= max(0, seq_len-1-W)).
    """
    seq_evict = np.asarray(seq_evict, dtype=bool)
    t = np.arange(seq_evict.shape[0])
    in_window = t >= max(0, int(seq_len) - 1 - int(window_size))
    return (t[:, None] < seq_len) & ((~seq_evict) | in_window[:, None])


def streaming_pack_fused_rank_prepare(seq_evict, seq_len: int, window_size: int):
    """compact_kv.py:265-296: per-256-token-chunk keep counts, live per head
    and the exclusive chunk offsets [Hkv, chunks]."""
    if seq_len <= 0:
        raise ValueError("seq_len must be positive")
    keep = prefill_keep(np.asarray(seq_evict)[:seq_len], seq_len, window_size)
    h = keep.shape[1]
    chunks = -(-seq_len // PACK_BLOCK_T)
    padded = np.zeros((chunks * PACK_BLOCK_T, h), dtype=np.int64)
    padded[:seq_len] = keep
    counts = padded.reshape(chunks, PACK_BLOCK_T, h).sum(axis=1).T.astype(np.int32)  # [H, chunks]
    live = counts.sum(axis=1).astype(np.int32)
    offsets = (np.cumsum(counts, axis=1) - counts).astype(np.int32)
    return live, offsets


def inv_scales(scale) -> np.ndarray:
    """fp32 1 / scale per kv head (an IEEE division, as the kernels compute it)."""
    s = np.asarray(scale, np.float32)
    return (np.float32(1.0) / s).astype(np.float32)


def streaming_pack_scatter(*, k, v, keep, rank, seq_evict, compact_k, compact_v, token_positions,
                           evict_mask, base_offsets, start: int, seq_len: int, dtype_code: int, k_scale=None, v_scale=None):
    """compact_kv.py:38-137 (precomputed keep/rank) — in place on numpy arrays.

    k, v: float32 values [T_total, Hkv, D]; compact_*: storage [slots, D];
    token_positions [Hkv, C] int32; evict_mask [Hkv, C] bool; base_offsets [Hkv].
    """
    keep = np.asarray(keep, dtype=bool)[:seq_len]
    rank = np.asarray(rank, dtype=np.int64)[:seq_len]
    t_idx, h_idx = np.nonzero(keep)
    dst_rank = rank[t_idx, h_idx]
    dst = np.asarray(base_offsets, dtype=np.int64)[h_idx] + dst_rank
    kv = np.asarray(k, np.float32)[start + t_idx, h_idx]
    vv = np.asarray(v, np.float32)[start + t_idx, h_idx]
    if k_scale is not None:  # per-kv-head FP8 scale: stored = x * fp32(1 / scale)
        kv = (kv * inv_scales(k_scale)[h_idx, None]).astype(np.float32)
    if v_scale is not None:
        vv = (vv * inv_scales(v_scale)[h_idx, None]).astype(np.float32)
    compact_k[dst] = numerics.to_storage(kv, dtype_code)
    compact_v[dst] = numerics.to_storage(vv, dtype_code)
    token_positions[h_idx, dst_rank] = t_idx.astype(np.int32)
    evict_mask[h_idx, dst_rank] = np.asarray(seq_evict, dtype=bool)[t_idx, h_idx]


def streaming_pack_rank_scatter(*, k, v, seq_evict, compact_k, compact_v, token_positions, evict_mask,
                                base_offsets, start: int, seq_len: int, window_size: int, dtype_code: int,
                                k_scale=None, v_scale=None):
    """compact_kv.py:168-262 fused count/rank scatter; rank = stable order of
    kept tokens (cumsum(keep) - 1), so it equals the precomputed-rank form."""
    if seq_len <= 0:
        return np.zeros(np.asarray(seq_evict).shape[1], dtype=np.int32)
    seq_evict = np.asarray(seq_evict, dtype=bool)[:seq_len]
    keep = prefill_keep(seq_evict, seq_len, window_size)
    rank = np.cumsum(keep.astype(np.int64), axis=0) - 1
    streaming_pack_scatter(k=k, v=v, keep=keep, rank=rank, seq_evict=seq_evict, compact_k=compact_k,
                           compact_v=compact_v, token_positions=token_positions, evict_mask=evict_mask,
                           base_offsets=base_offsets, start=start, seq_len=seq_len, dtype_code=dtype_code,
                           k_scale=k_scale, v_scale=v_scale)
    return keep.sum(axis=0).astype(np.int32)


def pack_compact_kv(k, v, live_mask):
    """compact_kv.py:1798-1850: canonical dense -> flat span pack.

    k, v: [B, T, Hkv, D]; live_mask [B, Hkv, T].  Returns (compact_k,
    compact_v, base_offsets [B,Hkv], live_counts [B,Hkv], token_positions).
    """
    k = np.asarray(k)
    v = np.asarray(v)
    live_mask = np.asarray(live_mask, dtype=bool)
    b, t, h, d = k.shape
    live_counts = live_mask.sum(axis=-1).astype(np.int32)
    total = int(live_counts.sum())
    ck = np.empty((total, d), dtype=k.dtype)
    cv = np.empty((total, d), dtype=v.dtype)
    base = np.empty((b, h), dtype=np.int32)
    positions = np.empty((total,), dtype=np.int32)
    cursor = 0
    for bi in range(b):
        for hi in range(h):
            keep = np.nonzero(live_mask[bi, hi])[0]
            base[bi, hi] = cursor
            n = keep.size
            if n:
                ck[cursor:cursor + n] = k[bi, keep, hi]
                cv[cursor:cursor + n] = v[bi, keep, hi]
                positions[cursor:cursor + n] = keep
                cursor += n
    return ck, cv, base, live_counts, positions


def build_emulated_dms_live_mask(*, num_layers, num_kv_heads, num_tokens, mode, stride, recent_tokens):
    """compact_kv.py:523-551 (non-DMS retention modes)."""
    if mode == "all":
        return np.ones((num_layers, num_kv_heads, num_tokens), dtype=bool)
    if mode != "dms_stride":
        raise ValueError(f"unknown compact KV retention mode: {mode}")
    if stride <= 0:
        raise ValueError("stride must be positive")
    if recent_tokens < 0:
        raise ValueError("recent_tokens must be non-negative")
    pos = np.arange(num_tokens)
    mask = np.zeros((num_layers, num_kv_heads, num_tokens), dtype=bool)
    if recent_tokens:
        mask[..., max(0, num_tokens - recent_tokens):] = True
    if num_tokens:
        for l in range(num_layers):
            for h in range(num_kv_heads):
                mask[l, h] |= (pos + l + h) % stride == 0
                mask[l, h, -1] = True
    return mask


# ---------------------------------------------------------------------------
# expiry (A11 exact path, A12 full kernel, A13 incremental kernel)
# ---------------------------------------------------------------------------

def expiry_exact(*, positions, evict, live, base, compact_k, compact_v, current_position: int, window_size: int):
    """One (seq, head) span, in place.  compact_kv.py:1270-1337 and
    compact_attention.py:690-773: keep = (slot < live) & (~evict | cur-pos <= W);
    kept slots move to cumsum-rank order; trailing metadata -> (-1, False).
    Returns the new live count."""
    cap = positions.shape[0]
    s = np.arange(cap)
    pos = positions.astype(np.int64)
    keep = (s < live) & ((~evict) | ((int(current_position) - pos) <= int(window_size)))
    src = np.nonzero(keep)[0]
    new_live = src.size
    if compact_k is not None:
        rows_k = compact_k[base + src].copy()
        rows_v = compact_v[base + src].copy()
        compact_k[base:base + new_live] = rows_k
        compact_v[base:base + new_live] = rows_v
    new_pos = np.full(cap, -1, dtype=np.int32)
    new_ev = np.zeros(cap, dtype=bool)
    new_pos[:new_live] = positions[src]
    new_ev[:new_live] = evict[src]
    positions[:] = new_pos
    evict[:] = new_ev
    return int(new_live)


def expiry_incremental(*, positions, evict, live, base, compact_k, compact_v, current_position: int,
                       window_size: int):
    """compact_attention.py:776-858: remove only the *first* slot with
    evict & pos < cur - W and shift the tail left by one.  Returns new live."""
    cap = positions.shape[0]
    live = int(live)
    cutoff = int(current_position) - int(window_size)
    s = np.arange(min(live, cap))
    expired = evict[s] & (positions[s].astype(np.int64) < cutoff)
    hits = np.nonzero(expired)[0]
    if hits.size == 0:
        return live
    e = int(hits[0])
    positions[e:live - 1] = positions[e + 1:live].copy()
    evict[e:live - 1] = evict[e + 1:live].copy()
    if compact_k is not None:
        compact_k[base + e:base + live - 1] = compact_k[base + e + 1:base + live].copy()
        compact_v[base + e:base + live - 1] = compact_v[base + e + 1:base + live].copy()
    positions[live - 1] = -1
    evict[live - 1] = False
    return live - 1


# ---------------------------------------------------------------------------
# stateful manager (A7, A8, A11, A14, A15) — first-fit per-layer ranges
# ---------------------------------------------------------------------------

def spans_from_pages(arenas_k, arenas_v, block_tables, live_counts, slots, caps, page_size=16):
    """Flat spans of paged compact KV (no reference counterpart: the reference
    stores flat spans only).  arenas_*: per-layer [rows, row_bytes] storage;
    block_tables [L, S, H, pages]; live_counts [L, S, H]; slots / caps: the
    metadata row and span capacity of each sequence.  Span (l, slots[i], h) is
    copied in rank order (rank r from row table[r // P] * P + r % P) to rows
    base .. base + live of a new arena, spans laid out one after another with
    caps[i] rows each.  Returns (new_k, new_v, bases) with bases[i] [L, H]."""
    L, _, H, _ = block_tables.shape
    width = arenas_k[0].shape[1]
    total = int(sum(caps)) * H
    new_k = [np.zeros((total, width), arenas_k[0].dtype) for _ in range(L)]
    new_v = [np.zeros((total, width), arenas_v[0].dtype) for _ in range(L)]
    bases = []
    at = 0
    for slot, cap in zip(slots, caps):
        base = np.zeros((L, H), np.int32)
        for h in range(H):
            base[:, h] = at
            for l in range(L):
                n = int(live_counts[l, slot, h])
                r = np.arange(n)
                rows = block_tables[l, slot, h][r // page_size].astype(np.int64) * page_size + r % page_size
                new_k[l][at:at + n] = arenas_k[l][rows]
                new_v[l][at:at + n] = arenas_v[l][rows]
            at += int(cap)
        bases.append(base)
    return new_k, new_v, bases


@dataclass
class SeqState:
    seq_id: int
    base_offsets: np.ndarray     # [L, H] int32, -1 = unallocated
    range_capacity: np.ndarray   # [L, H] int32
    live_counts: np.ndarray      # [L, H] int32
    token_positions: np.ndarray  # [L, H, C] int32
    evict_mask: np.ndarray       # [L, H, C] bool
    max_capacity_per_lh: int
    decode_headroom: int
    dms_initial_expiry_done: bool = False
    last_dms_expiry_position: int = -1


_TRUTHY = {"1", "true", "yes", "on"}


@dataclass
class OracleCompactKVManager:
    """CPU restatement of CompactKVManager with per-layer storage
    (compact_kv.py:554-1795, per_layer_storage=True branch)."""
    num_layers: int
    num_kv_heads: int
    capacity_tokens: int
    max_model_len: int
    head_dim: int = 0
    dtype_code: int = numerics.DT_FP8
    target_live_tokens_per_seq: int | None = None
    free_ranges_per_layer: list = field(default_factory=list)
    seq_states: dict = field(default_factory=dict)
    compact_k_per_layer: list = field(default_factory=list)
    compact_v_per_layer: list = field(default_factory=list)

    def __post_init__(self):
        if self.capacity_tokens <= 0:
            raise ValueError("capacity_tokens must be positive")
        self.free_ranges_per_layer = [[(0, self.capacity_tokens)] for _ in range(self.num_layers)]
        self.compact_k_per_layer = [None] * self.num_layers
        self.compact_v_per_layer = [None] * self.num_layers

    # -- allocator (compact_kv.py:697-751) --
    def free_tokens_in_layer(self, layer_id):
        return sum(n for _, n in self.free_ranges_per_layer[layer_id])

    @property
    def free_tokens(self):
        return sum(self.free_tokens_in_layer(l) for l in range(self.num_layers))

    def _alloc_range(self, layer_id, length):
        free = self.free_ranges_per_layer[layer_id]
        for idx, (start, avail) in enumerate(free):
            if avail < length:
                continue
            if avail == length:
                free.pop(idx)
            else:
                free[idx] = (start + length, avail - length)
            return start
        raise RuntimeError(f"compact KV capacity exhausted in layer {layer_id}: requested {length}")

    def _free_range(self, layer_id, start, length):
        if length <= 0:
            return
        free = self.free_ranges_per_layer[layer_id]
        free.append((start, length))
        free.sort()
        merged = []
        for rs, rl in free:
            if merged and rs <= merged[-1][0] + merged[-1][1]:
                ps, pl = merged[-1]
                merged[-1] = (ps, max(ps + pl, rs + rl) - ps)
            else:
                merged.append((rs, rl))
        self.free_ranges_per_layer[layer_id] = merged

    def _reservation_tokens(self, num_prompt_tokens, max_tokens):
        worst = min(self.max_model_len, num_prompt_tokens + max_tokens)
        if self.target_live_tokens_per_seq is not None:
            return min(worst, max(1, int(self.target_live_tokens_per_seq)))
        return worst

    def allocate(self, seq_id, num_prompt_tokens, max_tokens):
        """compact_kv.py:753-828 (non-layer-major branch)."""
        if seq_id in self.seq_states:
            return self.seq_states[seq_id]
        cap = self._reservation_tokens(num_prompt_tokens, max_tokens)
        if cap <= 0:
            raise ValueError("invalid reservation")
        L, H = self.num_layers, self.num_kv_heads
        st = SeqState(seq_id, np.full((L, H), -1, np.int32), np.zeros((L, H), np.int32),
                      np.zeros((L, H), np.int32), np.full((L, H, cap), -1, np.int32),
                      np.zeros((L, H, cap), bool), cap, int(max_tokens))
        self.seq_states[seq_id] = st
        return st

    def allocate_layer_ranges_for_seq(self, st, layer_id, live_per_head):
        """compact_kv.py:830-857: size = max(min(live + headroom, cap), 1),
        first-fit head by head, rollback on failure."""
        sizes = [max(min(int(x) + st.decode_headroom, st.max_capacity_per_lh), 1) for x in live_per_head]
        bases = []
        try:
            for size in sizes:
                bases.append(self._alloc_range(layer_id, size))
        except Exception:
            for h2, b2 in enumerate(bases):
                self._free_range(layer_id, b2, sizes[h2])
            raise
        st.base_offsets[layer_id] = bases
        st.range_capacity[layer_id] = sizes
        return np.asarray(bases, dtype=np.int32)

    def _ensure_layer_storage(self, layer_id, min_tokens):
        """compact_kv.py:661-695: grow to a 256 multiple and keep old rows."""
        cur = self.compact_k_per_layer[layer_id]
        if cur is not None and cur.shape[0] >= min_tokens:
            return
        new = max(256, -(-min_tokens // 256) * 256)
        sd = numerics.storage_dtype(self.dtype_code)
        nk = np.zeros((new, self.head_dim), dtype=sd)
        nv = np.zeros((new, self.head_dim), dtype=sd)
        if cur is not None:
            nk[:cur.shape[0]] = cur
            nv[:cur.shape[0]] = self.compact_v_per_layer[layer_id]
        self.compact_k_per_layer[layer_id] = nk
        self.compact_v_per_layer[layer_id] = nv

    def streaming_pack_layer(self, *, layer_id, k, v, evict_mask, cu_seqlens_q, seq_ids, window_size,
                             k_scale=None, v_scale=None):
        """compact_kv.py:915-1099 (per-layer storage branch); optional
        per-kv-head FP8 scales of the layer (no reference counterpart)."""
        cu = [int(x) for x in cu_seqlens_q]
        lives = {}
        high = 0
        for i, sid in enumerate(seq_ids):
            st = self.seq_states.get(sid)
            if st is None:
                continue
            n = cu[i + 1] - cu[i]
            seq_ev = np.asarray(evict_mask)[cu[i]:cu[i + 1]]
            live, _ = streaming_pack_fused_rank_prepare(seq_ev, n, window_size)
            lives[sid] = live
            self.allocate_layer_ranges_for_seq(st, layer_id, live)
            high = max(high, int((st.base_offsets[layer_id].astype(np.int64)
                                  + st.range_capacity[layer_id]).max()))
        self._ensure_layer_storage(layer_id, high)
        ck, cv = self.compact_k_per_layer[layer_id], self.compact_v_per_layer[layer_id]
        for i, sid in enumerate(seq_ids):
            st = self.seq_states.get(sid)
            if st is None:
                raise RuntimeError(f"sequence {sid} has no compact KV allocation")
            n = cu[i + 1] - cu[i]
            if n <= 0:
                continue
            live = lives[sid]
            if int(live.max()) > st.max_capacity_per_lh:
                raise RuntimeError("streaming pack live count exceeds metadata capacity")
            st.token_positions[layer_id] = -1
            st.evict_mask[layer_id] = False
            if int(live.max()) == 0:
                st.live_counts[layer_id] = 0
                continue
            streaming_pack_rank_scatter(k=k, v=v, seq_evict=np.asarray(evict_mask)[cu[i]:cu[i + 1]],
                                        compact_k=ck, compact_v=cv,
                                        token_positions=st.token_positions[layer_id],
                                        evict_mask=st.evict_mask[layer_id],
                                        base_offsets=st.base_offsets[layer_id], start=cu[i], seq_len=n,
                                        window_size=window_size, dtype_code=self.dtype_code, k_scale=k_scale,
                                        v_scale=v_scale)
            st.live_counts[layer_id] = live

    # -- decode metadata (compact_kv.py:1727-1770) --
    def prepare_decode_metadata(self, seq_ids):
        sts = [self.seq_states[s] for s in seq_ids]
        base = np.stack([s.base_offsets for s in sts], axis=1)
        slot = np.stack([s.base_offsets + s.live_counts for s in sts], axis=1).astype(np.int32)
        for s in sts:
            s.live_counts += 1
        live = np.stack([s.live_counts for s in sts], axis=1)
        return base, live, slot, max(s.max_capacity_per_lh for s in sts)

    # -- decision recording (compact_kv.py:1562-1725) --
    def record_appended_dms_decisions(self, seq_ids, current_positions, evict_all):
        evict_all = np.asarray(evict_all, dtype=bool)  # [L, B, H]
        for b, sid in enumerate(seq_ids):
            st = self.seq_states[sid]
            idx = st.live_counts - 1
            for l in range(self.num_layers):
                for h in range(self.num_kv_heads):
                    st.token_positions[l, h, idx[l, h]] = int(current_positions[b])
                    st.evict_mask[l, h, idx[l, h]] = evict_all[l, b, h]
        return {"eviction_decisions_true": int(evict_all.sum()), "eviction_decisions_total": int(evict_all.size)}

    # -- expiry policy (compact_kv.py:1174-1560) --
    def _expire_all(self, seq_ids, current_positions, window_size, incremental):
        before = np.stack([self.seq_states[s].live_counts for s in seq_ids]).astype(np.int64)
        for sid, cur in zip(seq_ids, current_positions):
            st = self.seq_states[sid]
            for l in range(self.num_layers):
                ck, cv = self.compact_k_per_layer[l], self.compact_v_per_layer[l]
                for h in range(self.num_kv_heads):
                    fn = expiry_incremental if incremental else expiry_exact
                    st.live_counts[l, h] = fn(positions=st.token_positions[l, h], evict=st.evict_mask[l, h],
                                              live=int(st.live_counts[l, h]), base=int(st.base_offsets[l, h]),
                                              compact_k=ck, compact_v=cv, current_position=int(cur),
                                              window_size=window_size)
        after = np.stack([self.seq_states[s].live_counts for s in seq_ids]).astype(np.int64)
        return {"evicted_tokens": int((before - after).sum()),
                "live_tokens_before_min": int(before.min()), "live_tokens_before_max": int(before.max()),
                "live_tokens_after_min": int(after.min()), "live_tokens_after_max": int(after.max())}

    def expiry_action(self, seq_ids, current_positions, window_size, triton_mode="auto", interval_env=None):
        """The branch compact_kv.py:1189-1241 takes: 'exact', 'full',
        'incremental' or 'skip' (the reference's env flags are arguments)."""
        b = len(seq_ids)
        mode = (triton_mode or "").strip().lower()
        auto = mode in {"", "auto"} and (b == 1 or b >= 4)
        use_fast = b > 0 and (mode in _TRUTHY or auto)
        if use_fast:
            sts = [self.seq_states[s] for s in seq_ids]
            sequential = all(s.dms_initial_expiry_done and int(c) == s.last_dms_expiry_position + 1
                             for s, c in zip(sts, current_positions))
            if sequential:
                interval = int(interval_env) if interval_env is not None else (max(1, int(window_size)) if auto else 1)
                if interval > 1:
                    if not any(int(c) % interval == 0 for c in current_positions):
                        return "skip"
                    return "full"
                return "incremental"
        return "exact"

    def apply_dms_evictions(self, seq_ids, current_positions, *, window_size, triton_mode="auto",
                            interval_env=None):
        action = self.expiry_action(seq_ids, current_positions, window_size, triton_mode, interval_env)
        sts = [self.seq_states[s] for s in seq_ids]
        if action == "skip":
            for s, c in zip(sts, current_positions):
                s.last_dms_expiry_position = int(c)
            live = np.stack([s.live_counts for s in sts]).astype(np.int64)
            return action, {"evicted_tokens": 0, "live_tokens_before_min": int(live.min()),
                            "live_tokens_before_max": int(live.max()), "live_tokens_after_min": int(live.min()),
                            "live_tokens_after_max": int(live.max())}
        stats = self._expire_all(seq_ids, current_positions, window_size, incremental=(action == "incremental"))
        for s, c in zip(sts, current_positions):
            if action != "incremental":
                s.dms_initial_expiry_done = True
            s.last_dms_expiry_position = int(c)
        return action, stats

    def free(self, seq_id):
        """compact_kv.py:1772-1795."""
        st = self.seq_states.pop(seq_id, None)
        if st is None:
            return
        for l in range(self.num_layers):
            for h in range(self.num_kv_heads):
                b, n = int(st.base_offsets[l, h]), int(st.range_capacity[l, h])
                if b >= 0 and n > 0:
                    self._free_range(l, b, n)
