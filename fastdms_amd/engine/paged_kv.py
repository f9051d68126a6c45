"""Compact KV in 16-row FP8 pages with a device-resident page pool.

No reference counterpart as a layout: the reference packs each (layer, seq,
kv head) into a flat span carved from a per-layer arena by a first-fit host
allocator (compact_kv.py:697-857) and syncs the live counts to the host per
prefill layer to size the spans (compact_kv.py:955-1099).  Here every span is
a list of 16-row pages from its layer's free-page stack, and every allocation
happens on the device:

* prefill pack: the count/scan kernel pops ceil(live / 16) pages per
  (seq, head) and writes the span's block-table row; the rank scatter writes
  rank r to row table[r >> 4] * 16 + (r & 15).  No host sync per layer;
* decode append: one launch for all layers pops a page when a span's pages
  are full and returns the physical row of the new rank;
* expiry re-compacts through the tables and returns the pages past
  ceil(live / 16) to the stack; a sequence-free pushes all of its pages back.

Ranks, token positions, evict flags and live counts are exactly those of the
span layout (the DMS metadata is rank-indexed, unchanged); only the rows the
K / V bytes live in differ.  The host never learns which pages a span holds.
It keeps, per sequence, an upper bound of the pages the sequence can hold in
any layer and admits work only while the bounds fit the pool, so the device
pops never find the pool short; a pool that is short anyway sets a device
flag that the next host sync turns into an error.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _native as nat
from .compact_kv import PACK_CHUNK, CompactCapacityExhausted, CompactKVManager, _pack_vec
from .sequence import Sequence

PAGE_SIZE = 16  # rows per page; the kernels address rank r as table[r >> 4] * 16 + (r & 15)


@dataclass(slots=True)
class _PageBound:
    """Host bound of one sequence's pages per layer: at most ``sync_pages``
    at the last sync point, plus, per kv head, one page per 16 appends since
    then (``appended``) and still reserved (``reserve_left``).  Before its
    prefill has completed (``packed`` False) only the reserve counts: the
    prompt's pages come out of the prefill's page budget."""
    sync_pages: int
    appended: int
    reserve_left: int
    packed: bool = False


class PagedCompactKVManager(CompactKVManager):
    """CompactKVManager on the paged layout (same methods and metadata; the
    arenas hold ``capacity_tokens // 16`` pages per layer)."""

    paged = True

    def __init__(self, *, num_layers: int, num_kv_heads: int, capacity_tokens: int, max_model_len: int,
                 device: torch.device | str, head_dim: int, compact_dtype: torch.dtype, max_active_seqs: int,
                 decode_reserve_tokens: int | None = None, fp8_scales: str = "unit"):
        num_pages = int(capacity_tokens) // PAGE_SIZE
        if num_pages <= 0:
            raise ValueError(f"paged compact KV needs at least {PAGE_SIZE} tokens of capacity per layer")
        super().__init__(num_layers=num_layers, num_kv_heads=num_kv_heads, capacity_tokens=num_pages * PAGE_SIZE,
                         max_model_len=max_model_len, device=device, head_dim=head_dim,
                         compact_dtype=compact_dtype, per_layer_storage=True, layer_major_metadata=True,
                         max_active_seqs=max_active_seqs, preallocate=True,
                         decode_reserve_tokens=decode_reserve_tokens, fp8_scales=fp8_scales)
        self.free_ranges_per_layer = [[] for _ in range(num_layers)]  # no host ranges in this layout
        self.num_pages = num_pages
        self.max_pages = -(-int(max_model_len) // PAGE_SIZE)
        L, S, H = num_layers, self.max_active_seqs, num_kv_heads
        dev = self.device
        self.block_tables = torch.full((L, S, H, self.max_pages), -1, device=dev, dtype=torch.int32)
        self.pages_held = torch.zeros((L, S, H), device=dev, dtype=torch.int32)
        # per-layer free-page stacks: ids page_stack[l, 0 .. page_top[l])
        self.page_stack = torch.arange(num_pages, device=dev, dtype=torch.int32).repeat(L, 1).contiguous()
        self.page_top = torch.full((L,), num_pages, device=dev, dtype=torch.int32)
        self.overflow = torch.zeros(1, device=dev, dtype=torch.int32)
        # pages a prefill's packs may take per layer (what the running
        # sequences' bounds leave), debited by the pack kernels' pops
        self.page_budget = torch.zeros(L, device=dev, dtype=torch.int32)
        pin = dev.type == "cuda"
        self._overflow_host = torch.zeros(1, dtype=torch.int32, pin_memory=pin)
        self._overflow_staged = False
        self._prefill_pages_host = torch.zeros(self.max_active_seqs, dtype=torch.int32, pin_memory=pin)
        self._prefill_check: list[tuple[int, int]] = []
        self._bounds: dict[int, _PageBound] = {}
        self.page_syncs = 0

    # -- host page accounting ------------------------------------------------
    def _seq_bound(self, b: _PageBound, steps: int = 1) -> int:
        future = b.appended + max(b.reserve_left, steps)
        grow = self.num_kv_heads * (-(-future // PAGE_SIZE))
        if not b.packed:
            return grow
        return min(self.num_kv_heads * self.max_pages, b.sync_pages + grow)

    def pages_bound(self, steps: int = 1) -> int:
        """Upper bound of the pages any one layer can hold after the next
        ``steps`` decode appends of every sequence (or its reserved appends,
        whichever is more)."""
        return sum(self._seq_bound(b, steps) for b in self._bounds.values())

    def refresh_page_bounds(self) -> None:
        """One device->host copy of the page counts: each packed sequence's
        bound becomes its exact page count (largest over layers)."""
        held = self.pages_held.cpu()
        self.page_syncs += 1
        for sid, b in self._bounds.items():
            if not b.packed:
                continue
            slot = self.seq_states[sid].active_slot
            b.sync_pages = int(held[:, slot, :].sum(dim=-1).max())
            b.appended = 0
        self.check_overflow(sync=False)

    def _fits(self, extra: int = 0, steps: int = 1) -> bool:
        if self.pages_bound(steps) + extra <= self.num_pages:
            return True
        self.refresh_page_bounds()
        return self.pages_bound(steps) + extra <= self.num_pages

    def free_tokens_in_layer(self, layer_id: int) -> int:
        return max(0, self.num_pages - self.pages_bound()) * PAGE_SIZE

    def _initial_bound(self, seq: Sequence) -> _PageBound:
        """Before the prefill: the decode reserve only (the prompt's pages are
        counted when the prefill has packed them)."""
        return _PageBound(0, 0, self._decode_headroom(seq))

    def can_allocate(self, seq: Sequence) -> bool:
        """Room for the sequence's decode reserve and one page per kv head of
        prompt (whether the prompt's survivors fit is known after its pack)."""
        return self.pages_bound() + self._seq_bound(self._initial_bound(seq)) + self.num_kv_heads <= self.num_pages

    def begin_prefill(self) -> None:
        """Before a prefill forward: each layer's packs may take the pages the
        registered sequences' bounds leave free (device budget), and the
        overflow flag starts clear."""
        if all(b.packed for b in self._bounds.values()):
            return
        if any(b.packed and b.appended for b in self._bounds.values()):
            self.refresh_page_bounds()  # give the prefill the pages expiry has returned
        self.page_budget.fill_(max(0, self.num_pages - self.pages_bound()))
        self.overflow.zero_()

    def stage_prefill_check(self, seq_ids: list[int]) -> None:
        """After the prefill's launches, before its host sync: queue copies of
        the overflow flag and of each packed sequence's page count (largest
        over layers) into pinned memory."""
        self._overflow_host.copy_(self.overflow, non_blocking=True)
        self._overflow_staged = True
        slots = [self.seq_states[sid].active_slot for sid in seq_ids if sid in self._bounds]
        self._prefill_check = [(sid, i) for i, sid in enumerate(sid for sid in seq_ids if sid in self._bounds)]
        if slots:
            idx = torch.tensor(slots, dtype=torch.int64).to(self.device, non_blocking=True)
            pages = self.pages_held.index_select(1, idx).sum(dim=-1).amax(dim=0).to(torch.int32)
            self._prefill_pages_host[:len(slots)].copy_(pages, non_blocking=True)

    def finish_prefill_check(self) -> None:
        """After the prefill's host sync: a pack that did not fit raises
        CompactCapacityExhausted (the caller frees the batch and retries it
        later); otherwise the packed sequences' bounds become their exact page
        counts."""
        self._overflow_staged = False
        flag = int(self._overflow_host[0])
        if flag >= 2:
            raise RuntimeError("paged compact KV: a page pop found the stack shorter than the prefill's page budget "
                               "(host page accounting failed)")
        if flag:
            self.admission_denied_count += 1
            self.overflow.zero_()
            self._prefill_check = []
            raise CompactCapacityExhausted("paged compact KV: the prefill batch's pages do not fit next to the "
                                           "running sequences' reserves")
        for sid, i in self._prefill_check:
            b = self._bounds[sid]
            b.sync_pages, b.appended, b.packed = int(self._prefill_pages_host[i]), 0, True
        self._prefill_check = []

    def bind_overflow(self, flag: torch.Tensor) -> None:
        """Keep the overflow flag in ``flag`` (int32 [1] on this device), e.g.
        beside the decode step's sampled ids so that one copy reads both back.
        Before any launch that records ``self.overflow`` (graph capture)."""
        if flag.dtype != torch.int32 or flag.numel() != 1 or flag.device != self.overflow.device:
            raise ValueError("the overflow flag must be one int32 on the pool's device")
        flag.copy_(self.overflow)
        self.overflow = flag

    def raise_if_overflow(self, flag: int) -> None:
        """check_overflow on a flag value the caller read back itself."""
        if flag:
            raise RuntimeError("paged compact KV: a page pop found the pool empty (host page accounting failed)")

    def stage_overflow_check(self) -> None:
        """Queue a copy of the device overflow flag into pinned memory (read by
        check_overflow after the caller's next host sync)."""
        self._overflow_host.copy_(self.overflow, non_blocking=True)
        self._overflow_staged = True

    def check_overflow(self, *, sync: bool = True) -> None:
        if sync or not self._overflow_staged:
            self._overflow_host.copy_(self.overflow)
        self._overflow_staged = False
        if int(self._overflow_host[0]):
            raise RuntimeError("paged compact KV: a page pop found the pool empty (host page accounting failed)")

    # -- sequences -------------------------------------------------------------
    def _reservation_tokens(self, seq: Sequence) -> int:
        # the metadata rows of a span: the whole sequence (pages, not this
        # number, bound the memory; target_live_tokens_per_seq does not apply)
        return min(self.max_model_len, seq.num_prompt_tokens + seq.max_tokens)

    def allocate(self, seq: Sequence):
        """Register a sequence before its prefill: its pages (bounded by its
        tokens plus the reserved decode appends) must fit next to the running
        sequences' bounds, else CompactCapacityExhausted."""
        existing = self.seq_states.get(seq.seq_id)
        if existing is not None:
            return existing
        bound = self._initial_bound(seq)
        need = self._seq_bound(bound) + self.num_kv_heads
        if not self._fits(need):
            self.admission_denied_count += 1
            raise CompactCapacityExhausted(
                f"paged compact KV: sequence {seq.seq_id} needs up to {need} pages per layer, "
                f"{max(0, self.num_pages - self.pages_bound())} of {self.num_pages} free")
        state = super().allocate(seq)
        slot = state.active_slot
        self.block_tables[:, slot].fill_(-1)
        self.pages_held[:, slot].zero_()
        self._bounds[seq.seq_id] = bound
        return state

    def mark_live_counts(self, seq_id: int, live_counts: torch.Tensor) -> None:
        raise NotImplementedError("paged compact KV sets live counts only through the pack and decode kernels")

    def decode_room_needed(self, seq: Sequence) -> bool:
        return False  # paged spans grow page by page on the device

    def grow_for_decode(self, seq: Sequence) -> None:
        raise NotImplementedError("paged compact KV grows spans on the device")

    def decode_pages_fit(self, steps: int = 1) -> bool:
        """True when the next ``steps`` decode appends of every sequence fit the
        pool (one sync of the page counts when the host bound says no)."""
        return self._fits(0, steps)

    def note_decode_step(self, states) -> None:
        super().note_decode_step(states)
        for st in states:
            b = self._bounds[st.seq_id]
            b.appended += 1
            b.reserve_left = max(0, b.reserve_left - 1)

    def _slot_tables(self):
        tensors, fills = super()._slot_tables()
        return tensors + (self.block_tables, self.pages_held), fills + (-1, 0)

    def free(self, seq_id: int) -> None:
        """Every page of the sequence back to its layer's stack (one launch),
        metadata rows reset, slot returned; no host sync."""
        state = self.seq_states.pop(seq_id, None)
        self._bounds.pop(seq_id, None)
        if state is None:
            return
        slot = int(state.active_slot)
        rows = torch.tensor([slot], dtype=torch.int32).to(self.device, non_blocking=True)
        bt, held, live = self.block_tables, self.pages_held, self.layer_major_live_counts
        nat.call("fdms_paged_free", rows.data_ptr(), 1, bt.data_ptr(), bt.stride(0), bt.stride(1), bt.stride(2),
                 held.data_ptr(), held.stride(0), held.stride(1), held.stride(2), live.data_ptr(), live.stride(0),
                 live.stride(1), live.stride(2), self.page_stack.data_ptr(), self.page_stack.stride(0),
                 self.page_top.data_ptr(), self.num_layers, self.num_kv_heads, nat.stream())
        self.active_slot_by_seq.pop(seq_id, None)
        self.layer_major_token_positions[:, slot].fill_(-1)
        self.layer_major_evict_mask[:, slot].zero_()
        self.free_active_slots.append(slot)
        self.free_active_slots.sort()

    # -- streaming prefill pack ---------------------------------------------------
    def streaming_pack_layer(self, *, layer_id: int, k: torch.Tensor, v: torch.Tensor, evict_mask: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, seq_ids: list[int], window_size: int,
                             cu_seqlens_host: list[int] | None = None) -> None:
        """Pack one layer's post-RoPE K/V of every prefill sequence into pages:
        the count/scan launch pops each span's pages and writes its block-table
        row, the rank-scatter launch stores the survivors (two launches, no
        host sync)."""
        nat.require_cuda(k, v, evict_mask, cu_seqlens_q, what="streaming_pack_layer")
        cu = list(cu_seqlens_host) if cu_seqlens_host is not None else [int(x) for x in cu_seqlens_q.tolist()]
        states = [self.seq_states.get(sid) for sid in seq_ids]
        H, D = k.shape[1], k.shape[2]
        if k.stride(2) != 1 or v.stride(2) != 1:
            raise ValueError("streaming pack needs a contiguous head_dim axis")
        if any(st is None for st in states):
            missing = [sid for sid, st in zip(seq_ids, states) if st is None]
            raise RuntimeError(f"sequence {missing[0]} has no compact KV allocation")
        lens = [cu[i + 1] - cu[i] for i in range(len(seq_ids))]
        if not any(n > 0 for n in lens):
            return
        for st, n in zip(states, lens):
            # live <= n: a prompt that fits its metadata rows cannot overflow them
            if n > st.max_capacity_per_lh:
                raise RuntimeError(f"streaming pack of {n} tokens exceeds metadata capacity "
                                   f"{st.max_capacity_per_lh} (layer {layer_id}, seq {st.seq_id})")
        B = len(seq_ids)
        max_chunks = max(-(-n // PACK_CHUNK) for n in lens if n > 0)
        ev = evict_mask.view(torch.uint8)
        live = torch.empty((B, H), device=self.device, dtype=torch.int32)
        offsets = torch.empty((B, H, max_chunks), device=self.device, dtype=torch.int32)
        rows = self._meta_rows(states)
        pos_l = self.layer_major_token_positions[layer_id]
        ev_l = self.layer_major_evict_mask[layer_id].view(torch.uint8)
        bt_l, held_l = self.block_tables[layer_id], self.pages_held[layer_id]
        # no metadata reset (meta_cap 0): allocate() and free() leave a slot's
        # rows at (-1, False), and a slot is packed once between them
        meta_cap = 0
        nat.call("fdms_paged_pack_prepare", ev.data_ptr(), ev.stride(0), ev.stride(1), cu_seqlens_q.data_ptr(), B,
                 int(window_size), H, max_chunks, live.data_ptr(), live.stride(0), live.stride(1),
                 offsets.data_ptr(), offsets.stride(0), offsets.stride(1), offsets.stride(2), pos_l.data_ptr(),
                 ev_l.data_ptr(), rows.data_ptr(), pos_l.stride(0), pos_l.stride(1), ev_l.stride(0), ev_l.stride(1),
                 meta_cap, self.page_stack[layer_id].data_ptr(), self.page_top[layer_id:layer_id + 1].data_ptr(),
                 self.page_budget[layer_id:layer_id + 1].data_ptr(),
                 bt_l.data_ptr(), bt_l.stride(0), bt_l.stride(1), held_l.data_ptr(), held_l.stride(0),
                 held_l.stride(1), self.max_pages, self.overflow.data_ptr(), nat.stream())
        compact_k, compact_v = self._layer_arena(layer_id)
        vec = _pack_vec(k, v, compact_k, D)
        self._calibrate_layer_scales(layer_id, k, v)
        ks, vs = self.layer_kv_scales(layer_id)
        nat.call("fdms_paged_pack_scatter", k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype), k.stride(0),
                 k.stride(1), v.stride(0), v.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1),
                 cu_seqlens_q.data_ptr(), B, offsets.data_ptr(), offsets.stride(0), offsets.stride(1),
                 offsets.stride(2), compact_k.data_ptr(), compact_v.data_ptr(), nat.dtype_code(compact_k.dtype),
                 compact_k.stride(0), pos_l.data_ptr(), ev_l.data_ptr(), rows.data_ptr(), pos_l.stride(0),
                 pos_l.stride(1), pos_l.stride(2), ev_l.stride(0), ev_l.stride(1), ev_l.stride(2), bt_l.data_ptr(),
                 bt_l.stride(0), bt_l.stride(1), int(window_size), H, D, max_chunks, vec, nat.ptr(ks), nat.ptr(vs),
                 nat.stream())
        self.layer_major_live_counts[layer_id].index_copy_(0, rows.long(), live)
        for st, n in zip(states, lens):
            if n > 0:
                st.live_upper_bound = max(st.live_upper_bound, n)

    # -- decode ------------------------------------------------------------------
    def paged_prepare_decode(self, start: int, batch: int, slot_out: torch.Tensor, plan=None,
                             positions: torch.Tensor | None = None) -> tuple:
        """Decode append rows of slots start .. start + batch - 1, all layers,
        one launch (pops a page where a span's pages are full); returns the
        (block tables [L, B, H, P], live counts [L, B, H]) views the step's
        attention reads.  With ``plan`` (layers.compact_attention.DecodePlan)
        and the step's ``positions`` (int64 [batch]) the same launch also
        writes the step's attention work plan."""
        L, H = self.num_layers, self.num_kv_heads
        live = self.layer_major_live_counts[:, start:start + batch]
        bt = self.block_tables[:, start:start + batch]
        held = self.pages_held[:, start:start + batch]
        args = (live.data_ptr(), live.stride(0), live.stride(1), live.stride(2), slot_out.data_ptr(),
                slot_out.stride(0), slot_out.stride(1), slot_out.stride(2), bt.data_ptr(), bt.stride(0),
                bt.stride(1), bt.stride(2), held.data_ptr(), held.stride(0), held.stride(1), held.stride(2),
                self.page_stack.data_ptr(), self.page_stack.stride(0), self.page_top.data_ptr(), self.max_pages,
                self.overflow.data_ptr())
        if plan is None:
            nat.call("fdms_paged_prepare_decode", *args, L, batch, H, nat.stream())
        else:
            if positions is None or positions.dtype != torch.int64 or positions.shape[0] < batch:
                raise ValueError("a planned decode step needs the step's int64 positions")
            if batch * H > plan.pairs:
                raise ValueError(f"the plan holds {plan.pairs} pairs, the batch has {batch * H}")
            rows, heavy, splits = plan.partition(batch * H)
            nat.call("fdms_paged_prepare_decode_plan", *args, positions.data_ptr(), plan.items.data_ptr(),
                     plan.items.stride(0), rows, heavy, splits, L, batch, H, nat.stream())
        return bt, live

    def prepare_decode_metadata(self, seqs: list[Sequence]):
        """Paged form of compact_kv.py:1727-1770: returns (block tables
        [L, B, H, P], live [L, B, H], slot [L, B, H], max_capacity); the batch
        must occupy contiguous slots."""
        states = [self.seq_states[s.seq_id] for s in seqs]
        start = self._contiguous_active_slot_start(states)
        if start is None:
            raise RuntimeError("paged decode needs the batch in contiguous active slots (pack_active_slots)")
        slot = torch.empty((self.num_layers, len(seqs), self.num_kv_heads), device=self.device, dtype=torch.int32)
        self.note_decode_step(states)
        bt, live = self.paged_prepare_decode(start, len(seqs), slot)
        return bt, live, slot, max(st.max_capacity_per_lh for st in states)

    def _run_expiry(self, states, current_positions, window_size: int, *, incremental: bool) -> None:
        ptr_k, ptr_v = self._layer_arena_ptrs()
        ck0, _ = self._layer_arena(0)
        esz = ck0.element_size()
        row_bytes, cs_bytes = ck0.shape[-1] * esz, ck0.stride(0) * esz
        cur = torch.tensor([int(c) for c in current_positions], dtype=torch.int64).to(self.device, non_blocking=True)
        start = self._contiguous_active_slot_start(states)
        spans = [(start, len(states), cur)] if start is not None else [
            (st.active_slot, 1, cur[i:i + 1]) for i, st in enumerate(states)]
        for s0, n, c in spans:
            pos = self.layer_major_token_positions[:, s0:]
            ev = self.layer_major_evict_mask[:, s0:].view(torch.uint8)
            live = self.layer_major_live_counts[:, s0:]
            bt, held = self.block_tables[:, s0:], self.pages_held[:, s0:]
            nat.call("fdms_paged_expiry", int(incremental), pos.data_ptr(), pos.stride(0), pos.stride(1),
                     pos.stride(2), ev.data_ptr(), ev.stride(0), ev.stride(1), ev.stride(2), live.data_ptr(),
                     live.stride(0), live.stride(1), live.stride(2), bt.data_ptr(), bt.stride(0), bt.stride(1),
                     bt.stride(2), held.data_ptr(), held.stride(0), held.stride(1), held.stride(2),
                     self.page_stack.data_ptr(), self.page_stack.stride(0), self.page_top.data_ptr(),
                     ptr_k.data_ptr(), ptr_v.data_ptr(), row_bytes, cs_bytes, c.data_ptr(), self.num_layers, n,
                     self.num_kv_heads, int(window_size), nat.stream())

    # -- inspection (tests, debugging) ------------------------------------------------
    def gather_span(self, seq_id: int, layer_id: int, head: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(K rows, V rows) [live, D] of one span in rank order (a host sync)."""
        slot = self.seq_states[seq_id].active_slot
        n = int(self.layer_major_live_counts[layer_id, slot, head])
        table = self.block_tables[layer_id, slot, head].long()
        r = torch.arange(n, device=self.device)
        rows = table[r // PAGE_SIZE] * PAGE_SIZE + r % PAGE_SIZE
        ck, cv = self._layer_arena(layer_id)
        return ck[rows], cv[rows]
