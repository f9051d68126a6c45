"""Compact-KV allocator / block manager (mirror of fastdms/engine/compact_kv.py).

Same class, methods and error behaviour as the reference's ``CompactKVManager``
(compact_kv.py:554-1795): per-(layer, sequence, kv head) flat spans carved out
of per-layer arenas by a first-fit range allocator on the host, DMS metadata
(token positions, evict flags, live counts) on the device, and the decode
expiry policy of ``apply_dms_evictions``.

What changes is where the device work runs and how often the host waits:

* streaming prefill pack: one count/scan launch and one rank-scatter launch per
  layer for the whole ragged batch, with a single device->host copy of the live
  counts per layer (the reference syncs several times per sequence per layer);
* expiry, decode-slot preparation and decision recording: one launch each for
  all layers (the reference loops layer by layer);
* arenas can be allocated up front (``preallocate=True``) so their addresses
  never change and captured decode graphs stay valid.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from .. import _native as nat
from .sequence import Sequence

PACK_CHUNK = 256  # compact_kv.py:276, 318
_TRUTHY = {"1", "true", "yes", "on"}


def _env_flag(name: str, default: str) -> bool:
    return os.environ.get(name, default).strip().lower() in _TRUTHY


def streaming_pack_cache_live_enabled() -> bool:
    """compact_kv.py:11-17 (accepted for compatibility; live counts are always
    computed once per layer here)."""
    return _env_flag("FASTDMS_STREAMING_PACK_CACHE_LIVE", "1")


def streaming_pack_triton_enabled() -> bool:
    """compact_kv.py:20-26 (the pack always runs the HIP kernels)."""
    return _env_flag("FASTDMS_STREAMING_PACK_TRITON", "1")


def streaming_pack_fused_rank_triton_enabled() -> bool:
    """compact_kv.py:29-35 (the pack always uses the fused rank kernel)."""
    return _env_flag("FASTDMS_STREAMING_PACK_FUSED_RANK_TRITON", "1")


# ---------------------------------------------------------------------------
# single-sequence pack ops with the reference's private signatures
# ---------------------------------------------------------------------------

def _streaming_pack_fused_rank_prepare(*, seq_evict: torch.Tensor, seq_len: int, window_size: int):
    """compact_kv.py:265-296 -> (live_count_per_head [H], block_offsets [H, chunks])."""
    if seq_len <= 0:
        raise ValueError("seq_len must be positive")
    if seq_evict.ndim != 2:
        raise ValueError(f"expected seq_evict [seq_len, kv_heads], got {tuple(seq_evict.shape)}")
    nat.require_cuda(seq_evict, what="streaming pack")
    num_kv_heads = seq_evict.shape[1]
    chunks = -(-seq_len // PACK_CHUNK)
    live = torch.empty((num_kv_heads,), device=seq_evict.device, dtype=torch.int32)
    offsets = torch.empty((num_kv_heads, chunks), device=seq_evict.device, dtype=torch.int32)
    nat.call("fdms_streaming_pack_prepare", seq_evict.data_ptr(), seq_evict.stride(0), seq_evict.stride(1), None,
             int(seq_len), 1, int(window_size), num_kv_heads, chunks, live.data_ptr(), 0, live.stride(0),
             offsets.data_ptr(), 0, offsets.stride(0), offsets.stride(1), None, None, None, 0, 0, 0, 0, 0,
             nat.stream())
    return live, offsets


def _pack_vec(k, v, compact_k, head_dim):
    return min(nat.vec_width(head_dim, (k, (k.stride(0), k.stride(1))), (v, (v.stride(0), v.stride(1)))),
               nat.vec_width(head_dim, (compact_k, (compact_k.stride(0),))))


def _streaming_pack_rank_scatter_hip(*, k, v, seq_evict, block_offsets, compact_k, compact_v, token_positions,
                                     evict_mask, base_offsets, start: int, seq_len: int, window_size: int,
                                     k_scale=None, v_scale=None) -> None:
    """compact_kv.py:299-361 (fused rank scatter of one sequence); optional
    per-kv-head FP8 scales [Hkv] (stored = x / scale; no reference counterpart)."""
    if seq_len <= 0:
        return
    num_kv_heads, head_dim = k.shape[1], k.shape[2]
    chunks = -(-seq_len // PACK_CHUNK)
    if block_offsets.shape != (num_kv_heads, chunks):
        raise ValueError(f"expected block_offsets {(num_kv_heads, chunks)}, got {tuple(block_offsets.shape)}")
    nat.require_cuda(k, v, seq_evict, compact_k, token_positions, what="streaming pack")
    if k.stride(2) != 1 or v.stride(2) != 1 or compact_k.stride(1) != 1:
        raise ValueError("streaming pack needs a contiguous head_dim axis")
    ev = seq_evict.view(torch.uint8)
    em = evict_mask.view(torch.uint8)
    nat.call("fdms_streaming_pack_rank_scatter", k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype), k.stride(0),
             k.stride(1), v.stride(0), v.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), None, int(start),
             int(seq_len), 1, block_offsets.data_ptr(), 0, block_offsets.stride(0), block_offsets.stride(1),
             base_offsets.data_ptr(), 0, base_offsets.stride(0), compact_k.data_ptr(), compact_v.data_ptr(),
             nat.dtype_code(compact_k.dtype), compact_k.stride(0), token_positions.data_ptr(), em.data_ptr(), None,
             0, token_positions.stride(0), token_positions.stride(1), 0, em.stride(0), em.stride(1),
             int(window_size), num_kv_heads, head_dim, chunks, _pack_vec(k, v, compact_k, head_dim),
             nat.ptr(k_scale), nat.ptr(v_scale), nat.stream())


def _streaming_pack_scatter_hip(*, k, v, keep, rank, seq_evict, compact_k, compact_v, token_positions, evict_mask,
                                base_offsets, start: int, seq_len: int, k_scale=None, v_scale=None) -> None:
    """compact_kv.py:364-423 (scatter with precomputed keep / rank)."""
    if seq_len <= 0:
        return
    num_kv_heads, head_dim = k.shape[1], k.shape[2]
    nat.require_cuda(k, v, keep, rank, seq_evict, compact_k, what="streaming pack")
    if k.stride(2) != 1 or v.stride(2) != 1 or compact_k.stride(1) != 1:
        raise ValueError("streaming pack needs a contiguous head_dim axis")
    kp = keep.view(torch.uint8)
    rk = rank.to(torch.int32)
    ev = seq_evict.view(torch.uint8)
    em = evict_mask.view(torch.uint8)
    nat.call("fdms_streaming_pack_scatter", k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype), k.stride(0),
             k.stride(1), v.stride(0), v.stride(1), kp.data_ptr(), kp.stride(0), kp.stride(1), rk.data_ptr(),
             rk.stride(0), rk.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), base_offsets.data_ptr(),
             base_offsets.stride(0), compact_k.data_ptr(), compact_v.data_ptr(), nat.dtype_code(compact_k.dtype),
             compact_k.stride(0), token_positions.data_ptr(), token_positions.stride(0), token_positions.stride(1),
             em.data_ptr(), em.stride(0), em.stride(1), int(start), int(seq_len), num_kv_heads, head_dim,
             _pack_vec(k, v, compact_k, head_dim), nat.ptr(k_scale), nat.ptr(v_scale), nat.stream())


# ---------------------------------------------------------------------------
# manager
# ---------------------------------------------------------------------------

@dataclass(slots=True)
class CompactKVMetadata:
    """compact_kv.py:487-497."""
    base_offsets: torch.Tensor
    live_counts: torch.Tensor
    token_positions: torch.Tensor | None = None

    @property
    def max_live_count(self) -> int:
        if self.live_counts.numel() == 0:
            return 0
        return int(self.live_counts.max().item())


@dataclass(slots=True)
class CompactKVSequenceState:
    """compact_kv.py:500-520."""
    seq_id: int
    base_offsets: torch.Tensor
    range_capacity: torch.Tensor
    live_counts: torch.Tensor
    token_positions: torch.Tensor
    evict_mask: torch.Tensor
    max_capacity_per_lh: int
    decode_headroom: int
    active_slot: int | None = None
    dms_initial_expiry_done: bool = False
    last_dms_expiry_position: int = -1
    # host upper bound of the live counts of every (layer, head), kept without
    # device syncs: exact after the prefill pack, +1 per appended token,
    # never below the true value (expiry only lowers it on the device)
    live_upper_bound: int = 0
    # host lower bound of min over (layer, head) of range capacity - live count
    # (free rows for decode appends): exact after the pack or a sync, -1 per
    # appended token
    decode_slack: int = 1 << 30


class CompactCapacityExhausted(RuntimeError):
    """No free range of a layer can hold a span (compact_kv.py:715-718 raises a
    plain RuntimeError here; the subclass lets the engine preempt or defer)."""


class CompactKVManager:
    """Per-(layer, sequence, kv head) compact spans (compact_kv.py:554-1795)."""

    paged = False  # flat spans; engine.paged_kv.PagedCompactKVManager stores pages

    def __init__(self, *, num_layers: int, num_kv_heads: int, capacity_tokens: int, max_model_len: int,
                 device: torch.device | str, target_live_tokens_per_seq: int | None = None,
                 head_dim: int | None = None, compact_dtype: torch.dtype | None = None,
                 per_layer_storage: bool = False, layer_major_metadata: bool = False,
                 max_active_seqs: int | None = None, preallocate: bool = False,
                 decode_reserve_tokens: int | None = None, fp8_scales: str = "unit"):
        if capacity_tokens <= 0:
            raise ValueError(f"capacity_tokens must be positive, got {capacity_tokens}")
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.capacity_tokens = capacity_tokens
        self.max_model_len = max_model_len
        self.device = torch.device(device)
        self.per_layer_storage = per_layer_storage
        # decode rows reserved per span after the pack: max_tokens (the
        # reference's sizing, compact_kv.py:830-857) or, overcommitting, at most
        # this many (spans then grow during decode, grow_for_decode)
        self.decode_reserve_tokens = decode_reserve_tokens
        self.num_span_moves = 0
        self.head_dim = head_dim
        self.compact_dtype = compact_dtype
        self.layer_major_metadata = layer_major_metadata
        self.max_active_seqs = int(max_active_seqs or 0)
        self.compact_k_per_layer: list[torch.Tensor | None] = [None] * num_layers
        self.compact_v_per_layer: list[torch.Tensor | None] = [None] * num_layers
        self.layer_major_base_offsets = None
        self.layer_major_range_capacity = None
        self.layer_major_live_counts = None
        self.layer_major_token_positions = None
        self.layer_major_evict_mask = None
        self.active_slot_by_seq: dict[int, int] = {}
        self.free_active_slots: list[int] = []
        if self.layer_major_metadata:
            if self.max_active_seqs <= 0:
                raise ValueError("layer-major metadata requires max_active_seqs > 0")
            shape = (num_layers, self.max_active_seqs, num_kv_heads)
            self.layer_major_base_offsets = torch.full(shape, -1, device=self.device, dtype=torch.int32)
            self.layer_major_range_capacity = torch.zeros(shape, device=self.device, dtype=torch.int32)
            self.layer_major_live_counts = torch.zeros(shape, device=self.device, dtype=torch.int32)
            self.layer_major_token_positions = torch.full(shape + (int(max_model_len),), -1, device=self.device,
                                                          dtype=torch.int32)
            self.layer_major_evict_mask = torch.zeros(shape + (int(max_model_len),), device=self.device,
                                                      dtype=torch.bool)
            self.free_active_slots = list(range(self.max_active_seqs))
        self._attn_modules: list = []
        self.target_live_tokens_per_seq = target_live_tokens_per_seq
        self.free_ranges_per_layer: list[list[tuple[int, int]]] = [[(0, capacity_tokens)] for _ in range(num_layers)]
        self.seq_states: dict[int, CompactKVSequenceState] = {}
        self.admission_denied_count = 0
        self.debug_checks = os.environ.get("FASTDMS_COMPACT_DEBUG_CHECKS") == "1"
        self.compact_k: torch.Tensor | None = None
        self.compact_v: torch.Tensor | None = None
        self._layer_ptrs: tuple[torch.Tensor, torch.Tensor] | None = None
        self.storage_version = 0
        # Per-(layer, kv head) FP8 scales (no reference counterpart; the
        # reference stores with a bare cast, i.e. scale 1): kv_scales[l, 0] for
        # K and [l, 1] for V, stored = x / scale, dequantised in the attention
        # kernels.  "unit": no tables (the reference's numerics); "calibrate":
        # each layer's scales are set at its first prefill pack from the prompt's
        # post-RoPE K / V (amax / 224, i.e. twice the range seen), then frozen.
        if fp8_scales not in ("unit", "calibrate"):
            raise ValueError(f"fp8_scales must be 'unit' or 'calibrate', got {fp8_scales!r}")
        self.fp8_scales = fp8_scales
        self.kv_scales: torch.Tensor | None = None
        self._scales_calibrated = [False] * num_layers
        if fp8_scales != "unit":
            if compact_dtype != getattr(torch, "float8_e4m3fn", None):
                raise ValueError("per-head KV scales need FP8 compact storage")
            self.kv_scales = torch.ones((num_layers, 2, num_kv_heads), device=self.device, dtype=torch.float32)
        if preallocate and per_layer_storage:
            for layer_id in range(num_layers):
                self._ensure_layer_storage(layer_id, capacity_tokens)

    # -- storage ------------------------------------------------------------
    def attach_compact_storage(self, compact_kv_cache: torch.Tensor) -> None:
        """compact_kv.py:650-653: [2, num_layers, capacity, head_dim] arena."""
        self.compact_k = compact_kv_cache[0]
        self.compact_v = compact_kv_cache[1]
        self._layer_ptrs = None
        self.storage_version += 1

    def attach_attention_modules(self, attn_modules: list) -> None:
        self._attn_modules = attn_modules
        for layer_id, module in enumerate(attn_modules):
            if self.compact_k_per_layer[layer_id] is not None:
                module.compact_k_cache = self.compact_k_per_layer[layer_id]
                module.compact_v_cache = self.compact_v_per_layer[layer_id]
            module.compact_k_scale, module.compact_v_scale = self.layer_kv_scales(layer_id)

    def layer_kv_scales(self, layer_id: int) -> tuple[torch.Tensor | None, torch.Tensor | None]:
        """(K scales, V scales) [Hkv] of a layer, or (None, None) without tables."""
        if self.kv_scales is None:
            return None, None
        return self.kv_scales[layer_id, 0], self.kv_scales[layer_id, 1]

    def set_kv_scales(self, scales: torch.Tensor) -> None:
        """Set every layer's FP8 scales ([num_layers, 2, num_kv_heads], > 0)
        before any sequence is packed; the tables keep their storage, so captured
        graphs stay valid."""
        if self.kv_scales is None:
            raise RuntimeError("the manager was built without KV scale tables (fp8_scales='unit')")
        if self.seq_states:
            raise RuntimeError("KV scales must be set before any sequence is packed")
        if tuple(scales.shape) != tuple(self.kv_scales.shape):
            raise ValueError(f"expected scales {tuple(self.kv_scales.shape)}, got {tuple(scales.shape)}")
        self.kv_scales.copy_(scales.to(device=self.device, dtype=torch.float32))
        self._scales_calibrated = [True] * self.num_layers

    def _calibrate_layer_scales(self, layer_id: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """First pack of a layer in "calibrate" mode: scale = amax / 224 per
        kv head (on the device, no host sync); an all-zero head keeps 1."""
        if self.fp8_scales != "calibrate" or self._scales_calibrated[layer_id]:
            return
        for i, x in enumerate((k, v)):
            amax = x.detach().abs().amax(dim=(0, 2)).float()
            self.kv_scales[layer_id, i].copy_(torch.where(amax > 0, amax / 224.0, torch.ones_like(amax)))
        self._scales_calibrated[layer_id] = True

    def _ensure_layer_storage(self, layer_id: int, min_tokens: int):
        """compact_kv.py:661-695: grow to a 256-token multiple, keep old rows."""
        existing_k = self.compact_k_per_layer[layer_id]
        if existing_k is not None and existing_k.shape[0] >= min_tokens:
            return existing_k, self.compact_v_per_layer[layer_id]
        if self.head_dim is None or self.compact_dtype is None:
            raise RuntimeError("per-layer storage requires head_dim and compact_dtype set on manager")
        new_size = max(256, ((min_tokens + 255) // 256) * 256)
        with torch.inference_mode(False):
            new_k = torch.empty(new_size, self.head_dim, device=self.device, dtype=self.compact_dtype)
            new_v = torch.empty(new_size, self.head_dim, device=self.device, dtype=self.compact_dtype)
            if existing_k is not None:
                n = existing_k.shape[0]
                new_k[:n].copy_(existing_k)
                new_v[:n].copy_(self.compact_v_per_layer[layer_id])
        self.compact_k_per_layer[layer_id] = new_k
        self.compact_v_per_layer[layer_id] = new_v
        if self._attn_modules and layer_id < len(self._attn_modules):
            self._attn_modules[layer_id].compact_k_cache = new_k
            self._attn_modules[layer_id].compact_v_cache = new_v
        self._layer_ptrs = None
        self.storage_version += 1
        return new_k, new_v

    def _layer_arena_ptrs(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Device tables of per-layer arena base addresses (for one-launch
        all-layer kernels)."""
        if self._layer_ptrs is None:
            if self.per_layer_storage:
                ks = [0 if t is None else t.data_ptr() for t in self.compact_k_per_layer]
                vs = [0 if t is None else t.data_ptr() for t in self.compact_v_per_layer]
            else:
                if self.compact_k is None:
                    raise RuntimeError("CompactKVManager.attach_compact_storage was not called")
                ks = [self.compact_k[l].data_ptr() for l in range(self.num_layers)]
                vs = [self.compact_v[l].data_ptr() for l in range(self.num_layers)]
            self._layer_ptrs = (torch.tensor(ks, dtype=torch.int64, device=self.device),
                                torch.tensor(vs, dtype=torch.int64, device=self.device))
        return self._layer_ptrs

    def _layer_arena(self, layer_id: int) -> tuple[torch.Tensor, torch.Tensor]:
        if self.per_layer_storage:
            return self.compact_k_per_layer[layer_id], self.compact_v_per_layer[layer_id]
        if self.compact_k is None or self.compact_v is None:
            raise RuntimeError("CompactKVManager.attach_compact_storage was not called")
        return self.compact_k[layer_id], self.compact_v[layer_id]

    # -- allocator (compact_kv.py:697-857) ----------------------------------
    def free_tokens_in_layer(self, layer_id: int) -> int:
        return sum(length for _, length in self.free_ranges_per_layer[layer_id])

    @property
    def free_tokens(self) -> int:
        return sum(self.free_tokens_in_layer(l) for l in range(self.num_layers))

    def _alloc_range(self, layer_id: int, length: int) -> int:
        free = self.free_ranges_per_layer[layer_id]
        for idx, (start, available) in enumerate(free):
            if available < length:
                continue
            if available == length:
                free.pop(idx)
            else:
                free[idx] = (start + length, available - length)
            return start
        raise CompactCapacityExhausted(f"compact KV capacity exhausted in layer {layer_id}: requested {length}, "
                                       f"free {self.free_tokens_in_layer(layer_id)}")

    def _free_range(self, layer_id: int, start: int, length: int) -> None:
        if length <= 0:
            return
        free = self.free_ranges_per_layer[layer_id]
        free.append((start, length))
        free.sort()
        merged: list[tuple[int, int]] = []
        for range_start, range_len in free:
            if merged and range_start <= merged[-1][0] + merged[-1][1]:
                prev_start, prev_len = merged[-1]
                merged[-1] = (prev_start, max(prev_start + prev_len, range_start + range_len) - prev_start)
            else:
                merged.append((range_start, range_len))
        self.free_ranges_per_layer[layer_id] = merged

    def can_allocate(self, seq: Sequence) -> bool:
        needed = self._reservation_tokens(seq) * self.num_kv_heads
        return all(self.free_tokens_in_layer(l) >= needed for l in range(self.num_layers))

    def _reservation_tokens(self, seq: Sequence) -> int:
        worst_case = min(self.max_model_len, seq.num_prompt_tokens + seq.max_tokens)
        if self.target_live_tokens_per_seq is not None:
            return min(worst_case, max(1, int(self.target_live_tokens_per_seq)))
        return worst_case

    def allocate(self, seq: Sequence) -> CompactKVSequenceState:
        """compact_kv.py:753-828: register a sequence; ranges come per layer at pack time."""
        existing = self.seq_states.get(seq.seq_id)
        if existing is not None:
            return existing
        cap = self._reservation_tokens(seq)
        if cap <= 0:
            raise ValueError(f"invalid reservation {cap} for seq {seq.seq_id}")
        active_slot = None
        L, H = self.num_layers, self.num_kv_heads
        if self.layer_major_metadata:
            if not self.free_active_slots:
                raise RuntimeError(f"compact KV active-slot capacity exhausted: max_active_seqs={self.max_active_seqs}")
            active_slot = self.free_active_slots.pop(0)
            self.active_slot_by_seq[seq.seq_id] = active_slot
            base = self.layer_major_base_offsets[:, active_slot, :]
            rcap = self.layer_major_range_capacity[:, active_slot, :]
            live = self.layer_major_live_counts[:, active_slot, :]
            pos = self.layer_major_token_positions[:, active_slot, :, :cap]
            ev = self.layer_major_evict_mask[:, active_slot, :, :cap]
            base.fill_(-1)
            rcap.zero_()
            live.zero_()
            pos.fill_(-1)
            ev.zero_()
        else:
            base = torch.full((L, H), -1, device=self.device, dtype=torch.int32)
            rcap = torch.zeros((L, H), device=self.device, dtype=torch.int32)
            live = torch.zeros((L, H), device=self.device, dtype=torch.int32)
            pos = torch.full((L, H, cap), -1, device=self.device, dtype=torch.int32)
            ev = torch.zeros((L, H, cap), device=self.device, dtype=torch.bool)
        state = CompactKVSequenceState(seq_id=seq.seq_id, base_offsets=base, range_capacity=rcap, live_counts=live,
                                       token_positions=pos, evict_mask=ev, active_slot=active_slot,
                                       max_capacity_per_lh=cap, decode_headroom=self._decode_headroom(seq))
        self.seq_states[seq.seq_id] = state
        return state

    def _decode_headroom(self, seq: Sequence) -> int:
        if self.decode_reserve_tokens is None:
            return int(seq.max_tokens)
        return max(1, min(int(seq.max_tokens), int(self.decode_reserve_tokens)))

    def _layer_range_sizes(self, state: CompactKVSequenceState, live_per_head: list[int]) -> list[int]:
        return [max(min(int(x) + int(state.decode_headroom), state.max_capacity_per_lh), 1) for x in live_per_head]

    def _alloc_layer_ranges_host(self, state, layer_id: int, live_per_head: list[int]) -> tuple[list, list]:
        """First-fit head by head; roll back this call's heads on failure (compact_kv.py:830-852)."""
        sizes = self._layer_range_sizes(state, live_per_head)
        bases: list[int] = []
        try:
            for size in sizes:
                bases.append(self._alloc_range(layer_id, size))
        except Exception:
            for h2, base2 in enumerate(bases):
                self._free_range(layer_id, base2, sizes[h2])
            raise
        return bases, sizes

    def _allocate_layer_ranges_for_seq(self, state, layer_id: int, live_count_per_head) -> torch.Tensor:
        """compact_kv.py:830-857."""
        live_cpu = live_count_per_head.tolist() if torch.is_tensor(live_count_per_head) else list(live_count_per_head)
        bases, sizes = self._alloc_layer_ranges_host(state, layer_id, live_cpu)
        bases_t = torch.tensor(bases, device=self.device, dtype=torch.int32)
        state.base_offsets[layer_id].copy_(bases_t)
        state.range_capacity[layer_id].copy_(torch.tensor(sizes, device=self.device, dtype=torch.int32))
        return bases_t

    def mark_all_heads_live(self, seq_id: int, live_count: int) -> None:
        self.mark_live_counts(seq_id, torch.full((self.num_layers, self.num_kv_heads), live_count,
                                                 device=self.device, dtype=torch.int32))

    def mark_live_counts(self, seq_id: int, live_counts: torch.Tensor) -> None:
        """compact_kv.py:868-882."""
        state = self.seq_states[seq_id]
        if live_counts.shape != (self.num_layers, self.num_kv_heads):
            raise ValueError(f"expected live_counts {(self.num_layers, self.num_kv_heads)}, "
                             f"got {tuple(live_counts.shape)}")
        live_counts = live_counts.to(device=self.device, dtype=torch.int32)
        if bool(torch.any(live_counts > state.range_capacity).item()):
            raise RuntimeError(f"compact KV live count {int(live_counts.max().item())} exceeds per-(layer,head) "
                               "range capacity")
        state.live_counts.copy_(live_counts)
        state.live_upper_bound = int(live_counts.max().item())

    # -- streaming prefill pack (compact_kv.py:915-1099) --------------------
    def streaming_pack_layer(self, *, layer_id: int, k: torch.Tensor, v: torch.Tensor, evict_mask: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, seq_ids: list[int], window_size: int,
                             cu_seqlens_host: list[int] | None = None) -> None:
        """Pack one layer's post-RoPE K/V of every prefill sequence into its spans.

        k, v: [T_total, Hkv, D]; evict_mask: bool [T_total, Hkv]; cu_seqlens_q
        int32 [B+1] on the device (``cu_seqlens_host`` is the same on the host,
        saving a sync when the caller has it).
        """
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
        batch_idx = [i for i, n in enumerate(lens) if n > 0]
        if not batch_idx:
            return
        B = len(seq_ids)
        max_chunks = max(-(-n // PACK_CHUNK) for n in lens if n > 0)
        ev = evict_mask.view(torch.uint8)
        live = torch.empty((B, H), device=self.device, dtype=torch.int32)
        offsets = torch.empty((B, H, max_chunks), device=self.device, dtype=torch.int32)
        rows = self._meta_rows(states)
        if rows is not None:
            pos_l = self.layer_major_token_positions[layer_id]
            ev_l = self.layer_major_evict_mask[layer_id].view(torch.uint8)
            meta_cap = max(st.max_capacity_per_lh for st in states)
            nat.call("fdms_streaming_pack_prepare", ev.data_ptr(), ev.stride(0), ev.stride(1), cu_seqlens_q.data_ptr(),
                     0, B, int(window_size), H, max_chunks, live.data_ptr(), live.stride(0), live.stride(1),
                     offsets.data_ptr(), offsets.stride(0), offsets.stride(1), offsets.stride(2), pos_l.data_ptr(),
                     ev_l.data_ptr(), rows.data_ptr(), pos_l.stride(0), pos_l.stride(1), ev_l.stride(0),
                     ev_l.stride(1), meta_cap, nat.stream())
        else:
            nat.call("fdms_streaming_pack_prepare", ev.data_ptr(), ev.stride(0), ev.stride(1), cu_seqlens_q.data_ptr(),
                     0, B, int(window_size), H, max_chunks, live.data_ptr(), live.stride(0), live.stride(1),
                     offsets.data_ptr(), offsets.stride(0), offsets.stride(1), offsets.stride(2), None, None, None,
                     0, 0, 0, 0, 0, nat.stream())
            for st, n in zip(states, lens):
                if n > 0:
                    st.token_positions[layer_id].fill_(-1)
                    st.evict_mask[layer_id].fill_(False)
        live_host = live.tolist()  # the one host sync of this layer
        # a span holds at most max_capacity_per_lh rows: a larger live count
        # would scatter past it (compact_kv.py:1018-1023), so fail before any
        # range of this layer is allocated
        for i, st in enumerate(states):
            if lens[i] > 0 and max(live_host[i]) > st.max_capacity_per_lh:
                raise RuntimeError(f"streaming pack live count {max(live_host[i])} exceeds metadata capacity "
                                   f"{st.max_capacity_per_lh} (layer {layer_id}, seq {st.seq_id})")
        # host first-fit allocation, all sequences of the batch (reference order)
        all_bases, all_sizes = [], []
        high_water = 0
        try:
            for i, st in enumerate(states):
                if lens[i] > 0:
                    bases, sizes = self._alloc_layer_ranges_host(st, layer_id, live_host[i])
                else:
                    bases, sizes = [-1] * H, [0] * H
                all_bases.append(bases)
                all_sizes.append(sizes)
                high_water = max(high_water, max(b + s for b, s in zip(bases, sizes)))
        except CompactCapacityExhausted:
            # this layer's ranges of the earlier sequences are not recorded in
            # their states yet: give them back before the caller frees the rest
            for bases, sizes in zip(all_bases, all_sizes):
                for b, n in zip(bases, sizes):
                    if b >= 0 and n > 0:
                        self._free_range(layer_id, b, n)
            raise
        if self.per_layer_storage:
            self._ensure_layer_storage(layer_id, high_water)
        compact_k, compact_v = self._layer_arena(layer_id)
        bases_t = torch.tensor(all_bases, dtype=torch.int32).to(self.device, non_blocking=True)
        sizes_t = torch.tensor(all_sizes, dtype=torch.int32).to(self.device, non_blocking=True)
        if rows is not None:
            rows_l = rows.long()
            self.layer_major_base_offsets[layer_id].index_copy_(0, rows_l, bases_t)
            self.layer_major_range_capacity[layer_id].index_copy_(0, rows_l, sizes_t)
        else:
            for i, st in enumerate(states):
                st.base_offsets[layer_id].copy_(bases_t[i])
                st.range_capacity[layer_id].copy_(sizes_t[i])
        vec = _pack_vec(k, v, compact_k, D)
        self._calibrate_layer_scales(layer_id, k, v)
        ks, vs = self.layer_kv_scales(layer_id)
        if rows is not None:
            pos_l = self.layer_major_token_positions[layer_id]
            ev_l = self.layer_major_evict_mask[layer_id].view(torch.uint8)
            nat.call("fdms_streaming_pack_rank_scatter", k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype),
                     k.stride(0), k.stride(1), v.stride(0), v.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1),
                     cu_seqlens_q.data_ptr(), 0, 0, B, offsets.data_ptr(), offsets.stride(0), offsets.stride(1),
                     offsets.stride(2), bases_t.data_ptr(), bases_t.stride(0), bases_t.stride(1),
                     compact_k.data_ptr(), compact_v.data_ptr(), nat.dtype_code(compact_k.dtype),
                     compact_k.stride(0), pos_l.data_ptr(), ev_l.data_ptr(), rows.data_ptr(), pos_l.stride(0),
                     pos_l.stride(1), pos_l.stride(2), ev_l.stride(0), ev_l.stride(1), ev_l.stride(2),
                     int(window_size), H, D, max_chunks, vec, nat.ptr(ks), nat.ptr(vs), nat.stream())
            self.layer_major_live_counts[layer_id].index_copy_(0, rows_l, live)
        else:
            for i, st in enumerate(states):
                if lens[i] <= 0:
                    continue
                pos = st.token_positions[layer_id]
                em = st.evict_mask[layer_id].view(torch.uint8)
                nat.call("fdms_streaming_pack_rank_scatter", k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype),
                         k.stride(0), k.stride(1), v.stride(0), v.stride(1), ev[cu[i]:].data_ptr(), ev.stride(0),
                         ev.stride(1), None, cu[i], lens[i], 1, offsets[i].data_ptr(), 0, offsets.stride(1),
                         offsets.stride(2), bases_t[i].data_ptr(), 0, 1, compact_k.data_ptr(), compact_v.data_ptr(),
                         nat.dtype_code(compact_k.dtype), compact_k.stride(0), pos.data_ptr(), em.data_ptr(), None,
                         0, pos.stride(0), pos.stride(1), 0, em.stride(0), em.stride(1), int(window_size), H, D,
                         -(-lens[i] // PACK_CHUNK), vec, nat.ptr(ks), nat.ptr(vs), nat.stream())
                st.live_counts[layer_id].copy_(live[i])
        for i, st in enumerate(states):
            if lens[i] > 0:
                st.live_upper_bound = max(st.live_upper_bound, max(live_host[i]))
                st.decode_slack = min(st.decode_slack, min(sz - lv for sz, lv in zip(all_sizes[i], live_host[i])))

    def _meta_rows(self, states) -> torch.Tensor | None:
        if not self.layer_major_metadata:
            return None
        return torch.tensor([st.active_slot for st in states], dtype=torch.int32).to(self.device, non_blocking=True)

    # -- decode growth of overcommitted spans (a build extension) ----------------
    def decode_room_needed(self, seq: Sequence) -> bool:
        """True when some (layer, head) span of ``seq`` has no free row for the
        next decode append.  Host-only while the slack bound allows; otherwise
        one small device->host copy of the sequence's live counts refreshes the
        bounds (expiry may have freed rows)."""
        st = self.seq_states[seq.seq_id]
        if st.decode_slack >= 1:
            return False
        live = st.live_counts.cpu()
        cap = st.range_capacity.cpu()
        st.decode_slack = int((cap - live).min())
        st.live_upper_bound = int(live.max())
        return st.decode_slack < 1

    def grow_for_decode(self, seq: Sequence) -> None:
        """Move every full (layer, head) span of ``seq`` to a new range of
        live + the decode reserve rows (first fit), copying its K / V rows; the
        rank-indexed positions / evict metadata do not move.  Raises
        CompactCapacityExhausted when a layer has no such range (spans moved
        before that stay valid)."""
        st = self.seq_states[seq.seq_id]
        live = st.live_counts.cpu().tolist()
        cap = st.range_capacity.cpu().tolist()
        base = st.base_offsets.cpu().tolist()
        try:
            for layer_id in range(self.num_layers):
                ck, cv = self._layer_arena(layer_id)
                for h in range(self.num_kv_heads):
                    n, old_base, old_size = int(live[layer_id][h]), int(base[layer_id][h]), int(cap[layer_id][h])
                    if old_size - n >= 1:
                        continue
                    new_size = min(n + max(int(st.decode_headroom), 1), st.max_capacity_per_lh)
                    if new_size <= old_size:
                        raise RuntimeError(f"sequence {seq.seq_id} reached its metadata capacity "
                                           f"{st.max_capacity_per_lh} in layer {layer_id}")
                    new_base = self._alloc_range(layer_id, new_size)
                    if n:
                        ck[new_base:new_base + n].copy_(ck[old_base:old_base + n])
                        cv[new_base:new_base + n].copy_(cv[old_base:old_base + n])
                    self._free_range(layer_id, old_base, old_size)
                    self.num_span_moves += 1
                    st.base_offsets[layer_id, h] = new_base
                    st.range_capacity[layer_id, h] = new_size
                    base[layer_id][h], cap[layer_id][h] = new_base, new_size
        finally:
            st.decode_slack = min(int(c) - int(v) for cr, lr in zip(cap, live) for c, v in zip(cr, lr))

    def _bind_slot_views(self, state: CompactKVSequenceState, slot: int) -> None:
        cap = state.max_capacity_per_lh
        state.active_slot = slot
        state.base_offsets = self.layer_major_base_offsets[:, slot, :]
        state.range_capacity = self.layer_major_range_capacity[:, slot, :]
        state.live_counts = self.layer_major_live_counts[:, slot, :]
        state.token_positions = self.layer_major_token_positions[:, slot, :, :cap]
        state.evict_mask = self.layer_major_evict_mask[:, slot, :, :cap]

    def pack_active_slots(self, states) -> None:
        """Move the layer-major metadata rows of ``states`` (every active
        sequence, in decode order) to slots 0 .. len-1 in that order, so one
        decode launch covers them.  Sequences that finish or are preempted leave
        holes; the reference then processes the batch sequence by sequence
        (compact_kv.py:1162-1172), this build moves the rows (5 small device
        copies per moved sequence) and keeps one launch.  Spans, arenas and the
        allocator are untouched."""
        if not self.layer_major_metadata:
            return
        if len(states) != len(self.active_slot_by_seq):
            raise RuntimeError("slot packing needs every active sequence in the batch")
        tensors, fills = self._slot_tables()
        target = {st.seq_id: i for i, st in enumerate(states)}
        moving = [st for st in states if st.active_slot != target[st.seq_id]]
        if not moving:
            return
        # rows of the moving sequences are copied out first, so cycles need no
        # staging slot; vacated slots that nobody moves into are reset
        saved = {st.seq_id: [t[:, st.active_slot].clone() for t in tensors] for st in moving}
        vacated = {st.active_slot for st in moving} - {target[st.seq_id] for st in moving}
        for st in moving:
            new = target[st.seq_id]
            for t, rows in zip(tensors, saved[st.seq_id]):
                t[:, new].copy_(rows)
            self._bind_slot_views(st, new)
            self.active_slot_by_seq[st.seq_id] = new
        for slot in vacated:
            for t, f in zip(tensors, fills):
                t[:, slot].fill_(f)
        used = set(self.active_slot_by_seq.values())
        self.free_active_slots = [i for i in range(self.max_active_seqs) if i not in used]

    def _slot_tables(self) -> tuple[tuple, tuple]:
        """The layer-major tables indexed [layer, slot, ...] and the value of
        an empty slot in each (what pack_active_slots moves)."""
        return ((self.layer_major_base_offsets, self.layer_major_range_capacity, self.layer_major_live_counts,
                 self.layer_major_token_positions, self.layer_major_evict_mask), (-1, 0, 0, -1, False))

    def note_decode_step(self, states) -> None:
        """Host bookkeeping of one decode append per sequence (no device work):
        the live-count upper bound grows by one, the free-row bound shrinks."""
        for st in states:
            st.live_upper_bound += 1
            st.decode_slack -= 1

    def _contiguous_active_slot_start(self, states) -> int | None:
        """compact_kv.py:1162-1172."""
        if not self.layer_major_metadata or not states:
            return None
        slots = [state.active_slot for state in states]
        if any(slot is None for slot in slots):
            return None
        start = int(slots[0])
        if [int(s) for s in slots] != list(range(start, start + len(slots))):
            return None
        return start

    # -- decode expiry (compact_kv.py:1174-1560) ----------------------------
    def expiry_action(self, seqs: list[Sequence], current_positions: list[int], window_size: int) -> str:
        """The branch apply_dms_evictions takes this step: 'exact' (full
        re-compaction), 'full', 'incremental' or 'skip' (compact_kv.py:1189-1241)."""
        triton_mode = os.environ.get("FASTDMS_DMS_EXPIRY_TRITON", "auto").strip().lower()
        n = len(seqs)
        auto_windowed = triton_mode in {"", "auto"} and (n == 1 or n >= 4)
        use_fast = self.per_layer_storage and n > 0 and (triton_mode in _TRUTHY or auto_windowed)
        if use_fast:
            states = [self.seq_states.get(seq.seq_id) for seq in seqs]
            if any(s is None for s in states):
                missing = [seq.seq_id for seq, s in zip(seqs, states) if s is None]
                raise RuntimeError(f"sequence(s) {missing} have no compact KV allocation")
            sequential = all(s.dms_initial_expiry_done and int(c) == s.last_dms_expiry_position + 1
                             for s, c in zip(states, current_positions))
            if sequential:
                interval_env = os.environ.get("FASTDMS_DMS_EXPIRY_INTERVAL")
                interval = int(interval_env) if interval_env is not None else (
                    max(1, int(window_size)) if auto_windowed else 1)
                if interval > 1:
                    if not any(int(c) % interval == 0 for c in current_positions):
                        return "skip"
                    return "full"
                return "incremental"
        return "exact"

    def apply_dms_evictions(self, seqs: list[Sequence], current_positions: list[int], *, window_size: int,
                            compact_k: torch.Tensor | None = None, compact_v: torch.Tensor | None = None,
                            sync_stats: bool = True) -> dict:
        if len(seqs) != len(current_positions):
            raise ValueError("seq/current_positions length mismatch")
        if not seqs:
            return {"evicted_tokens": 0, "live_tokens_before_min": 0, "live_tokens_before_max": 0,
                    "live_tokens_after_min": 0, "live_tokens_after_max": 0}
        action = self.expiry_action(seqs, current_positions, window_size)
        states = []
        for seq in seqs:
            st = self.seq_states.get(seq.seq_id)
            if st is None:
                raise RuntimeError(f"sequence {seq.seq_id} has no compact KV allocation")
            states.append(st)
        if compact_k is not None or compact_v is not None:
            if self.per_layer_storage:
                raise ValueError("explicit compact_k/compact_v apply only to single-tensor storage")
            self.compact_k, self.compact_v = compact_k, compact_v
            self._layer_ptrs = None
        if action == "skip" and not sync_stats:
            # compact_kv.py:1363-1379: a skipped step without synced stats touches no device memory
            for st, cur in zip(states, current_positions):
                st.last_dms_expiry_position = int(cur)
            return {"evicted_tokens": 0, "live_tokens_before_min": 0, "live_tokens_before_max": 0,
                    "live_tokens_after_min": 0, "live_tokens_after_max": 0}
        live_before = self._stack_live(states)
        if action != "skip":
            self._run_expiry(states, current_positions, window_size, incremental=(action == "incremental"))
        for st, cur in zip(states, current_positions):
            if action in ("exact", "full"):
                st.dms_initial_expiry_done = True
            st.last_dms_expiry_position = int(cur)
        if action == "skip":
            live_after = live_before
            zero = torch.zeros((), device=self.device, dtype=torch.int64)
            evicted = zero
        else:
            live_after = self._stack_live(states)
            evicted = (live_before - live_after).sum()
        stats = {"evicted_tokens": evicted, "live_tokens_before_min": live_before.min(),
                 "live_tokens_before_max": live_before.max(), "live_tokens_after_min": live_after.min(),
                 "live_tokens_after_max": live_after.max()}
        if sync_stats:
            return {key: int(value.item()) for key, value in stats.items()}
        return stats

    def _stack_live(self, states) -> torch.Tensor:
        start = self._contiguous_active_slot_start(states)
        if start is not None:
            return self.layer_major_live_counts[:, start:start + len(states), :].to(torch.int64).clone()
        return torch.stack([s.live_counts for s in states], dim=0).to(torch.int64)

    def _run_expiry(self, states, current_positions, window_size: int, *, incremental: bool) -> None:
        if any(self._layer_arena(l)[0] is None for l in range(self.num_layers)):
            raise RuntimeError("expiry before every layer's compact storage exists")
        ptr_k, ptr_v = self._layer_arena_ptrs()
        ck0, _ = self._layer_arena(0)
        esz = ck0.element_size()
        row_bytes, cs_bytes = ck0.shape[-1] * esz, ck0.stride(0) * esz
        cur = torch.tensor([int(c) for c in current_positions], dtype=torch.int64).to(self.device, non_blocking=True)
        start = self._contiguous_active_slot_start(states)
        if start is not None:
            pos = self.layer_major_token_positions[:, start:]
            ev = self.layer_major_evict_mask[:, start:].view(torch.uint8)
            live = self.layer_major_live_counts[:, start:]
            base = self.layer_major_base_offsets[:, start:]
            self._launch_expiry(incremental, pos, ev, live, base, ptr_k, ptr_v, row_bytes, cs_bytes, cur,
                                len(states), window_size, per_seq=False)
            return
        for i, st in enumerate(states):
            self._launch_expiry(incremental, st.token_positions, st.evict_mask.view(torch.uint8), st.live_counts,
                                st.base_offsets, ptr_k, ptr_v, row_bytes, cs_bytes, cur[i:i + 1], 1, window_size,
                                per_seq=True)

    def _launch_expiry(self, incremental, pos, ev, live, base, ptr_k, ptr_v, row_bytes, cs_bytes, cur, num_seqs,
                       window_size, *, per_seq: bool) -> None:
        if per_seq:  # [L, H, C] views of one sequence
            ps = (pos.stride(0), 0, pos.stride(1))
            es = (ev.stride(0), 0, ev.stride(1))
            ls = (live.stride(0), 0, live.stride(1))
            bs = (base.stride(0), 0, base.stride(1))
        else:        # [L, S, H, C] layer-major views
            ps = (pos.stride(0), pos.stride(1), pos.stride(2))
            es = (ev.stride(0), ev.stride(1), ev.stride(2))
            ls = (live.stride(0), live.stride(1), live.stride(2))
            bs = (base.stride(0), base.stride(1), base.stride(2))
        nat.call("fdms_dms_expiry", int(incremental), pos.data_ptr(), *ps, ev.data_ptr(), *es, live.data_ptr(), *ls,
                 base.data_ptr(), *bs, None, None, ptr_k.data_ptr(), ptr_v.data_ptr(), row_bytes, cs_bytes,
                 cur.data_ptr(), self.num_layers, num_seqs, self.num_kv_heads, int(window_size), nat.stream())

    # -- decode metadata / recording (compact_kv.py:1562-1770) --------------
    def record_appended_dms_decisions(self, seqs: list[Sequence], current_positions, layer_evictions, *,
                                      sync_stats: bool = True) -> dict:
        if len(seqs) != len(current_positions):
            raise ValueError("seq/current_positions length mismatch")
        batch = len(seqs)
        if batch == 0:
            return {"eviction_decisions_true": 0, "eviction_decisions_total": 0}
        expected = (self.num_layers, batch, self.num_kv_heads)
        if isinstance(layer_evictions, torch.Tensor):
            if tuple(layer_evictions.shape) != expected:
                raise RuntimeError(f"expected DMS decode decisions {expected}, got {tuple(layer_evictions.shape)}")
            evict_all = layer_evictions
            if evict_all.device != self.device or evict_all.dtype != torch.bool:
                evict_all = evict_all.to(device=self.device, dtype=torch.bool)
        else:
            layers = []
            for layer_id in range(self.num_layers):
                e = layer_evictions.get(layer_id)
                if e is None:
                    raise RuntimeError(f"missing DMS decode eviction decisions for layer {layer_id}")
                if tuple(e.shape) != (batch, self.num_kv_heads):
                    raise RuntimeError(f"expected DMS decode decisions {(batch, self.num_kv_heads)}, "
                                       f"got {tuple(e.shape)}")
                layers.append(e)
            evict_all = torch.stack(layers, dim=0).to(device=self.device, dtype=torch.bool)
        if isinstance(current_positions, torch.Tensor):
            if current_positions.numel() != batch:
                raise ValueError("current_positions tensor length mismatch")
            pos_t = current_positions.to(device=self.device)
            if pos_t.dtype not in (torch.int32, torch.int64):
                pos_t = pos_t.to(torch.int32)
            pos_t = pos_t.contiguous()
        else:
            pos_t = torch.tensor(list(current_positions), dtype=torch.int32).to(self.device, non_blocking=True)
        states = []
        for seq in seqs:
            st = self.seq_states.get(seq.seq_id)
            if st is None:
                raise RuntimeError(f"sequence {seq.seq_id} has no compact KV allocation")
            states.append(st)
        nat.require_cuda(evict_all, what="record_appended_dms_decisions")
        ea = evict_all.view(torch.uint8)
        is64 = int(pos_t.dtype == torch.int64)
        start = self._contiguous_active_slot_start(states)
        if start is not None:
            live = self.layer_major_live_counts
            if self.debug_checks and bool(torch.any(live[:, start:start + batch] <= 0).item()):
                raise RuntimeError("at least one active (layer, slot, head) has no append slot")
            pos = self.layer_major_token_positions
            em = self.layer_major_evict_mask.view(torch.uint8)
            nat.call("fdms_record_dms_decisions", pos.data_ptr(), pos.stride(0), pos.stride(1), pos.stride(2),
                     pos.stride(3), em.data_ptr(), em.stride(0), em.stride(1), em.stride(2), em.stride(3),
                     live.data_ptr(), live.stride(0), live.stride(1), live.stride(2), ea.data_ptr(), ea.stride(0),
                     ea.stride(1), ea.stride(2), pos_t.data_ptr(), is64, None, start, self.num_layers, batch,
                     self.num_kv_heads, nat.stream())
        else:
            for b, st in enumerate(states):
                if self.debug_checks and bool(torch.any(st.live_counts <= 0).item()):
                    raise RuntimeError(f"sequence {st.seq_id} has at least one (layer, head) without an append slot")
                pos, em, live = st.token_positions, st.evict_mask.view(torch.uint8), st.live_counts
                eb = ea[:, b:b + 1, :]
                nat.call("fdms_record_dms_decisions", pos.data_ptr(), pos.stride(0), 0, pos.stride(1), pos.stride(2),
                         em.data_ptr(), em.stride(0), 0, em.stride(1), em.stride(2), live.data_ptr(),
                         live.stride(0), 0, live.stride(1), eb.data_ptr(), eb.stride(0), eb.stride(1), eb.stride(2),
                         pos_t[b:b + 1].data_ptr(), is64, None, 0, self.num_layers, 1, self.num_kv_heads,
                         nat.stream())
        total = self.num_layers * batch * self.num_kv_heads
        total_true = evict_all.sum()
        if sync_stats:
            total_true = int(total_true.item())
        return {"eviction_decisions_true": total_true, "eviction_decisions_total": total}

    def prepare_decode_metadata(self, seqs: list[Sequence]):
        """slot = base + live; live += 1 on the device; returns
        (base [L,B,H], live [L,B,H], slot [L,B,H], max_capacity) (compact_kv.py:1727-1770)."""
        batch = len(seqs)
        states = []
        for seq in seqs:
            st = self.seq_states.get(seq.seq_id)
            if st is None:
                raise RuntimeError(f"sequence {seq.seq_id} has no compact KV allocation")
            states.append(st)
        max_capacity = max((st.max_capacity_per_lh for st in states), default=0)
        for st in states:
            st.live_upper_bound += 1
        start = self._contiguous_active_slot_start(states)
        L, H = self.num_layers, self.num_kv_heads
        if start is not None:
            base = self.layer_major_base_offsets[:, start:start + batch, :]
            live = self.layer_major_live_counts[:, start:start + batch, :]
            slot = torch.empty((L, batch, H), device=self.device, dtype=torch.int32)
            nat.require_cuda(base, what="prepare_decode_metadata")
            nat.call("fdms_prepare_decode_metadata", base.data_ptr(), base.stride(0), base.stride(1),
                     base.stride(2), live.data_ptr(), live.stride(0), live.stride(1), live.stride(2),
                     slot.data_ptr(), slot.stride(0), slot.stride(1), slot.stride(2), L, batch, H, nat.stream())
            return base, live, slot, max_capacity
        base = torch.empty((L, batch, H), device=self.device, dtype=torch.int32)
        live = torch.empty_like(base)
        slot = torch.empty_like(base)
        for b, st in enumerate(states):
            base[:, b, :] = st.base_offsets
            slot[:, b, :] = st.base_offsets + st.live_counts
            st.live_counts += 1
            live[:, b, :] = st.live_counts
        return base, live, slot, max_capacity

    def max_live_upper_bound(self, seqs: list[Sequence]) -> int:
        """Host-side bound of the largest live count among ``seqs`` (no sync)."""
        return max((self.seq_states[s.seq_id].live_upper_bound for s in seqs), default=0)

    def free(self, seq_id: int) -> None:
        """compact_kv.py:1772-1795."""
        state = self.seq_states.pop(seq_id, None)
        if state is None:
            return
        bases = state.base_offsets.cpu().tolist()
        sizes = state.range_capacity.cpu().tolist()
        for layer_id in range(self.num_layers):
            for h in range(self.num_kv_heads):
                base, size = int(bases[layer_id][h]), int(sizes[layer_id][h])
                if base >= 0 and size > 0:
                    self._free_range(layer_id, base, size)
        if state.active_slot is not None:
            slot = int(state.active_slot)
            self.active_slot_by_seq.pop(seq_id, None)
            if self.layer_major_base_offsets is not None:
                self.layer_major_base_offsets[:, slot, :].fill_(-1)
                self.layer_major_range_capacity[:, slot, :].zero_()
                self.layer_major_live_counts[:, slot, :].zero_()
                self.layer_major_token_positions[:, slot, :, :].fill_(-1)
                self.layer_major_evict_mask[:, slot, :, :].zero_()
            self.free_active_slots.append(slot)
            self.free_active_slots.sort()
