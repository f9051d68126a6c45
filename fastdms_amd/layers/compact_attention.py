"""Compact-KV attention and expiry ops (mirror of fastdms/layers/compact_attention.py).

Same public names, arguments and ValueError checks as the reference; every op
runs one HIP kernel of libfastdms_amd.  Triton tuning knobs of the reference
(``block_n``, ``grouped``, the split-K / block-N env flags) are accepted and do
not change the math; the split count is chosen here from the batch shape.
"""
from __future__ import annotations

import os

import torch

from .. import _native as nat
from ..engine.dms import dms_threshold_args

_TRUTHY = {"1", "true", "yes", "on"}
_FALSY = {"0", "false", "no", "off"}


def _env_on(name: str, default: str) -> bool:
    return os.environ.get(name, default).strip().lower() not in _FALSY


# Env flags of the reference (compact_attention.py:7-64), read at import like
# the reference.  They select behaviour of the engine glue, not kernel math.
_COMPACT_DEBUG_CHECKS = os.environ.get("FASTDMS_COMPACT_DEBUG_CHECKS") == "1"
_COMPACT_ATTN_SPLITK = _env_on("FASTDMS_COMPACT_ATTN_SPLITK", "auto")
_DMS_FUSED_DECODE_PREPROCESS = _env_on("FASTDMS_DMS_FUSED_DECODE_PREPROCESS", "1")
_COMPACT_ATTN_INLINE_Q_ROPE = os.environ.get("FASTDMS_COMPACT_ATTN_INLINE_Q_ROPE", "1").strip().lower() in _TRUTHY


def compact_attention_splitk_enabled() -> bool:
    return _COMPACT_ATTN_SPLITK


def dms_fused_decode_preprocess_enabled() -> bool:
    return _DMS_FUSED_DECODE_PREPROCESS


def dms_decode_store_transient_k_enabled() -> bool:
    return os.environ.get("FASTDMS_DMS_DECODE_STORE_TRANSIENT_K", "0").strip().lower() in _TRUTHY


def compact_attention_inline_q_rope_enabled() -> bool:
    return _COMPACT_ATTN_INLINE_Q_ROPE


def _next_power_of_2(value: int) -> int:
    if value < 1:
        raise ValueError(f"value must be positive, got {value}")
    return 1 << (value - 1).bit_length()


# ---------------------------------------------------------------------------
# split-K workspace: per device, grown on demand; counters start (and stay) 0
# ---------------------------------------------------------------------------
_WORKSPACE: dict[int, list] = {}
_TARGET_BLOCKS_PER_CU = 1
_NUM_CUS: dict[int, int] = {}


def _num_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _NUM_CUS:
        _NUM_CUS[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _NUM_CUS[idx]


_RETIRED: list[torch.Tensor] = []  # outgrown workspaces: captured graphs may still point at them


def attention_workspace(device: torch.device, n_floats: int, n_counters: int):
    """Return (workspace, counters) with at least the requested sizes.

    A buffer that is outgrown is replaced but never freed, so a HIP graph
    captured against the old one stays valid.  Size it up front with
    reserve_attention_workspace() before capturing."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    entry = _WORKSPACE.setdefault(idx, [None, None])
    if entry[0] is None or entry[0].numel() < n_floats:
        if entry[0] is not None:
            _RETIRED.append(entry[0])
        entry[0] = torch.empty(max(n_floats, 1), device=device, dtype=torch.float32)
    if entry[1] is None or entry[1].numel() < n_counters:
        if entry[1] is not None:
            _RETIRED.append(entry[1])
        entry[1] = torch.zeros(max(n_counters, 1), device=device, dtype=torch.int32)
    return entry[0], entry[1]


_MFMA_CAP_SPLITS = 64


def attention_waves(head_dim: int, fused: bool, pairs: int) -> int:
    """Waves per workgroup of the matrix-core kernel for a launch over `pairs`
    (seq, kv head) pairs, the choice fdms_compact_decode_attention and
    fdms_fused_decode_attention[_paged] make (FASTDMS_AMD_ATTN_WAVES = 4 or 8
    overrides it for the fused head_dim-64 kernel; speed only, never
    results)."""
    if not fused:
        return 4
    if head_dim == 128:
        return 8
    env = os.environ.get("FASTDMS_AMD_ATTN_WAVES", "").strip()
    if env in ("4", "8"):
        return int(env)
    return 8 if 16 < pairs <= 128 else 4


def mfma_split_rows(pairs: int, waves: int = 4, head_dim: int = 64) -> int:
    """Rows per split of the matrix-core kernel (measured on MI355X with the
    bench's own decode states, fused paged decode kernel): with at most 128
    (seq, kv head) pairs, two 64-row groups per wave (a decode step there is
    a chain of memory round trips and more, smaller splits only add merge
    work), beyond that
    1024 rows at head_dim 64 (2048 was 10-20 % slower at 32 and 128
    sequences of the 1B shape: its heavy pairs' single workgroups set the
    launch time) and 2048 at head_dim 128 (the 8B shape's pairs hold ~1600
    rows: 1024-row splits made most of them pay a merge, 25 % slower)."""
    if pairs <= 128:
        return 128 * waves
    return 1024 if head_dim <= 64 else 2048


def mfma_heavy_rows(rows: int, head_dim: int, pairs: int) -> int:
    """Rows per split of a pair longer than `rows` (the matrix-core kernel's
    choice: half of `rows` at head_dim 64 with at most 128 pairs, else
    `rows`; FASTDMS_AMD_ATTN_SPLIT_DIV overrides), which bounds the launch's
    split count."""
    env = os.environ.get("FASTDMS_AMD_ATTN_SPLIT_DIV", "").strip()
    div = int(env) if env in ("1", "2", "4") else (2 if head_dim == 64 and pairs <= 128 else 1)
    return max(64, -(-(rows // div) // 64) * 64)


def reserve_attention_workspace(device: torch.device, max_pairs: int, group_size: int, head_dim: int,
                                max_live: int = 1 << 17) -> None:
    """Allocate the split workspace for the largest split count attention_split_plan
    can return for up to max_pairs (seq, kv head) pairs."""
    target = _TARGET_BLOCKS_PER_CU * _num_cus(device)
    worst = max(p * max(min(1024, -(-target // p)), _MFMA_CAP_SPLITS) for p in range(1, max_pairs + 1))
    attention_workspace(device, worst * group_size * (head_dim + 2), max_pairs)


def mfma_attention_path(q: torch.Tensor, kv: torch.Tensor, group: int) -> bool:
    """True when fdms_compact_decode_attention runs the matrix-core kernel for
    these operands (bf16 q, FP8 K/V, G <= 4, D = 64 / 128, 16-byte rows)."""
    if os.environ.get("FASTDMS_AMD_ATTN_MFMA", "1").strip() == "0":
        return False
    if os.environ.get("FASTDMS_AMD_ATTN_GENERIC", "0").strip() == "1":
        return False
    fp8 = getattr(torch, "float8_e4m3fn", None)
    return (q.dtype == torch.bfloat16 and kv.dtype == fp8 and group <= 4 and q.shape[-1] in (64, 128)
            and kv.stride(0) % 16 == 0 and kv.data_ptr() % 16 == 0)


def attention_split_plan(device: torch.device, pairs: int, max_live: int, mfma: bool,
                         waves: int = 4, head_dim: int = 64) -> tuple[int, int]:
    """(num_splits, split_rows) for fdms_compact_decode_attention.

    Matrix-core kernel: a pair gets one workgroup per split_rows live rows
    (mfma_split_rows), decided per pair inside the kernel from the step's live
    count, so a captured graph stays valid as spans grow; num_splits only
    bounds it from the batch's live bound (at most 64).  Other kernels:
    choose_num_splits, even splits."""
    if mfma:
        rows = mfma_split_rows(pairs, waves, head_dim)
        env = os.environ.get("FASTDMS_AMD_ATTN_SPLIT_ROWS", "").strip()
        if env.isdigit() and int(env) >= 64:  # tuning override
            rows = int(env)
        heavy = mfma_heavy_rows(-(-rows // 64) * 64, head_dim, pairs)
        return int(min(_MFMA_CAP_SPLITS, max(1, -(-int(max_live) // heavy)))), rows
    return choose_num_splits(device, pairs, max_live), 0


def choose_num_splits(device: torch.device, pairs: int, max_live: int) -> int:
    """Even splits per (seq, kv head) for the VALU kernels: about one
    workgroup per CU, each split keeping >= 128 live tokens so the merge
    stays cheap."""
    target = _TARGET_BLOCKS_PER_CU * _num_cus(device)
    s = max(1, -(-target // max(1, pairs)))
    s = min(s, max(1, -(-int(max_live) // 128)))
    return int(min(s, 1024))


def _scale_table(t, num_kv_heads: int, what: str):
    """A per-kv-head FP8 scale table [Hkv] fp32 (contiguous) or None."""
    if t is None:
        return None
    if t.dtype != torch.float32 or t.shape != (num_kv_heads,) or t.stride(0) != 1:
        raise ValueError(f"{what} must be a contiguous float32 [{num_kv_heads}] tensor")
    return t


def _attention_launch(q, kv_k, kv_v, *, base_offsets, block_tables, page_size, live_counts, scale, max_live,
                      rope_positions=None, rope_cache=None, out=None, k_scale=None, v_scale=None):
    batch, num_q_heads, head_dim = q.shape
    num_kv_heads = live_counts.shape[1]
    group = num_q_heads // num_kv_heads
    if out is None:
        out = torch.empty_like(q)
    pairs = batch * num_kv_heads
    # the matrix-core kernel reads pages of at least 16 rows
    mfma = mfma_attention_path(q, kv_k, group) and (block_tables is None or page_size >= 16)
    splits, split_rows = attention_split_plan(q.device, pairs, max_live, mfma,
                                              waves=attention_waves(head_dim, False, pairs), head_dim=head_dim)
    ws, counters = attention_workspace(q.device, pairs * splits * group * (head_dim + 2), pairs)
    if q.stride(2) != 1 or kv_k.stride(1) != 1 or out.stride(2) != 1:
        raise ValueError("compact attention needs a contiguous head_dim axis")
    bt = block_tables
    k_scale = _scale_table(k_scale, num_kv_heads, "k_scale")
    v_scale = _scale_table(v_scale, num_kv_heads, "v_scale")
    if (k_scale is not None or v_scale is not None) and not mfma:
        raise ValueError("per-head FP8 KV scales need the matrix-core path (bf16 q, FP8 K/V, group <= 4, "
                         "head_dim 64 / 128)")
    nat.call("fdms_compact_decode_attention", q.data_ptr(), nat.dtype_code(q.dtype), q.stride(0), q.stride(1),
             kv_k.data_ptr(), kv_v.data_ptr(), nat.dtype_code(kv_k.dtype), kv_k.stride(0),
             nat.ptr(base_offsets), 0 if base_offsets is None else base_offsets.stride(0),
             0 if base_offsets is None else base_offsets.stride(1),
             nat.ptr(bt), 0 if bt is None else bt.stride(0), 0 if bt is None else bt.stride(1), int(page_size),
             live_counts.data_ptr(), live_counts.stride(0), live_counts.stride(1), out.data_ptr(), out.stride(0),
             out.stride(1), ws.data_ptr(), counters.data_ptr(), batch, num_kv_heads, group, head_dim, splits,
             split_rows, float(scale), nat.ptr(rope_cache), 0 if rope_cache is None else rope_cache.stride(0),
             0 if rope_cache is None else rope_cache.stride(2), nat.ptr(rope_positions), nat.ptr(k_scale),
             nat.ptr(v_scale), nat.stream())
    return out


def compact_decode_attention(q: torch.Tensor, compact_k: torch.Tensor, compact_v: torch.Tensor,
                             base_offsets: torch.Tensor, live_counts: torch.Tensor, scale: float | None = None,
                             max_live_count: int | None = None, block_n: int = 128, grouped: bool = True,
                             q_rope_positions: torch.Tensor | None = None,
                             q_rope_cos_sin_cache: torch.Tensor | None = None, *, k_scale: torch.Tensor | None = None,
                             v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention over flat compact K/V spans (compact_attention.py:1116-1336).
    k_scale / v_scale: optional per-kv-head FP8 scales [Hkv] (K = fp8 * k_scale,
    V = fp8 * v_scale; no reference counterpart, the reference casts bare)."""
    if q.ndim != 3:
        raise ValueError(f"expected q as [batch, q_heads, head_dim], got {q.shape}")
    if compact_k.shape != compact_v.shape:
        raise ValueError(f"compact k/v shape mismatch: {compact_k.shape} != {compact_v.shape}")
    if compact_k.ndim != 2:
        raise ValueError(f"expected compact K/V as [total_live, head_dim], got {compact_k.shape}")
    batch, num_q_heads, head_dim = q.shape
    if compact_k.shape[1] != head_dim:
        raise ValueError(f"K/V head_dim {compact_k.shape[1]} does not match q head_dim {head_dim}")
    if base_offsets.shape != live_counts.shape or base_offsets.ndim != 2:
        raise ValueError("base_offsets and live_counts must both be [batch, kv_heads]")
    if base_offsets.shape[0] != batch:
        raise ValueError(f"metadata batch {base_offsets.shape[0]} does not match q batch {batch}")
    num_kv_heads = base_offsets.shape[1]
    if num_q_heads % num_kv_heads != 0:
        raise ValueError(f"q_heads={num_q_heads} must be divisible by kv_heads={num_kv_heads}")
    nat.require_cuda(q, compact_k, compact_v, base_offsets, live_counts, what="compact_decode_attention")
    if max_live_count is None:
        max_live_count = int(live_counts.max().item())
    if max_live_count <= 0:
        raise ValueError("compact decode requires at least one live token per active KV head")
    if _COMPACT_DEBUG_CHECKS and bool(torch.any(live_counts <= 0).item()):
        raise ValueError("compact decode prototype expects every active KV head to have live_count > 0")
    if head_dim > 256:
        raise ValueError(f"head_dim={head_dim} is above the kernel limit")
    if num_q_heads // num_kv_heads > 8:
        raise ValueError(f"group_size={num_q_heads // num_kv_heads} is above the grouped kernel limit")
    compact_k = compact_k.contiguous()
    compact_v = compact_v.contiguous()
    base_offsets = base_offsets.to(device=q.device, dtype=torch.int32).contiguous()
    live_counts = live_counts.to(device=q.device, dtype=torch.int32).contiguous()
    if scale is None:
        scale = head_dim ** -0.5
    inline = q_rope_positions is not None or q_rope_cos_sin_cache is not None
    if inline:
        if q_rope_positions is None or q_rope_cos_sin_cache is None:
            raise ValueError("inline q RoPE requires both positions and cos_sin_cache")
        if head_dim % 2 != 0:
            raise ValueError(f"inline q RoPE requires even head_dim, got {head_dim}")
        if q_rope_positions.shape != (batch,):
            raise ValueError(f"expected q_rope_positions {(batch,)}, got {tuple(q_rope_positions.shape)}")
        q_rope_positions = q_rope_positions.to(device=q.device, dtype=torch.int64).contiguous()
        q_rope_cos_sin_cache = q_rope_cos_sin_cache.to(device=q.device, dtype=torch.float32)
        if q_rope_cos_sin_cache.ndim != 3 or q_rope_cos_sin_cache.shape[2] != head_dim:
            raise ValueError(f"expected q_rope_cos_sin_cache [positions, 1, {head_dim}], "
                             f"got {tuple(q_rope_cos_sin_cache.shape)}")
    return _attention_launch(q, compact_k, compact_v, base_offsets=base_offsets, block_tables=None, page_size=0,
                             live_counts=live_counts, scale=scale, max_live=max_live_count,
                             rope_positions=q_rope_positions if inline else None,
                             rope_cache=q_rope_cos_sin_cache if inline else None, k_scale=k_scale, v_scale=v_scale)


def compact_decode_attention_paged(q: torch.Tensor, kv_k: torch.Tensor, kv_v: torch.Tensor,
                                   block_tables: torch.Tensor, live_counts: torch.Tensor, page_size: int,
                                   scale: float | None = None, max_live_count: int | None = None,
                                   out: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
                                   v_scale: torch.Tensor | None = None,
                                   q_rope_positions: torch.Tensor | None = None,
                                   q_rope_cos_sin_cache: torch.Tensor | None = None) -> torch.Tensor:
    """Same attention over paged compact storage: rank r of (b, h) lives at
    block_tables[b, h, r // page_size] * page_size + r % page_size.
    (No reference counterpart: the reference stores flat spans.)"""
    if q.ndim != 3 or kv_k.ndim != 2 or kv_k.shape != kv_v.shape or kv_k.shape[1] != q.shape[2]:
        raise ValueError("expected q [B, Hq, D] and paged K/V [slots, D]")
    if block_tables.ndim != 3 or block_tables.shape[:2] != live_counts.shape:
        raise ValueError("block_tables must be [batch, kv_heads, max_pages] matching live_counts")
    if page_size <= 0 or page_size & (page_size - 1):
        raise ValueError("page_size must be a power of two")
    nat.require_cuda(q, kv_k, kv_v, block_tables, live_counts, what="compact_decode_attention_paged")
    if max_live_count is None:
        max_live_count = int(live_counts.max().item())
    if scale is None:
        scale = q.shape[2] ** -0.5
    block_tables = block_tables.to(dtype=torch.int32)
    if block_tables.stride(2) != 1:
        block_tables = block_tables.contiguous()
    if (q_rope_positions is None) != (q_rope_cos_sin_cache is None):
        raise ValueError("inline q RoPE requires both positions and cos_sin_cache")
    if q_rope_positions is not None:
        q_rope_positions = q_rope_positions.to(dtype=torch.int64).contiguous()
        q_rope_cos_sin_cache = q_rope_cos_sin_cache.to(dtype=torch.float32)
    return _attention_launch(q, kv_k, kv_v, base_offsets=None, block_tables=block_tables, page_size=page_size,
                             live_counts=live_counts.to(dtype=torch.int32), scale=scale, max_live=max_live_count,
                             out=out, k_scale=k_scale, v_scale=v_scale, rope_positions=q_rope_positions,
                             rope_cache=q_rope_cos_sin_cache)


def store_compact_kvcache(key: torch.Tensor, value: torch.Tensor, compact_k: torch.Tensor, compact_v: torch.Tensor,
                          slot_mapping: torch.Tensor, *, k_scale: torch.Tensor | None = None,
                          v_scale: torch.Tensor | None = None) -> None:
    """compact[slot] = key/value for slot >= 0 (compact_attention.py:968-1007);
    with per-kv-head FP8 scales the stored value is x / scale."""
    if key.shape != value.shape:
        raise ValueError(f"key/value shape mismatch: {key.shape} != {value.shape}")
    if key.ndim != 3:
        raise ValueError(f"expected key/value as [batch, kv_heads, head_dim], got {key.shape}")
    batch, num_kv_heads, head_dim = key.shape
    if compact_k.shape != compact_v.shape:
        raise ValueError(f"compact cache shape mismatch: {compact_k.shape} != {compact_v.shape}")
    if compact_k.ndim != 2 or compact_k.shape[1] != head_dim:
        raise ValueError(f"expected compact cache [slots, {head_dim}], got {compact_k.shape}")
    if slot_mapping.shape != (batch, num_kv_heads):
        raise ValueError(f"expected slot_mapping {(batch, num_kv_heads)}, got {tuple(slot_mapping.shape)}")
    nat.require_cuda(key, value, compact_k, compact_v, what="store_compact_kvcache")
    slot_mapping = slot_mapping.to(device=key.device, dtype=torch.int32).contiguous()
    if key.stride(2) != 1 or value.stride(2) != 1 or compact_k.stride(1) != 1:
        raise ValueError("store_compact_kvcache needs a contiguous head_dim axis")
    nat.call("fdms_store_compact_kvcache", key.data_ptr(), value.data_ptr(), nat.dtype_code(key.dtype),
             key.stride(0), key.stride(1), value.stride(0), value.stride(1), compact_k.data_ptr(),
             compact_v.data_ptr(), nat.dtype_code(compact_k.dtype), compact_k.stride(0), slot_mapping.data_ptr(),
             slot_mapping.stride(0), slot_mapping.stride(1), batch, num_kv_heads, head_dim,
             nat.ptr(_scale_table(k_scale, num_kv_heads, "k_scale")),
             nat.ptr(_scale_table(v_scale, num_kv_heads, "v_scale")), nat.stream())


def fused_dms_rope_store_compact_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                        cos_sin_cache: torch.Tensor, compact_k: torch.Tensor,
                                        compact_v: torch.Tensor, slot_mapping: torch.Tensor,
                                        evict_out: torch.Tensor, positions: torch.Tensor, *, num_kv_heads: int,
                                        alpha_scale: float, alpha_offset: float, store_q: bool = True,
                                        store_transient_k: bool = True, k_scale: torch.Tensor | None = None,
                                        v_scale: torch.Tensor | None = None) -> None:
    """Decode DMS extraction + RoPE + compact append (compact_attention.py:1010-1113);
    with per-kv-head FP8 scales the appended rows are x / scale."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("expected q/k/v as [batch, heads, head_dim]")
    if k.shape != v.shape:
        raise ValueError(f"k/value shape mismatch: {k.shape} != {v.shape}")
    batch, num_q_heads, head_dim = q.shape
    if k.shape[0] != batch or k.shape[1] != num_kv_heads or k.shape[2] != head_dim:
        raise ValueError(f"q/k shape mismatch: q={q.shape}, k={k.shape}, num_kv_heads={num_kv_heads}")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError(f"q_heads={num_q_heads} must be divisible by kv_heads={num_kv_heads}")
    if head_dim % 2 != 0:
        raise ValueError(f"RoPE head_dim must be even, got {head_dim}")
    if compact_k.shape != compact_v.shape or compact_k.ndim != 2 or compact_k.shape[1] != head_dim:
        raise ValueError(f"expected compact cache [slots, {head_dim}], got {compact_k.shape}/{compact_v.shape}")
    if slot_mapping.shape != (batch, num_kv_heads):
        raise ValueError(f"expected slot_mapping {(batch, num_kv_heads)}, got {tuple(slot_mapping.shape)}")
    if evict_out.shape != (batch, num_kv_heads) or evict_out.dtype != torch.bool:
        raise ValueError(f"expected evict_out bool {(batch, num_kv_heads)}, got {tuple(evict_out.shape)} "
                         f"{evict_out.dtype}")
    if positions.shape != (batch,):
        raise ValueError(f"expected positions {(batch,)}, got {tuple(positions.shape)}")
    if head_dim > 256:
        raise ValueError(f"head_dim={head_dim} is above the fused decode preprocess kernel limit")
    nat.require_cuda(q, k, v, compact_k, positions, what="fused decode preprocess")
    slot_mapping = slot_mapping.to(device=q.device, dtype=torch.int32)
    if evict_out.device != q.device:
        raise ValueError(f"expected evict_out on {q.device}, got {evict_out.device}")
    positions = positions.to(device=q.device, dtype=torch.int64)
    cos_sin_cache = cos_sin_cache.to(device=q.device, dtype=torch.float32)
    if cos_sin_cache.ndim != 3 or cos_sin_cache.shape[2] != head_dim:
        raise ValueError(f"expected cos_sin_cache [positions, 1, {head_dim}], got {tuple(cos_sin_cache.shape)}")
    if num_q_heads // num_kv_heads > 8:
        raise ValueError(f"group_size={num_q_heads // num_kv_heads} is above the fused prototype limit")
    if q.stride(2) != 1 or k.stride(2) != 1 or v.stride(2) != 1 or compact_k.stride(1) != 1:
        raise ValueError("fused decode preprocess needs a contiguous head_dim axis")
    scale, offset, thr, positive = dms_threshold_args(alpha_scale, alpha_offset)
    nat.call("fdms_dms_rope_store_compact_decode", q.data_ptr(), nat.dtype_code(q.dtype), q.stride(0), q.stride(1),
             k.data_ptr(), v.data_ptr(), nat.dtype_code(k.dtype), k.stride(0), k.stride(1), v.stride(0),
             v.stride(1), cos_sin_cache.data_ptr(), cos_sin_cache.stride(0), cos_sin_cache.stride(2),
             compact_k.data_ptr(), compact_v.data_ptr(), nat.dtype_code(compact_k.dtype), compact_k.stride(0),
             slot_mapping.data_ptr(), slot_mapping.stride(0), slot_mapping.stride(1), evict_out.data_ptr(),
             evict_out.stride(0), evict_out.stride(1), positions.data_ptr(), batch, num_kv_heads,
             num_q_heads // num_kv_heads, head_dim, scale, offset, thr, positive, int(bool(store_q)),
             int(bool(store_transient_k)), nat.ptr(_scale_table(k_scale, num_kv_heads, "k_scale")),
             nat.ptr(_scale_table(v_scale, num_kv_heads, "v_scale")), nat.stream())


def fused_decode_attention_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                     compact_k: torch.Tensor) -> bool:
    """True when fused_dms_rope_store_compact_decode_attention can run: the
    matrix-core attention path with bf16 q/k/v rows."""
    group = q.shape[1] // max(1, k.shape[1])
    return (mfma_attention_path(q, compact_k, group) and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
            and q.stride(2) == 1 and k.stride(2) == 1 and v.stride(2) == 1 and compact_k.stride(1) == 1
            and os.environ.get("FASTDMS_AMD_FUSED_DECODE_ATTN", "1").strip() != "0")


def fused_dms_rope_store_compact_decode_attention(
        q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos_sin_cache: torch.Tensor, compact_k: torch.Tensor,
        compact_v: torch.Tensor, slot_mapping: torch.Tensor, evict_out: torch.Tensor, positions: torch.Tensor,
        base_offsets: torch.Tensor, live_counts: torch.Tensor, *, num_kv_heads: int, alpha_scale: float,
        alpha_offset: float, scale: float | None = None, max_live_count: int | None = None,
        out: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
        v_scale: torch.Tensor | None = None, block_tables: torch.Tensor | None = None,
        page_size: int = 16, q_norm_weight: torch.Tensor | None = None,
        k_norm_weight: torch.Tensor | None = None, norm_eps: float = 1e-6) -> torch.Tensor:
    """One launch for fused_dms_rope_store_compact_decode(store_q=False,
    store_transient_k=False) followed by compact_decode_attention with the q
    RoPE done in the kernel (the reference's inline-q-RoPE decode order,
    llama.py:112-134).  q, k, v are the raw rows of the step and are not
    modified; ``live_counts`` already counts the appended token (rank
    live - 1, stored at ``slot_mapping``).  k_scale / v_scale: optional
    per-kv-head FP8 scales [Hkv] for the append and the dequant.  With
    ``block_tables`` [B, Hkv, pages] the storage is paged (rank r at row
    block_tables[b, h, r // page_size] * page_size + r % page_size) and
    ``base_offsets`` is ignored (may be None).  q_norm_weight /
    k_norm_weight (bf16 [head_dim]): Qwen3's QK-norm applied in the kernel
    to the raw q / k heads first (RMSNorm with norm_eps, qwen3.py:92-94).
    Returns the attention output."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3 or k.shape != v.shape:
        raise ValueError("expected q [B, Hq, D] and k/v [B, Hkv, D]")
    batch, num_q_heads, head_dim = q.shape
    if k.shape != (batch, num_kv_heads, head_dim) or num_q_heads % num_kv_heads:
        raise ValueError(f"q/k shape mismatch: q={tuple(q.shape)}, k={tuple(k.shape)}, num_kv_heads={num_kv_heads}")
    group = num_q_heads // num_kv_heads
    paged = block_tables is not None
    for name, t in (("slot_mapping", slot_mapping), ("evict_out", evict_out),
                    ("block_tables" if paged else "base_offsets", block_tables if paged else base_offsets),
                    ("live_counts", live_counts)):
        if tuple(t.shape[:2] if paged and name == "block_tables" else t.shape) != (batch, num_kv_heads):
            raise ValueError(f"expected {name} {(batch, num_kv_heads)}, got {tuple(t.shape)}")
    if evict_out.dtype != torch.bool:
        raise ValueError("evict_out must be bool")
    if positions.shape != (batch,):
        raise ValueError(f"expected positions {(batch,)}, got {tuple(positions.shape)}")
    if cos_sin_cache.ndim != 3 or cos_sin_cache.shape[2] != head_dim or cos_sin_cache.dtype != torch.float32:
        raise ValueError(f"expected an fp32 cos_sin_cache [positions, 1, {head_dim}]")
    if not fused_decode_attention_supported(q, k, v, compact_k):
        raise ValueError("fused decode attention needs bf16 q/k/v, FP8 16-byte compact rows, group <= 4, "
                         "head_dim 64 or 128")
    nat.require_cuda(q, k, v, compact_k, compact_v, positions, what="fused decode attention")
    if max_live_count is None:
        max_live_count = int(live_counts.max().item())
    if scale is None:
        scale = head_dim ** -0.5
    if out is None:
        out = torch.empty_like(q)
    if out.stride(2) != 1:
        raise ValueError("out needs a contiguous head_dim axis")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w is not None and (w.dtype != torch.bfloat16 or w.shape != (head_dim,) or not w.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous bf16 [{head_dim}] tensor")
    norms = (nat.ptr(q_norm_weight), nat.ptr(k_norm_weight), float(norm_eps))
    pairs = batch * num_kv_heads
    splits, split_rows = attention_split_plan(q.device, pairs, max_live_count, True,
                                              waves=attention_waves(head_dim, True, pairs), head_dim=head_dim)
    ws, counters = attention_workspace(q.device, pairs * splits * group * (head_dim + 2), pairs)
    slot_mapping = slot_mapping.to(dtype=torch.int32)
    live_counts = live_counts.to(dtype=torch.int32)
    positions = positions.to(dtype=torch.int64)
    s_, off, thr, positive = dms_threshold_args(alpha_scale, alpha_offset)
    ev = evict_out.view(torch.uint8)
    if paged:
        if block_tables.ndim != 3 or block_tables.dtype != torch.int32 or block_tables.stride(2) != 1:
            raise ValueError("block_tables must be int32 [batch, kv_heads, pages] with contiguous pages")
        if page_size < 16 or page_size & (page_size - 1):
            raise ValueError("fused paged decode attention needs a power-of-two page_size >= 16")
        nat.call("fdms_fused_decode_attention_paged", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                 k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cos_sin_cache.data_ptr(),
                 cos_sin_cache.stride(0), cos_sin_cache.stride(2), positions.data_ptr(), slot_mapping.data_ptr(),
                 slot_mapping.stride(0), slot_mapping.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), s_, off,
                 thr, positive, compact_k.data_ptr(), compact_v.data_ptr(), compact_k.stride(0),
                 block_tables.data_ptr(), block_tables.stride(0), block_tables.stride(1), int(page_size),
                 live_counts.data_ptr(), live_counts.stride(0), live_counts.stride(1), out.data_ptr(), out.stride(0),
                 out.stride(1), ws.data_ptr(), counters.data_ptr(), batch, num_kv_heads, group, head_dim, splits,
                 split_rows, float(scale), nat.ptr(_scale_table(k_scale, num_kv_heads, "k_scale")),
                 nat.ptr(_scale_table(v_scale, num_kv_heads, "v_scale")), *norms, nat.stream())
        return out
    base_offsets = base_offsets.to(dtype=torch.int32)
    nat.call("fdms_fused_decode_attention", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
             k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cos_sin_cache.data_ptr(), cos_sin_cache.stride(0),
             cos_sin_cache.stride(2), positions.data_ptr(), slot_mapping.data_ptr(), slot_mapping.stride(0),
             slot_mapping.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), s_, off, thr, positive,
             compact_k.data_ptr(), compact_v.data_ptr(), compact_k.stride(0), base_offsets.data_ptr(),
             base_offsets.stride(0), base_offsets.stride(1), live_counts.data_ptr(), live_counts.stride(0),
             live_counts.stride(1), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), counters.data_ptr(),
             batch, num_kv_heads, group, head_dim, splits, split_rows, float(scale),
             nat.ptr(_scale_table(k_scale, num_kv_heads, "k_scale")),
             nat.ptr(_scale_table(v_scale, num_kv_heads, "v_scale")), *norms, nat.stream())
    return out


PLAN_ROWS = 1024  # ranks per work item at most (fdms_plan.h kPlanRows: two 64-row groups per wave)
PLAN_INTS = 72    # int32 per work item


def decode_plan_enabled(head_dim: int) -> bool:
    """Whether the paged decode step plans its attention work once per step
    (fdms_paged_prepare_decode_plan + fdms_fused_decode_attention_planned)
    instead of partitioning inside each layer's launch.  Default: at head_dim
    128 (measured on MI355X, Qwen3-8B shape c=8: 15.2 against 17.3 us per
    launch, 1 854 against 1 823 decode tok/s); not at head_dim 64 (Llama-3.2-1B
    shape c=8: the same bits 2.5 % slower, 9.26 against 9.02 us -- the heavy
    pairs' later splits learn their pair only from the item -- and the plan
    kernel costs more than the slot kernel it replaces).
    FASTDMS_AMD_ATTN_PLAN=1 / 0 forces it on / off."""
    env = os.environ.get("FASTDMS_AMD_ATTN_PLAN", "").strip()
    if env in ("0", "1"):
        return env == "1"
    return head_dim == 128


def plan_partition(pairs: int, head_dim: int, max_live: int) -> tuple[int, int, int]:
    """(split_rows, heavy_rows, num_splits) of the planned launch for `pairs`
    (seq, kv head) pairs: a pair of at most split_rows ranks is one workgroup
    (two 64-row groups per wave of its eight), a longer one takes pieces of
    heavy_rows ranks, at most num_splits.  At head_dim 64 this is the
    unplanned eight-wave launch's partition (1024 / 512 rows up to 128
    pairs, 1024 / 1024 beyond), so the two give the same bits; at head_dim
    128 pieces of one group per wave (512 rows: the eight-wave loop over a
    128-dim group is the longer part of a pair's chain; measured on the
    Qwen3-8B shape).  FASTDMS_AMD_PLAN_SPLIT_ROWS / _HEAVY_ROWS override
    (multiples of 64, heavy <= split <= 1024; tuning only)."""
    if head_dim <= 64:
        rows, heavy = PLAN_ROWS, (512 if pairs <= 128 else PLAN_ROWS)
    else:
        rows = heavy = 512
    env_r = os.environ.get("FASTDMS_AMD_PLAN_SPLIT_ROWS", "").strip()
    env_h = os.environ.get("FASTDMS_AMD_PLAN_HEAVY_ROWS", "").strip()
    if env_r.isdigit():
        rows = int(env_r)
    if env_h.isdigit():
        heavy = int(env_h)
    heavy = min(heavy, rows)
    if rows % 64 or heavy % 64 or not 64 <= heavy <= rows <= PLAN_ROWS:
        raise ValueError(f"plan partition {rows} / {heavy} rows: multiples of 64, heavy <= split <= {PLAN_ROWS}")
    return rows, heavy, int(min(_MFMA_CAP_SPLITS, max(1, -(-int(max_live) // heavy))))


PLAN_LEAD = 4  # ints before a layer's items (the last: its count of further splits)


class DecodePlan:
    """Static buffer of the step's attention work plan, ``items`` [layers,
    4 + items * 72] int32: per layer 4 ints (the last: the number of further
    splits) and one item per live workgroup of a planned launch (split 0 of
    pair p at item p, the further splits after the pairs).  Sized for every
    batch of up to ``max_pairs`` (seq, kv head) pairs whose live counts stay
    within ``max_live``; its address never changes, so captured decode graphs
    keep it."""

    def __init__(self, device, num_layers: int, max_pairs: int, max_live: int, head_dim: int):
        self.max_live, self.head_dim, self.pairs = int(max_live), int(head_dim), int(max_pairs)
        need = max(p * self.partition(p)[2] for p in range(1, max_pairs + 1))
        self.items = torch.zeros((num_layers, PLAN_LEAD + need * PLAN_INTS), device=device, dtype=torch.int32)

    def layer_items(self, layer_id: int) -> torch.Tensor:
        """Layer ``layer_id``'s items (the attention launch's plan pointer)."""
        return self.items[layer_id, PLAN_LEAD:]

    def further_splits(self) -> torch.Tensor:
        """[layers] view of each layer's count of further splits."""
        return self.items[:, PLAN_LEAD - 1]

    def partition(self, pairs: int) -> tuple[int, int, int]:
        return plan_partition(pairs, self.head_dim, self.max_live)


def fused_decode_attention_planned(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos_sin_cache: torch.Tensor,
                                   compact_k: torch.Tensor, compact_v: torch.Tensor, evict_out: torch.Tensor,
                                   positions: torch.Tensor, plan: DecodePlan, layer_id: int, *, num_kv_heads: int,
                                   alpha_scale: float,
                                   alpha_offset: float, scale: float | None = None, out: torch.Tensor | None = None,
                                   k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
                                   q_norm_weight: torch.Tensor | None = None,
                                   k_norm_weight: torch.Tensor | None = None, norm_eps: float = 1e-6) -> torch.Tensor:
    """fused_dms_rope_store_compact_decode_attention on the paged layout with
    the step's work plan (written by PagedCompactKVManager.paged_prepare_decode
    with a plan): the plan's items of layer ``layer_id`` carry the pairs'
    rank ranges, live counts, append rows and page ids, so no live counts,
    slots or block tables are passed; ``positions`` are the step's int64
    positions.  Same checks and results as the unplanned launch (bit for
    bit where both use the same partition, see plan_partition)."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3 or k.shape != v.shape:
        raise ValueError("expected q [B, Hq, D] and k/v [B, Hkv, D]")
    batch, num_q_heads, head_dim = q.shape
    if k.shape != (batch, num_kv_heads, head_dim) or num_q_heads % num_kv_heads:
        raise ValueError(f"q/k shape mismatch: q={tuple(q.shape)}, k={tuple(k.shape)}, num_kv_heads={num_kv_heads}")
    if batch * num_kv_heads > plan.pairs:
        raise ValueError(f"the plan holds {plan.pairs} pairs, the batch has {batch * num_kv_heads}")
    if positions.dtype != torch.int64 or positions.shape[0] < batch:
        raise ValueError("positions must be int64 [batch]")
    if evict_out.dtype != torch.bool or tuple(evict_out.shape) != (batch, num_kv_heads):
        raise ValueError(f"evict_out must be bool {(batch, num_kv_heads)}")
    if cos_sin_cache.ndim != 3 or cos_sin_cache.shape[2] != head_dim or cos_sin_cache.dtype != torch.float32:
        raise ValueError(f"expected an fp32 cos_sin_cache [positions, 1, {head_dim}]")
    if not fused_decode_attention_supported(q, k, v, compact_k):
        raise ValueError("fused decode attention needs bf16 q/k/v, FP8 16-byte compact rows, group <= 4, "
                         "head_dim 64 or 128")
    nat.require_cuda(q, k, v, compact_k, compact_v, what="planned decode attention")
    group = num_q_heads // num_kv_heads
    if scale is None:
        scale = head_dim ** -0.5
    if out is None:
        out = torch.empty_like(q)
    if out.stride(2) != 1:
        raise ValueError("out needs a contiguous head_dim axis")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w is not None and (w.dtype != torch.bfloat16 or w.shape != (head_dim,) or not w.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous bf16 [{head_dim}] tensor")
    pairs = batch * num_kv_heads
    splits = plan.partition(pairs)[2]
    ws, counters = attention_workspace(q.device, pairs * splits * group * (head_dim + 2), pairs)
    s_, off, thr, positive = dms_threshold_args(alpha_scale, alpha_offset)
    ev = evict_out.view(torch.uint8)
    items = plan.layer_items(layer_id)
    nat.call("fdms_fused_decode_attention_planned", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
             k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cos_sin_cache.data_ptr(),
             cos_sin_cache.stride(0), cos_sin_cache.stride(2), positions.data_ptr(), items.data_ptr(), ev.data_ptr(),
             ev.stride(0),
             ev.stride(1), s_, off, thr, positive, compact_k.data_ptr(), compact_v.data_ptr(), compact_k.stride(0),
             out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), counters.data_ptr(), batch, num_kv_heads,
             group, head_dim, splits, float(scale), nat.ptr(_scale_table(k_scale, num_kv_heads, "k_scale")),
             nat.ptr(_scale_table(v_scale, num_kv_heads, "v_scale")), nat.ptr(q_norm_weight),
             nat.ptr(k_norm_weight), float(norm_eps), nat.stream())
    return out


def _expiry(incremental: bool, *, positions_per_lh, evict_per_lh, live_counts, base_offsets, compact_k, compact_v,
            current_positions, window_size):
    num_seqs, num_kv_heads, max_capacity = positions_per_lh.shape
    if evict_per_lh.shape != positions_per_lh.shape:
        raise ValueError("positions_per_lh and evict_per_lh must match")
    if live_counts.shape != (num_seqs, num_kv_heads) or base_offsets.shape != (num_seqs, num_kv_heads):
        raise ValueError("live_counts/base_offsets must be [num_seqs, num_kv_heads]")
    if positions_per_lh.stride(2) != 1 or evict_per_lh.stride(2) != 1:
        raise ValueError("expiry metadata needs a contiguous slot axis")
    nat.require_cuda(positions_per_lh, evict_per_lh, live_counts, compact_k, what="dms expiry")
    cur = current_positions.to(device=positions_per_lh.device, dtype=torch.int64).contiguous()
    esz = compact_k.element_size()
    nat.call("fdms_dms_expiry", int(incremental), positions_per_lh.data_ptr(), 0, positions_per_lh.stride(0),
             positions_per_lh.stride(1), evict_per_lh.data_ptr(), 0, evict_per_lh.stride(0), evict_per_lh.stride(1),
             live_counts.data_ptr(), 0, live_counts.stride(0), live_counts.stride(1), base_offsets.data_ptr(), 0,
             base_offsets.stride(0), base_offsets.stride(1), compact_k.data_ptr(), compact_v.data_ptr(), None, None,
             compact_k.shape[-1] * esz, compact_k.stride(0) * esz, cur.data_ptr(), 1, num_seqs, num_kv_heads,
             int(window_size), nat.stream())


def dms_expiry_one_layer(*, positions_per_lh, evict_per_lh, live_counts, base_offsets, compact_k, compact_v,
                         current_positions, window_size: int) -> None:
    """Full per-(seq, head) re-compaction of one layer (compact_attention.py:861-911)."""
    _expiry(False, positions_per_lh=positions_per_lh, evict_per_lh=evict_per_lh, live_counts=live_counts,
            base_offsets=base_offsets, compact_k=compact_k, compact_v=compact_v,
            current_positions=current_positions, window_size=window_size)


def dms_expiry_incremental_one_layer(*, positions_per_lh, evict_per_lh, live_counts, base_offsets, compact_k,
                                     compact_v, current_positions, window_size: int) -> None:
    """Steady-state single-slot expiry of one layer (compact_attention.py:914-965)."""
    _expiry(True, positions_per_lh=positions_per_lh, evict_per_lh=evict_per_lh, live_counts=live_counts,
            base_offsets=base_offsets, compact_k=compact_k, compact_v=compact_v,
            current_positions=current_positions, window_size=window_size)
