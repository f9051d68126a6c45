"""DMS metadata and decision extraction (mirror of fastdms/engine/dms.py).

``extract_dms_eviction_decisions`` has the reference's signature and checks
(dms.py:152-195) and runs the HIP kernel ``fdms_extract_dms_decisions``.
The reference's CPU-tensor branch (dms.py:222-232) has no counterpart here:
CPU tensors raise instead of falling back.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from pathlib import Path

import numpy as np
import torch

from .. import _native as nat


@dataclass(frozen=True, slots=True)
class DMSMetadata:
    """dms.py:45-59."""
    model_path: str
    source_path: str
    source_kind: str
    packaged_metadata_found: bool
    window_size: int
    alpha_scale: float
    alpha_offset: float
    target_cr: int | None = None
    context_len: int | None = None
    compression_mode: str | None = None

    def to_dict(self) -> dict:
        return asdict(self)


def _metadata_from_config(*, model_path: Path, source_path: Path, source_kind: str,
                          packaged_metadata_found: bool, config: dict) -> DMSMetadata:
    """dms.py:62-89: key aliases and defaults (window 256, scale 100, offset 5)."""
    window_size = config.get("window_size", config.get("dms_window_size", 256))
    alpha_scale = config.get("alpha_scale", config.get("dms_alpha_scale", 100.0))
    alpha_offset = config.get("alpha_offset",
                              config.get("dms_alpha_offset", config.get("dms_initial_alpha_offset", 5.0)))
    target_cr = config.get("target_cr", config.get("dms_cr"))
    context_len = config.get("context_len", config.get("max_position_embeddings"))
    return DMSMetadata(
        model_path=str(model_path), source_path=str(source_path), source_kind=source_kind,
        packaged_metadata_found=packaged_metadata_found, window_size=int(window_size),
        alpha_scale=float(alpha_scale), alpha_offset=float(alpha_offset),
        target_cr=None if target_cr is None else int(target_cr),
        context_len=None if context_len is None else int(context_len),
        compression_mode=config.get("compression_mode"))


def load_dms_metadata(model_path: str | Path, metadata_path: str | Path | None = None) -> DMSMetadata:
    """dms.py:92-149: explicit file -> dms_metadata.json -> parent
    training_log.json -> HF config.json dms_* keys."""
    model_path = Path(model_path)
    if metadata_path is not None:
        path = Path(metadata_path)
        data = json.loads(path.read_text(encoding="utf-8"))
        return _metadata_from_config(model_path=model_path, source_path=path, source_kind="explicit_metadata",
                                     packaged_metadata_found=path.name == "dms_metadata.json",
                                     config=data.get("config", data))
    packaged = model_path / "dms_metadata.json"
    if packaged.exists():
        data = json.loads(packaged.read_text(encoding="utf-8"))
        return _metadata_from_config(model_path=model_path, source_path=packaged, source_kind="packaged_metadata",
                                     packaged_metadata_found=True, config=data.get("config", data))
    training_log = model_path.parent / "training_log.json"
    if training_log.exists():
        data = json.loads(training_log.read_text(encoding="utf-8"))
        return _metadata_from_config(model_path=model_path, source_path=training_log,
                                     source_kind="parent_training_log", packaged_metadata_found=False,
                                     config=data.get("config", {}))
    hf_config = model_path / "config.json"
    if hf_config.exists():
        data = json.loads(hf_config.read_text(encoding="utf-8"))
        if any(k in data for k in ("dms_window_size", "dms_alpha_scale", "dms_initial_alpha_offset", "dms_cr")):
            return _metadata_from_config(model_path=model_path, source_path=hf_config, source_kind="hf_config_dms",
                                         packaged_metadata_found=False, config=data)
    raise FileNotFoundError(f"no DMS metadata found for {model_path}; expected {packaged} or {training_log}")


def dms_threshold_args(alpha_scale: float, alpha_offset: float) -> tuple[float, float, float, int]:
    """(scale, offset, threshold, positive) for the kernels.  The positive-scale
    threshold is the Python-float quotient rounded to fp32, as torch and Triton
    compare it against fp32 values (dms.py:37-38, 224-225)."""
    positive = 1 if alpha_scale > 0 else 0
    thr = float(np.float32(float(alpha_offset) / float(alpha_scale))) if positive else 0.0
    return float(alpha_scale), float(alpha_offset), thr, positive


def extract_dms_eviction_decisions(q: torch.Tensor, *, num_kv_heads: int, num_qo_heads: int, head_dim: int,
                                   alpha_scale: float, alpha_offset: float, inplace: bool = False,
                                   out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-KV-head DMS eviction decisions; zeroes the borrowed channel (dms.py:152-232)."""
    if num_qo_heads % num_kv_heads != 0:
        raise ValueError(f"num_qo_heads={num_qo_heads} must be divisible by num_kv_heads={num_kv_heads}")
    if q.ndim == 2:
        if q.shape[1] != num_qo_heads * head_dim:
            raise ValueError(f"expected flat q width {num_qo_heads * head_dim}, got {q.shape[1]}")
        q_clean = q if inplace else q.clone()
        q_view = q_clean.view(q.shape[0], num_qo_heads, head_dim)
    elif q.ndim == 3:
        if q.shape[1:] != (num_qo_heads, head_dim):
            raise ValueError(f"expected q shape [tokens, {num_qo_heads}, {head_dim}], got {tuple(q.shape)}")
        q_clean = q if inplace else q.clone()
        q_view = q_clean
    else:
        raise ValueError(f"expected q as [tokens, heads, dim] or [tokens, heads*dim], got {tuple(q.shape)}")
    if out is not None:
        expected_shape = (q.shape[0], num_kv_heads)
        if tuple(out.shape) != expected_shape:
            raise ValueError(f"expected DMS output shape {expected_shape}, got {tuple(out.shape)}")
        if out.dtype != torch.bool:
            raise ValueError(f"expected DMS output dtype torch.bool, got {out.dtype}")
        if out.device != q_clean.device:
            raise ValueError(f"expected DMS output on {q_clean.device}, got {out.device}")
    nat.require_cuda(q_clean, what="extract_dms_eviction_decisions")
    evict_mask = out
    if evict_mask is None:
        evict_mask = torch.empty((q.shape[0], num_kv_heads), device=q_clean.device, dtype=torch.bool)
    if q_clean.numel() == 0:
        return q_clean, evict_mask
    scale, offset, thr, positive = dms_threshold_args(alpha_scale, alpha_offset)
    nat.call("fdms_extract_dms_decisions", q_view.data_ptr(), nat.dtype_code(q_view.dtype),
             q_view.stride(0), q_view.stride(1), q_view.stride(2), evict_mask.data_ptr(),
             evict_mask.stride(0), evict_mask.stride(1), q.shape[0], num_kv_heads,
             num_qo_heads // num_kv_heads, head_dim, scale, offset, thr, positive, nat.stream())
    return q_clean, evict_mask


def build_dms_live_mask(evict_mask: torch.Tensor, *, current_position: int, window_size: int,
                        positions: torch.Tensor | None = None) -> torch.Tensor:
    """dms.py:235-262: live = ~evict | (current - pos <= window)."""
    if evict_mask.ndim not in (2, 3):
        raise ValueError(f"expected evict_mask rank 2 or 3, got {evict_mask.ndim}")
    if window_size < 0:
        raise ValueError(f"window_size must be non-negative, got {window_size}")
    tokens = evict_mask.shape[-1]
    if positions is None:
        positions = torch.arange(tokens, device=evict_mask.device)
    else:
        positions = positions.to(device=evict_mask.device)
    if positions.shape != (tokens,):
        raise ValueError(f"expected positions shape {(tokens,)}, got {tuple(positions.shape)}")
    inside = (int(current_position) - positions.to(torch.long)) <= int(window_size)
    return (~evict_mask.bool()) | inside.view((1,) * (evict_mask.ndim - 1) + (tokens,))
