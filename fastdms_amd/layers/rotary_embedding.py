"""Rotary embedding (mirror of fastdms/layers/rotary_embedding.py).

The cos/sin table is built once at construction with the reference's fp32
torch formula (rotary_embedding.py:52-73) and then lives on the GPU; the
rotation itself runs in the HIP kernels (``fdms_rope_inplace`` for prefill,
fused into the decode preprocess for decode).
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .. import _native as nat


def _apply_llama3_freq_scaling(inv_freq: torch.Tensor, factor: float, low_freq_factor: float,
                               high_freq_factor: float, original_max_position: int) -> torch.Tensor:
    """rotary_embedding.py:18-36 (transformers' llama3 rope scaling)."""
    low_freq_wavelen = original_max_position / low_freq_factor
    high_freq_wavelen = original_max_position / high_freq_factor
    wavelen = 2 * math.pi / inv_freq
    inv_freq_low = inv_freq / factor
    smooth = (original_max_position / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    smooth_freq = (1.0 - smooth) * inv_freq_low + smooth * inv_freq
    out = torch.where(wavelen < high_freq_wavelen, inv_freq, smooth_freq)
    return torch.where(wavelen > low_freq_wavelen, inv_freq_low, out)


def build_cos_sin_cache(head_size: int, max_position: int, base: float, rope_scaling: dict | None = None):
    """fp32 [max_position, 1, head_size] table cat(cos, sin), built on the CPU."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float) / head_size))
    if rope_scaling is not None:
        rope_type = rope_scaling.get("rope_type") or rope_scaling.get("type")
        if rope_type == "llama3":
            inv_freq = _apply_llama3_freq_scaling(
                inv_freq, factor=float(rope_scaling["factor"]),
                low_freq_factor=float(rope_scaling.get("low_freq_factor", 1.0)),
                high_freq_factor=float(rope_scaling.get("high_freq_factor", 4.0)),
                original_max_position=int(rope_scaling["original_max_position_embeddings"]))
        elif rope_type in (None, "default", "linear"):
            if rope_type == "linear":
                inv_freq = inv_freq / float(rope_scaling.get("factor", 1.0))
        else:
            raise NotImplementedError(f"rope_type={rope_type!r} is not implemented")
    t = torch.arange(max_position, dtype=torch.float)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)


def rope_inplace(x: torch.Tensor, positions: torch.Tensor, cos_sin_cache: torch.Tensor) -> torch.Tensor:
    """x[t, h, :] <- rotate(x[t, h, :], positions[t]) in place (x: [T, H, D])."""
    if x.ndim != 3 or x.stride(2) != 1:
        raise ValueError("rope_inplace expects a [tokens, heads, head_dim] view with contiguous head_dim")
    nat.require_cuda(x, positions, cos_sin_cache, what="rope_inplace")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    nat.call("fdms_rope_inplace", x.data_ptr(), nat.dtype_code(x.dtype), x.stride(0), x.stride(1), x.shape[0],
             x.shape[1], x.shape[2], cos_sin_cache.data_ptr(), cos_sin_cache.stride(0), cos_sin_cache.stride(2),
             pos.data_ptr(), nat.stream())
    return x


class RotaryEmbedding(nn.Module):
    """rotary_embedding.py:39-86."""

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float,
                 rope_scaling: dict | None = None) -> None:
        super().__init__()
        self.head_size = head_size
        assert rotary_dim == head_size
        cache = build_cos_sin_cache(head_size, max_position_embeddings, base, rope_scaling)
        self.register_buffer("cos_sin_cache", cache, persistent=False)

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        """Rotate q [T, Hq, D] and k [T, Hkv, D] in place and return them."""
        rope_inplace(query, positions, self.cos_sin_cache)
        rope_inplace(key, positions, self.cos_sin_cache)
        return query, key


_ROPE_CACHE: dict[tuple, RotaryEmbedding] = {}


def _rope_scaling_key(rope_scaling: dict | None):
    if rope_scaling is None:
        return None
    return tuple(sorted((k, tuple(v) if isinstance(v, list) else v) for k, v in rope_scaling.items()))


def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float, rope_scaling: dict | None = None):
    """rotary_embedding.py:101-114."""
    key = (head_size, rotary_dim, max_position, base, _rope_scaling_key(rope_scaling))
    rope = _ROPE_CACHE.get(key)
    if rope is None:
        rope = RotaryEmbedding(head_size, rotary_dim, max_position, base, rope_scaling=rope_scaling)
        _ROPE_CACHE[key] = rope
    return rope
