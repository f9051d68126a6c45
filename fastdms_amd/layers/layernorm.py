"""RMSNorm with optional fused residual add (mirror of fastdms/layers/layernorm.py:5-50),
running the HIP kernel ``fdms_rmsnorm``."""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as nat


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None, residual_out: torch.Tensor | None = None):
    """bf16 [rows, hidden] (or a strided [tokens, heads, head_dim] view, normed
    per head).  Without residual returns normed x; with residual returns
    (normed(x + residual), x + residual).  x may also be the SplitPartials of a
    decode linear (fp32 split sums, merged here in split order)."""
    from .linear import SplitPartials
    if isinstance(x, SplitPartials):
        return _rms_norm_partials(x, weight, eps, residual, out, residual_out)
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or weight.dtype != torch.bfloat16:
        raise ValueError("rms_norm expects bf16 rows with a contiguous hidden axis and a bf16 weight")
    hidden = x.shape[-1]
    orig_shape = x.shape
    if x.ndim == 3 and not x.is_contiguous():
        tokens, heads = x.shape[0], x.shape[1]
        in_stride, head_stride = x.stride(0), x.stride(1)
    else:
        x = x.reshape(-1, hidden) if x.ndim != 2 else x
        tokens, heads = x.shape[0], 1
        in_stride, head_stride = x.stride(0), 0
    rows = tokens * heads
    if out is None:
        out = torch.empty((rows, hidden), device=x.device, dtype=x.dtype)
    if residual is not None:
        residual = residual.reshape(rows, hidden)
        if not residual.is_contiguous():
            raise ValueError("residual must be contiguous")
        if residual_out is None:
            residual_out = torch.empty_like(residual)
    nat.call("fdms_rmsnorm", x.data_ptr(), in_stride, head_stride, heads, nat.ptr(residual), weight.data_ptr(),
             out.data_ptr(), out.stride(0), nat.ptr(residual_out), rows, hidden, float(eps), nat.stream())
    if residual is None:
        return out.view(orig_shape)
    return out.view(orig_shape), residual_out.view(orig_shape)


def _rms_norm_partials(x, weight, eps, residual, out, residual_out):
    part = x.data
    k_splits, rows, hidden = part.shape
    if weight.dtype != torch.bfloat16 or not part.is_contiguous():
        raise ValueError("rms_norm of split partials expects contiguous fp32 partials and a bf16 weight")
    if out is None:
        out = torch.empty((rows, hidden), device=part.device, dtype=torch.bfloat16)
    if residual is not None:
        residual = residual.reshape(rows, hidden)
        if not residual.is_contiguous():
            raise ValueError("residual must be contiguous")
        if residual_out is None:
            residual_out = torch.empty_like(residual)
    nat.call("fdms_rmsnorm_partials", part.data_ptr(), k_splits, part.stride(0), nat.ptr(residual),
             weight.data_ptr(), out.data_ptr(), out.stride(0), nat.ptr(residual_out), rows, hidden, float(eps),
             nat.stream())
    if residual is None:
        return out
    return out, residual_out


class RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        return rms_norm(x, self.weight, self.eps, residual)
