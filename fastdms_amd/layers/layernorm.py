"""RMSNorm with optional fused residual add (mirror of fastdms/layers/layernorm.py:5-50),
running the HIP kernel ``fdms_rmsnorm``."""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as nat


def _q_args(amax_out, q_out, q_mode, rows, hidden):
    if amax_out is not None and (amax_out.dtype != torch.float32 or not amax_out.is_contiguous()
                                 or amax_out.numel() < rows):
        raise ValueError("amax_out must be contiguous fp32 with one entry per row")
    if q_out is None:
        return 0, 0, 0
    if (amax_out is None or q_out.dtype != torch.float8_e4m3fn or q_out.dim() != 2 or q_out.shape[0] < rows
            or q_out.shape[1] != hidden or q_out.stride(1) != 1 or q_mode not in (1, 2)):
        raise ValueError("q_out must be e4m3fn [rows, hidden] with amax_out and q_mode 1 or 2")
    return q_out.data_ptr(), q_out.stride(0), int(q_mode)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None, residual_out: torch.Tensor | None = None,
             amax_out: torch.Tensor | None = None, q_out: torch.Tensor | None = None, q_mode: int = 1,
             bf16_out: bool = True):
    """bf16 [rows, hidden] (or a strided [tokens, heads, head_dim] view, normed
    per head).  Without residual returns normed x; with residual returns
    (normed(x + residual), x + residual).  x may also be the SplitPartials of a
    decode linear (fp32 split sums, merged here in split order, with an FP8
    linear's row and column scales).  amax_out (fp32, one per output row)
    receives max |out| of each row (NaN if the row holds one), the statistic an
    FP8 consumer's activation quantisation needs; q_out (e4m3fn [rows, hidden])
    receives that quantisation, out * 448/amax (q_mode 1 divides, 2 rounds as
    the torch expression).  bf16_out=False skips the bf16 rows (returned as
    None) when only q_out is wanted."""
    from .linear import SplitPartials
    if isinstance(x, SplitPartials):
        return _rms_norm_partials(x, weight, eps, residual, out, residual_out, amax_out, q_out, q_mode, bf16_out)
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
    q_ptr, q_stride, q_mode = _q_args(amax_out, q_out, q_mode, rows, hidden)
    if not bf16_out and not q_ptr:
        raise ValueError("bf16_out=False needs q_out")
    if out is None and bf16_out:
        out = torch.empty((rows, hidden), device=x.device, dtype=x.dtype)
    if residual is not None:
        residual = residual.reshape(rows, hidden)
        if not residual.is_contiguous():
            raise ValueError("residual must be contiguous")
        if residual_out is None:
            residual_out = torch.empty_like(residual)
    nat.call("fdms_rmsnorm", x.data_ptr(), in_stride, head_stride, heads, nat.ptr(residual), weight.data_ptr(),
             nat.ptr(out), out.stride(0) if bf16_out else hidden, nat.ptr(residual_out), rows, hidden, float(eps),
             nat.ptr(amax_out), q_ptr or None, q_stride, q_mode, nat.stream())
    res = out.view(orig_shape) if bf16_out else None
    if residual is None:
        return res
    return res, residual_out.view(orig_shape)


def _rms_norm_partials(x, weight, eps, residual, out, residual_out, amax_out, q_out, q_mode, bf16_out):
    part = x.data
    k_splits, rows, hidden = part.shape
    if weight.dtype != torch.bfloat16 or not part.is_contiguous():
        raise ValueError("rms_norm of split partials expects contiguous fp32 partials and a bf16 weight")
    q_ptr, q_stride, q_mode = _q_args(amax_out, q_out, q_mode, rows, hidden)
    if not bf16_out and not q_ptr:
        raise ValueError("bf16_out=False needs q_out")
    if out is None and bf16_out:
        out = torch.empty((rows, hidden), device=part.device, dtype=torch.bfloat16)
    if residual is not None:
        residual = residual.reshape(rows, hidden)
        if not residual.is_contiguous():
            raise ValueError("residual must be contiguous")
        if residual_out is None:
            residual_out = torch.empty_like(residual)
    nat.call("fdms_rmsnorm_partials", part.data_ptr(), k_splits, part.stride(0), nat.ptr(residual),
             weight.data_ptr(), nat.ptr(out), out.stride(0) if bf16_out else hidden, nat.ptr(residual_out), rows,
             hidden, float(eps), nat.ptr(x.row_scale), nat.ptr(x.col_scale), nat.ptr(amax_out), q_ptr or None,
             q_stride, q_mode, nat.stream())
    if residual is None:
        return out
    return out, residual_out


class RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None, **quant):
        """``quant``: rms_norm's amax_out / q_out / q_mode / bf16_out."""
        return rms_norm(x, self.weight, self.eps, residual, **quant)
