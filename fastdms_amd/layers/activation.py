"""SiLU(gate) * up (mirror of fastdms/layers/activation.py), HIP kernel ``fdms_silu_mul``."""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as nat


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("silu_and_mul expects contiguous bf16 [rows, 2F]")
    f = x.shape[-1] // 2
    rows = x.numel() // x.shape[-1]
    if out is None:
        out = torch.empty(x.shape[:-1] + (f,), device=x.device, dtype=x.dtype)
    nat.call("fdms_silu_mul", x.data_ptr(), out.data_ptr(), rows, f, nat.stream())
    return out


class SiluAndMul(nn.Module):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return silu_and_mul(x)
