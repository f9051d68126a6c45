"""Shared test helpers: numpy storage arrays <-> torch device tensors."""
from __future__ import annotations

import numpy as np
import torch

from oracle import numerics

TORCH_DTYPE = {numerics.DT_F32: torch.float32, numerics.DT_F16: torch.float16, numerics.DT_BF16: torch.bfloat16,
               numerics.DT_FP8: torch.float8_e4m3fn}
CODE = {v: k for k, v in TORCH_DTYPE.items()}


def to_torch(storage: np.ndarray, code: int, device="cuda") -> torch.Tensor:
    """numpy storage (f32 / f16 / uint16 bf16 bits / uint8 fp8 bits) -> tensor of that dtype."""
    if code == numerics.DT_F32:
        return torch.from_numpy(np.ascontiguousarray(storage, dtype=np.float32)).to(device)
    if code == numerics.DT_F16:
        return torch.from_numpy(np.ascontiguousarray(storage, dtype=np.float16)).to(device)
    if code == numerics.DT_BF16:
        return torch.from_numpy(np.ascontiguousarray(storage).view(np.int16)).to(device).view(torch.bfloat16)
    if code == numerics.DT_FP8:
        return torch.from_numpy(np.ascontiguousarray(storage, dtype=np.uint8)).to(device).view(torch.float8_e4m3fn)
    raise ValueError(code)


def storage_of(t: torch.Tensor) -> np.ndarray:
    """tensor -> numpy storage array (bit-exact view)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    if t.dtype == torch.float16:
        return t.numpy().copy()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy().copy()
    if t.dtype == torch.bool:
        return t.numpy().copy()
    return t.numpy().copy()


def values_of(t: torch.Tensor) -> np.ndarray:
    """tensor -> float32 numpy values."""
    return t.detach().float().cpu().numpy()


def from_values(vals: np.ndarray, code: int, device="cuda") -> torch.Tensor:
    """float32 values -> rounded to dtype -> device tensor."""
    return to_torch(numerics.to_storage(vals, code), code, device)


def require_gpu():
    import pytest
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def torch_int4_reference(w: torch.Tensor, group: int, mode: str):
    """The reference's quantisation expressions (linear.py:433-452) evaluated by
    torch on w's device (on the CPU tensor / scalar is a true division, on the GPU
    a multiply by the scalar's fp32 reciprocal)."""
    n, k = w.shape
    grouped = w.reshape(n, k // group, group).to(torch.float32)
    one = torch.ones((), device=w.device, dtype=torch.float32)
    if mode == "symmetric":
        amax = grouped.abs().amax(dim=2)
        scale = torch.where(amax > 0, amax / 7.0, one)
        zero = torch.zeros_like(scale)
        q = (torch.round(grouped / scale.unsqueeze(2)).clamp(-8, 7).to(torch.int16) + 8).to(torch.uint8)
    else:
        w_min, w_max = grouped.amin(dim=2), grouped.amax(dim=2)
        span = w_max - w_min
        nz = span > 0
        scale = torch.where(nz, span / 15.0, one)
        zero = torch.where(nz, w_min + 8.0 * scale, w_min)
        q = torch.round((grouped - zero.unsqueeze(2)) / scale.unsqueeze(2) + 8.0).clamp(0, 15).to(torch.uint8)
    return (q.reshape(n, k).cpu().numpy(), scale.to(torch.bfloat16).float().cpu().numpy(),
            zero.to(torch.bfloat16).float().cpu().numpy())

