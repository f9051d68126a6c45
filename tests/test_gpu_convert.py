"""Library store casts vs the oracle: every bf16 / fp16 value to FP8, every
FP8 code back, and fp32 -> bf16 on random values (bit-exact)."""
import numpy as np
import pytest
import torch

from helpers import require_gpu, storage_of, to_torch
from oracle import numerics

pytestmark = pytest.mark.gpu


def _convert(src: torch.Tensor, dst_dtype: torch.dtype) -> torch.Tensor:
    from fastdms_amd import _native as nat
    out = torch.empty(src.shape, device=src.device, dtype=dst_dtype)
    nat.call("fdms_convert", src.data_ptr(), nat.dtype_code(src.dtype), out.data_ptr(), nat.dtype_code(dst_dtype),
             src.numel(), nat.stream())
    torch.cuda.synchronize()
    return out


def test_every_bf16_value_to_fp8_matches_oracle():
    require_gpu()
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = numerics.bf16_from_bits(bits)
    src = to_torch(bits, numerics.DT_BF16)
    got = storage_of(_convert(src, torch.float8_e4m3fn))
    exp = numerics.e4m3fn_encode(vals)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], exp[~nan])
    assert ((got[nan] & 0x7F) == 0x7F).all()


def test_random_fp32_to_fp8_and_bf16_match_oracle():
    require_gpu()
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(1 << 20) * 10 ** rng.uniform(-8, 4, 1 << 20)).astype(np.float32)
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    ties = ((numerics.e4m3fn_decode(codes).astype(np.float64) + numerics.e4m3fn_decode(codes + 1)) / 2)
    vals = np.concatenate([vals, ties.astype(np.float32), -ties.astype(np.float32)])
    src = torch.from_numpy(vals).cuda()
    assert np.array_equal(storage_of(_convert(src, torch.float8_e4m3fn)), numerics.e4m3fn_encode(vals))
    assert np.array_equal(storage_of(_convert(src, torch.bfloat16)), numerics.bf16_bits(vals))


def test_every_fp8_code_decodes_exactly():
    require_gpu()
    codes = np.arange(256, dtype=np.uint8)
    got = storage_of(_convert(to_torch(codes, numerics.DT_FP8), torch.float32))
    exp = numerics.e4m3fn_decode(codes)
    fin = np.isfinite(exp)
    assert np.array_equal(got[fin], exp[fin])
    assert np.isnan(got[~fin]).all()
