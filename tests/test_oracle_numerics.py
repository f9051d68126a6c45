"""Pin the oracle's FP8 / bf16 rounding against torch's own CPU casts."""
import numpy as np
import torch

from oracle import numerics


def _all_bf16_values():
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    return vals[np.isfinite(vals)]


def test_fp8_encode_matches_torch_cast_on_every_bf16_value_in_range():
    vals = _all_bf16_values()
    vals = vals[np.abs(vals) <= 448.0]
    ours = numerics.e4m3fn_encode(vals)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_fp8_encode_matches_torch_on_random_fp32_including_ties():
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(200_000) * rng.choice([1e-4, 1e-2, 1, 30, 200], 200_000)).astype(np.float32)
    # exact halfway points between neighbouring e4m3 values
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    lo = numerics.e4m3fn_decode(codes).astype(np.float64)
    hi = numerics.e4m3fn_decode(codes + 1).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    vals = np.concatenate([vals, ties, -ties])
    vals = vals[np.abs(vals) <= 448.0]
    ours = numerics.e4m3fn_encode(vals)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_fp8_saturates_above_448_like_a_satfinite_store():
    vals = np.array([448.0, 449.0, 463.9, 464.0, 465.0, 1e6, np.inf, -500.0, -np.inf], dtype=np.float32)
    assert numerics.e4m3fn_encode(vals).tolist() == [0x7E] * 7 + [0xFE, 0xFE]
    assert numerics.e4m3fn_encode(np.array([np.nan], np.float32))[0] & 0x7F == 0x7F


def test_fp8_decode_round_trips_every_code():
    codes = np.arange(256, dtype=np.uint8)
    vals = numerics.e4m3fn_decode(codes)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    finite = np.isfinite(ref)
    assert np.array_equal(vals[finite], ref[finite])
    assert np.isnan(vals[~finite]).all()
    back = numerics.e4m3fn_encode(vals[finite])
    # +0 and -0 keep their codes; every finite code round-trips
    assert np.array_equal(back, codes[finite])


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(100_000) * 10 ** rng.uniform(-30, 30, 100_000)).astype(np.float32)
    ours = numerics.bf16_round(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, ref)


def test_fp8_values_are_exact_in_bf16():
    vals = numerics.e4m3fn_decode(np.arange(256, dtype=np.uint8))
    vals = vals[np.isfinite(vals)]
    assert np.array_equal(numerics.bf16_round(vals), vals)
