"""Pins of oracle/linear.py (FP8 and INT4 linear layers, linear.py:386-478,
492-763, 813-847; embed_head.py:96-211) by library routines and closed forms."""
import numpy as np
import torch

from oracle import linear as olin
from oracle import numerics

from helpers import torch_int4_reference


def test_fp8_weight_quantisation_matches_torch_formula():
    """The reference's own torch expression (linear.py:386-388, 813-823),
    evaluated with torch's CPU float8 cast, bit for bit."""
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(64, 96, generator=g) * 0.03).to(torch.bfloat16).float()
    w[5] = 0.0
    amax = w.abs().amax(dim=1)
    scale = torch.where(amax > 0, 448.0 / amax, torch.ones(()))
    w8_t_ref = (w.t() * scale.unsqueeze(0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    sinv_ref = scale.reciprocal().reshape(1, -1).numpy()
    w8_t, sinv = olin.quantize_weight_to_fp8(w.numpy())
    assert np.array_equal(w8_t, w8_t_ref)
    assert np.array_equal(sinv.view(np.uint32), sinv_ref.view(np.uint32))


def test_activation_quantisation_matches_torch_formula():
    """linear.py:652-654 (_fp8_linear): x_scale = _amax_to_scale(amax(row)),
    x_fp8 = (x * x_scale).to(fp8) -- torch evaluates 448/amax as reciprocal*448."""
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(400, 128, generator=g) * 3).to(torch.bfloat16).float()
    x[2] = 0.0
    amax = x.abs().amax(dim=1)
    xs = torch.where(amax > 0, 448.0 / amax, torch.ones(()))
    ref = (x * xs.unsqueeze(1)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    xq, x_scale = olin.quantize_rows_fp8(x.numpy(), torch_form=True)
    assert np.array_equal(xq, ref)
    assert np.array_equal(x_scale, xs.numpy())


def test_scale_forms_differ_where_torch_rounds_twice():
    """The two scale forms are both needed: over many amax values some differ
    by one ulp (reciprocal-then-multiply vs a correctly rounded quotient)."""
    a = (np.random.default_rng(7).random(5000) * 10 + 1e-3).astype(np.float32)
    t = olin.amax_to_scale(a, torch_form=True)
    d = olin.amax_to_scale(a, torch_form=False)
    assert np.array_equal(d, (np.float32(448.0) / a).astype(np.float32))
    assert np.array_equal(t, torch.where(torch.from_numpy(a) > 0, 448.0 / torch.from_numpy(a), torch.ones(())).numpy())
    assert 0 < int((t != d).sum()) < a.size


def test_fp8_linear_closed_form_on_exact_inputs():
    """Weights/activations whose per-row amax is 448 quantise to themselves
    (scale 1): the FP8 linear is then exactly the integer matmul."""
    rng = np.random.default_rng(2)
    w = rng.integers(-8, 9, (12, 64)).astype(np.float32)
    x = rng.integers(-8, 9, (3, 64)).astype(np.float32)
    w[:, 0] = 448.0
    x[:, 0] = 448.0
    w8_t, sinv = olin.quantize_weight_to_fp8(w)
    assert np.all(sinv == 1.0)
    assert np.array_equal(olin.fp8_linear(x, w8_t, sinv, quantize_x=True), x.astype(np.float64) @ w.T)


def test_fp8_linear_is_scale_equivariant():
    """Scaling a row of x by 2^j changes x_scale by 2^-j and leaves xq equal,
    so y scales by exactly 2^j (a dropped 1/x_scale term fails this)."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((20, 96)) * 0.05).astype(np.float32)
    x = rng.standard_normal((4, 96)).astype(np.float32)
    w8_t, sinv = olin.quantize_weight_to_fp8(w)
    y = olin.fp8_linear(x, w8_t, sinv)
    y2 = olin.fp8_linear(x * np.float32(8.0), w8_t, sinv)
    assert np.array_equal(y2, y * 8.0)
    # and approximates the unquantised product to FP8 precision (reference test tolerance)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(y - ref).max() <= 0.1 * np.abs(ref).max()


def test_row1_argmax_lowest_index_on_ties():
    w = np.zeros((6, 32), np.float32)
    w[2, 0] = w[4, 0] = 1.0
    w8_t, sinv = olin.quantize_weight_to_fp8(w)
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    assert olin.fp8_row1_argmax(x, w8_t, sinv) == 2


def test_int4_symmetric_quantisation_bounds():
    """linear.py:436-441: s = amax/7, q = clamp(round(w/s), -8, 7) + 8;
    dequant (q-8)*s: error <= s/2 except the clamped -8 end, codes in 0..15."""
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((8, 256)) * 0.05).astype(np.float32)
    w[1, :128] = 0.0
    q, scale, zero = olin.quantize_weight_int4(w, 128, "symmetric")
    assert q.min() >= 1 and q.max() <= 15          # |round(w/s)| <= 7
    assert np.all(zero == 0)
    assert scale[1, 0] == 1.0                      # all-zero group
    deq = olin.int4_dequant(q, scale, zero, 128)
    s = np.repeat(scale, 128, axis=1)
    assert np.all(np.abs(deq - w) <= s / 2 * (1 + 2 ** -7) + 1e-7)


def test_int4_asymmetric_quantisation_bounds():
    """linear.py:442-452: s = span/15, zero = min + 8s, q = round((w-zero)/s + 8)."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((4, 64)) * 0.1 + 0.3).astype(np.float32)
    q, scale, zero = olin.quantize_weight_int4(w, 32, "asymmetric")
    assert q.min() == 0 and q.max() == 15
    deq = olin.int4_dequant(q, scale, zero, 32)
    s = np.repeat(scale.astype(np.float64), 32, axis=1)
    # scale / zero are stored in bf16 (linear.py:456-458): allow their rounding
    assert np.all(np.abs(deq - w) <= s / 2 + np.abs(w) * 2 ** -7 + 4 * s * 2 ** -8)


def test_int4_linear_is_dequantised_matmul():
    rng = np.random.default_rng(6)
    w = rng.standard_normal((16, 128)).astype(np.float32)
    x = rng.standard_normal((2, 128)).astype(np.float32)
    q, s, z = olin.quantize_weight_int4(w, 64)
    assert np.allclose(olin.int4_linear(x, q, s, z, 64), x.astype(np.float64) @ olin.int4_dequant(q, s, z, 64).T)
    assert numerics.bf16_round(s).dtype == np.float32


def test_int4_quantisation_matches_torch_formula():
    """With true division (torch on the CPU) the oracle equals the reference's
    torch expressions bit for bit; the device form (reciprocal multiply) is a
    different rounding that changes some fp32 scales."""
    g = torch.Generator().manual_seed(9)
    w = (torch.randn(64, 512, generator=g) * 0.05 + 0.01).to(torch.bfloat16)
    w[7, :128] = 0.0
    w[9, 128:256] = 0.25
    for mode in ("symmetric", "asymmetric"):
        q_t, s_t, z_t = torch_int4_reference(w, 128, mode)
        q, s, z = olin.quantize_weight_int4(w.float().numpy(), 128, mode, device_form=False)
        assert np.array_equal(q, q_t) and np.array_equal(s, s_t) and np.array_equal(z, z_t)
    a = np.random.default_rng(11).random(4000).astype(np.float32) + 0.01
    assert 0 < int((olin._div_scalar(a, 7.0, True) != olin._div_scalar(a, 7.0, False)).sum()) < a.size
