"""C1-C3/C6: FP8 weight quantisation and decode-shaped linears on the GPU.

Per-row FP8 quantisation is bit-exact against the oracle (linear.py:813-823).
Linear outputs are bf16: the kernel accumulates in fp32 in MFMA order, the
references in float64 / fp32, so each output may differ by one bf16 unit in
the last place (plus the reference tests' FP8 tolerance for the FP8 paths).
"""
import numpy as np
import pytest
import torch

from helpers import require_gpu, torch_int4_reference
from oracle import linear as olin
from oracle import numerics

pytestmark = pytest.mark.gpu


def _bf16(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _close_bf16(got, want, what, ulps=1.0, atol=0.0, mag=None):
    """Within `ulps` bf16 units of the larger of the two magnitudes (a value on
    a binade edge may round either way), plus fp32-accumulation noise relative
    to the output's scale for values that cancel to near zero.  ``mag``: the
    magnitude of an intermediate rounded to bf16 before a final add (the
    product before its bias), whose ulps then count too."""
    g, w = got.float().cpu(), want.float()
    m = torch.maximum(w.abs(), g.abs())
    if mag is not None:
        m = torch.maximum(m, mag.float().abs())
    tol = m * (ulps * 2.0 ** -7) + atol + 1e-5 * float(w.abs().max())
    bad = (g - w).abs() > tol
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())}/{bad.numel()} beyond {ulps} ulp; "
                                 f"max err {float((g - w).abs().max()):.4g}")


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("m,n,k,splits", [(8, 2048, 2048, 1), (8, 2048, 8192, 2), (3, 512, 4096, 4),
                                          (16, 1024, 2048, 2), (1, 2048, 8192, 1)])
def test_residual_stats_epilogue(m, n, k, splits, fp8):
    """Epilogue 4, the residual add of the RMSNorm after a decode linear
    (layernorm.py:32-40): with y the same launch's epilogue-0 result (bf16),
    f = fp32(y) + fp32(residual) bit for bit, the residual updated in place to
    bf16(f) bit for bit, each 16-column strip's sum of f^2 within fp32
    summation error of the float64 sum; bf16 and FP8 weights (no activation
    quantisation)."""
    require_gpu()
    from fastdms_amd.layers.linear import linear_residual_stats, linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(m * 131 + n + splits + fp8)
    x, w = _bf16((m, k), g).cuda(), _bf16((n, k), g, 0.02).cuda()
    sinv = None
    if fp8:
        w, sinv = quantize_fp8_rows(w)
    res = _bf16((m, n), g).cuda()
    y = linear_small_m(x, w, weight_scale_inv=sinv, quantize_x=False, k_splits=splits)
    res0 = res.clone()
    f = torch.full((m, n), float("nan"), device="cuda")
    ssq = torch.full((m, n // 16), float("nan"), device="cuda")
    linear_residual_stats(x, w, res, f, ssq, weight_scale_inv=sinv, k_splits=splits)
    torch.cuda.synchronize()
    f_want = y.float() + res0.float()
    assert torch.equal(f, f_want), "f = fp32(y) + fp32(residual)"
    assert torch.equal(res, f_want.to(torch.bfloat16)), "residual = bf16(f)"
    want = f_want.double().pow(2).view(m, n // 16, 16).sum(-1)
    err = float(((ssq.double() - want).abs() / want.clamp(min=1e-30)).max())
    assert err <= 2e-6, f"strip sums of squares: max rel err {err:.3e}"


@pytest.mark.parametrize("m,n,k,epi", [(8, 3072, 2048, 0), (8, 16384, 2048, 1), (1, 512, 2048, 0),
                                       (16, 1024, 4096, 1), (3, 4096, 8192, 0)])
def test_norm_stats_prologue(m, n, k, epi):
    """Prologue 2 on an epilogue-4 producer's output (fp32 rows f, strip sums
    of f^2): y = bf16(bf16(f * rsqrt(mean f^2 + eps)) * norm_w) @ W^T (+ SiLU*up
    for epilogue 1), within 2 bf16 ulps of the float64 product of that
    activation built from the oracle's own sum of squares (the kernel adds the
    strip sums in another order, so an element may round the other way); and
    the same chain against fdms_rmsnorm (+ residual) followed by the plain
    linear, the RMSNorm path the decode step had before."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    from fastdms_amd.layers.linear import (EPI_SILU_MUL, linear_norm_stats, linear_residual_stats,
                                           linear_small_m)
    g = torch.Generator().manual_seed(m * 7 + n + k + epi)
    kp = 2048
    xp, wp = _bf16((m, kp), g).cuda(), _bf16((k, kp), g, 0.03).cuda()  # the producer linear
    res = _bf16((m, k), g).cuda()
    nw = (1.0 + 0.2 * torch.randn(k, generator=g)).to(torch.bfloat16).cuda()
    w = _bf16((n, k), g, 0.02).cuda()
    eps = 1e-5
    # the previous path: the producer's bf16 rows, fdms_rmsnorm with the residual, a plain linear
    yp = linear_small_m(xp, wp)
    h_old, res_old = rms_norm(yp, nw, eps, residual=res)
    out_old = linear_small_m(h_old, w, epilogue=epi)
    f = torch.empty((m, k), device="cuda")
    ssq = torch.empty((m, k // 16), device="cuda")
    linear_residual_stats(xp, wp, res, f, ssq)
    out = linear_norm_stats(f, ssq, nw, eps, w, epilogue=EPI_SILU_MUL if epi else 0)
    torch.cuda.synchronize()
    assert torch.equal(res, res_old), "residual"
    ff = f.double().cpu()
    inv = torch.rsqrt(ff.pow(2).mean(-1, keepdim=True) + eps).float()
    a = (f.cpu() * inv).to(torch.bfloat16).float()
    a = (a * nw.float().cpu()).to(torch.bfloat16).double()
    ref = a @ w.double().cpu().T
    if epi:
        gt, up = ref[:, :n // 2].to(torch.bfloat16).float(), ref[:, n // 2:].to(torch.bfloat16).float()
        ref = torch.nn.functional.silu(gt) * up
    _close_bf16(out, ref.to(torch.bfloat16), "norm-stats linear vs oracle", ulps=2.0, atol=2e-3)
    _close_bf16(out, out_old.cpu(), "norm-stats linear vs rmsnorm + linear", ulps=2.0, atol=2e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quantize_fp8_rows_bit_exact(dtype):
    require_gpu()
    from fastdms_amd.layers.linear import quantize_fp8_rows
    g = torch.Generator().manual_seed(1)
    w = (torch.randn(37, 520, generator=g) * 0.05).to(dtype)
    w[3] = 0.0                     # all-zero row: scale 1
    w[5, 7] = 3.0                  # one large element
    q, sinv = quantize_fp8_rows(w.cuda())
    torch.cuda.synchronize()
    w8_t, sinv_ref = olin.quantize_weight_to_fp8(w.float().numpy())
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), w8_t.T)
    assert np.array_equal(sinv.cpu().numpy().view(np.uint32), sinv_ref.reshape(-1).view(np.uint32))


@pytest.mark.parametrize("k", [520, 2048, 3000, 8192, 12288, 16384, 16392])
@pytest.mark.parametrize("torch_form", [True, False])
def test_quantize_fp8_rows_widths(k, torch_form):
    """bf16 activation rows of every width class of fdms_quantize_fp8_rows (one
    16-byte chunk per thread up to 2048 columns, 2, 4 or 8 chunks up to 16384,
    the two-pass kernel beyond): codes and scale_inv bit-exact vs the oracle's
    quantize_rows_fp8 in both 448 / amax forms, an all-zero row scaled by 1."""
    require_gpu()
    from fastdms_amd.layers.linear import quantize_fp8_rows
    g = torch.Generator().manual_seed(k + torch_form)
    x = (torch.randn(9, k, generator=g) * 0.7).to(torch.bfloat16)
    x[2] = 0.0
    x[4, k - 1] = 40.0  # the row maximum in the last chunk
    q, sinv = quantize_fp8_rows(x.cuda(), torch_form=torch_form)
    torch.cuda.synchronize()
    q_ref, x_scale = olin.quantize_rows_fp8(x.float().numpy(), torch_form=torch_form)
    sinv_ref = (np.float32(1.0) / np.asarray(x_scale, np.float32)).astype(np.float32)  # scale_inv = 1 / s
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(sinv.cpu().numpy().reshape(-1).view(np.uint32), sinv_ref.reshape(-1).view(np.uint32))


def _ref_linear(a, w, bias):
    """bf16(a @ W^T + bias) with fp32 accumulation (F.linear semantics)."""
    y = a.float() @ w.float().T
    if bias is not None:
        y = y + bias.float()
    return y.to(torch.bfloat16)


@pytest.mark.parametrize("m", [1, 3, 8, 16])
@pytest.mark.parametrize("n,k", [(3072, 2048), (2048, 8192), (512, 256), (1024, 4096)])
def test_linear_small_m_bf16(m, n, k):
    require_gpu()
    from fastdms_amd.layers.linear import linear_small_m
    g = torch.Generator().manual_seed(m * 7 + n + k)
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    bias = _bf16((n,), g, 0.1)
    y = linear_small_m(x.cuda(), w.cuda())
    _close_bf16(y, _ref_linear(x, w, None), "no bias")
    y = linear_small_m(x.cuda(), w.cuda(), bias.cuda())
    _close_bf16(y, _ref_linear(x, w, bias), "bias")


def _rms_ref(x, r, nw, eps):
    f = x.float() + (r.float() if r is not None else 0.0)
    inv = torch.rsqrt(f.pow(2).mean(-1, keepdim=True) + eps)
    return (f * inv).to(torch.bfloat16).float().mul(nw.float()).to(torch.bfloat16), f.to(torch.bfloat16)


@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("m,n,k", [(8, 3072, 2048), (1, 256, 512), (16, 2048, 4096)])
def test_linear_small_m_rmsnorm_prologue(with_res, m, n, k):
    """RMSNorm(x + residual) feeding the GEMM (layernorm.py:19-40 + linear):
    residual_out = bf16(x + residual) bit-exact; the output matches
    rmsnorm -> linear up to the norm's fp32 reduction order."""
    require_gpu()
    from fastdms_amd.layers.linear import PRO_RMSNORM, linear_small_m
    g = torch.Generator().manual_seed(m + n + k + with_res)
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    r = _bf16((m, k), g) if with_res else None
    nw = (1.0 + 0.1 * torch.randn(k, generator=g)).to(torch.bfloat16)
    bias = _bf16((n,), g, 0.1)
    ro = torch.empty((m, k), device="cuda", dtype=torch.bfloat16)
    y = linear_small_m(x.cuda(), w.cuda(), bias.cuda(), prologue=PRO_RMSNORM, norm_weight=nw.cuda(), eps=1e-5,
                       residual=None if r is None else r.cuda(), residual_out=ro)
    a, r_new = _rms_ref(x, r, nw, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(ro.cpu(), r_new)
    _close_bf16(y, _ref_linear(a, w, bias), "rmsnorm prologue", ulps=2.0, atol=2e-3)


@pytest.mark.parametrize("m,f,k", [(8, 8192, 2048), (2, 256, 512), (16, 1024, 4096)])
def test_linear_small_m_silu_epilogue(m, f, k):
    """gate_up_proj followed by SiluAndMul in one launch: W = [gate; up] (2F
    rows) and the output is bf16(silu(bf16 gate) * bf16 up) (activation.py:8-11)."""
    require_gpu()
    from fastdms_amd.layers.linear import EPI_SILU_MUL, linear_small_m
    g = torch.Generator().manual_seed(m + f + k)
    x, w = _bf16((m, k), g), _bf16((2 * f, k), g, 0.05)
    y = linear_small_m(x.cuda(), w.cuda(), epilogue=EPI_SILU_MUL)
    gu = _ref_linear(x, w, None).float()
    want = (torch.nn.functional.silu(gu[:, :f]) * gu[:, f:]).to(torch.bfloat16)
    assert y.shape == (m, f)
    _close_bf16(y, want, "silu epilogue", ulps=2.0, atol=2e-3)


@pytest.mark.parametrize("splits", [1, 2, 4, 8])
def test_linear_small_m_split_k_is_consistent(splits):
    """K split over workgroups (merged by the last split through agent-scope
    atomics) gives the same result for every split count, bf16 and FP8, with and
    without the SiLU epilogue; repeated calls (counters reset) agree."""
    require_gpu()
    from fastdms_amd.layers.linear import EPI_SILU_MUL, linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(splits)
    m, n, k = 8, 512, 8192
    x, w = _bf16((m, k), g).cuda(), _bf16((n, k), g, 0.02).cuda()
    bias = _bf16((n,), g, 0.1).cuda()
    want = _ref_linear(x.cpu(), w.cpu(), bias.cpu())
    for _ in range(2):
        _close_bf16(linear_small_m(x, w, bias, k_splits=splits), want, f"bf16 split {splits}")
    w8, si = quantize_fp8_rows(w)
    base = linear_small_m(x, w8, weight_scale_inv=si, k_splits=1)
    _close_bf16(linear_small_m(x, w8, weight_scale_inv=si, k_splits=splits), base.cpu(), f"fp8 split {splits}")
    ye = linear_small_m(x, w, epilogue=EPI_SILU_MUL, k_splits=splits)
    gu = _ref_linear(x.cpu(), w.cpu(), None).float()
    _close_bf16(ye, (torch.nn.functional.silu(gu[:, :n // 2]) * gu[:, n // 2:]).to(torch.bfloat16),
                f"silu split {splits}", ulps=2.0, atol=2e-3)


@pytest.mark.parametrize("m,n,k,splits", [(8, 2048, 8192, 2), (8, 2048, 2048, 2), (3, 512, 4096, 4),
                                          (16, 256, 2048, 1), (1, 2048, 8192, 8)])
def test_linear_partials_sum_to_the_merged_linear(m, n, k, splits):
    """Epilogue 3 (split partials, merge left to the consumer): the fp32
    partials summed in split order and rounded to bf16 equal the merged
    split-K linear bit for bit; the RMSNorm of the partials (+ residual) equals
    the RMSNorm of that bf16 tensor bit for bit."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    from fastdms_amd.layers.linear import SplitPartials, linear_partials, linear_small_m
    g = torch.Generator().manual_seed(m * 31 + splits)
    x, w = _bf16((m, k), g).cuda(), _bf16((n, k), g, 0.02).cuda()
    merged = linear_small_m(x, w, k_splits=splits)
    part = linear_partials(x, w, k_splits=splits)
    assert tuple(part.data.shape) == (splits, m, n)
    acc = torch.zeros((m, n), device="cuda", dtype=torch.float32)
    for s in range(splits):
        acc = acc + part.data[s]
    assert torch.equal(acc.to(torch.bfloat16), merged), "partials do not sum to the merged linear"
    _close_bf16(merged, _ref_linear(x.cpu(), w.cpu(), None), f"partials split {splits}")
    nw = (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16).cuda()
    res = _bf16((m, n), g).cuda()
    want_h, want_res = rms_norm(merged, nw, 1e-5, residual=res)
    got_h, got_res = rms_norm(SplitPartials(part.data), nw, 1e-5, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(got_res, want_res) and torch.equal(got_h, want_h)
    assert torch.equal(rms_norm(SplitPartials(part.data), nw, 1e-5), rms_norm(merged, nw, 1e-5))


@pytest.mark.parametrize("quantize_x", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", [(1, 3072, 2048), (8, 2048, 8192), (5, 512, 256)])
def test_linear_small_m_fp8_matches_oracle(quantize_x, m, n, k):
    """FP8 weights (C2/C3, and C4's _fp8_linear at decode rows with
    quantize_x=2): y = bf16(sum xq*w8 / x_s * scale_inv) + bias in bf16, against
    the float64 oracle (linear.py:492-763)."""
    require_gpu()
    from fastdms_amd.layers.linear import linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(m * 3 + n + k + quantize_x)
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    bias = _bf16((n,), g, 0.1)
    w8, sinv = quantize_fp8_rows(w.cuda())
    y = linear_small_m(x.cuda(), w8, bias.cuda(), weight_scale_inv=sinv, quantize_x=quantize_x)
    w8_t, sinv_ref = olin.quantize_weight_to_fp8(w.float().numpy())
    acc = olin.fp8_linear(x.float().numpy(), w8_t, sinv_ref, quantize_x=bool(quantize_x),
                          torch_form=quantize_x == 2)
    pre = torch.from_numpy(numerics.bf16_round(acc.astype(np.float32)))
    want = (pre + bias.float()).to(torch.bfloat16)
    # the bias is added after a bf16 rounding: a pre-bias value on a rounding
    # edge moves y by one unit of the pre-bias value, whatever y's magnitude
    _close_bf16(y, want, "fp8", ulps=2.0, atol=1e-3 + 2.0 ** -7 * pre.abs())


def _chunk_amax(x, cuts, pad=0):
    """x's row amax as partial maxima over the column ranges between ``cuts``
    (fp32 [rows, parts], row stride parts + pad), as a producer hands them on."""
    edges = [0] + list(cuts) + [x.shape[1]]
    parts = [x[:, a:b].float().abs().amax(dim=1) for a, b in zip(edges[:-1], edges[1:])]
    buf = torch.zeros((x.shape[0], len(parts) + pad), device=x.device, dtype=torch.float32)
    buf[:, :len(parts)] = torch.stack(parts, dim=1)
    return buf[:, :len(parts)]


@pytest.mark.parametrize("quantize_x", [1, 2])
@pytest.mark.parametrize("m,n,k", [(1, 3072, 2048), (8, 2048, 8192), (8, 16384, 2048), (5, 512, 256),
                                   (16, 1024, 4096)])
def test_fp8_producer_amax_gives_the_same_result(quantize_x, m, n, k):
    """The activation's row amax handed in by its producer (one value per row,
    or partial maxima over column ranges, strided rows) replaces the kernel's
    pass over x without changing a bit of y; the same for split partials."""
    require_gpu()
    from fastdms_amd.layers.linear import linear_partials, linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(m + n + k + quantize_x)
    x, w = _bf16((m, k), g).cuda(), _bf16((n, k), g, 0.02).cuda()
    x[0, k // 3] = 40.0   # a dominant column: the amax must come from the right part
    w8, sinv = quantize_fp8_rows(w)
    want = linear_small_m(x, w8, weight_scale_inv=sinv, quantize_x=quantize_x)
    for am in (x.float().abs().amax(dim=1, keepdim=True), _chunk_amax(x, [k // 4, k // 2, k // 2 + 16], pad=3),
               _chunk_amax(x, list(range(8, k, 8)))):
        got = linear_small_m(x, w8, weight_scale_inv=sinv, quantize_x=quantize_x, x_amax=am)
        assert torch.equal(got, want), f"x_amax with {am.shape[1]} parts"
    # the activation quantised by its producer (codes + row amax): same y
    xq, _ = quantize_fp8_rows(x, torch_form=quantize_x == 2)
    got = linear_small_m(xq, w8, weight_scale_inv=sinv, quantize_x=quantize_x, x_amax=_chunk_amax(x, [k // 2]))
    assert torch.equal(got, want), "pre-quantised activation"
    p_want = linear_partials(x, w8, weight_scale_inv=sinv, quantize_x=quantize_x)
    p_want = (p_want.data.clone(), p_want.row_scale.clone())
    p_got = linear_partials(x, w8, weight_scale_inv=sinv, quantize_x=quantize_x,
                            x_amax=_chunk_amax(x, [k // 2]))
    torch.cuda.synchronize()
    assert torch.equal(p_got.data, p_want[0]) and torch.equal(p_got.row_scale, p_want[1])


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("epilogue", [0, 1])
@pytest.mark.parametrize("m,n,k", [(8, 16384, 2048), (3, 512, 256), (16, 2048, 8192)])
def test_strip_amax_output(fp8, epilogue, m, n, k):
    """amax_out[row, strip] = max |y[row, 16 strip : 16 strip + 16]| of the
    written output (gate_up's SiLU*up or a plain linear), split-K included."""
    require_gpu()
    from fastdms_amd.layers.linear import EPI_SILU_MUL, linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(m * 7 + n + epilogue + int(fp8))
    x, w = _bf16((m, k), g).cuda(), _bf16((n, k), g, 0.02).cuda()
    n_out = n // 2 if epilogue == EPI_SILU_MUL else n
    kw = {}
    if fp8:
        w, kw["weight_scale_inv"] = quantize_fp8_rows(w)
    am = torch.full((m, n_out // 16), -1.0, device="cuda", dtype=torch.float32)
    y = linear_small_m(x, w, epilogue=epilogue, amax_out=am, **kw)
    want = y.float().abs().reshape(m, n_out // 16, 16).amax(dim=2)
    torch.cuda.synchronize()
    assert torch.equal(am, want)
    assert torch.equal(linear_small_m(x, w, epilogue=epilogue, **kw), y), "amax_out changed y"


@pytest.mark.parametrize("quantize_x", [0, 1, 2])
@pytest.mark.parametrize("m,n,k,splits", [(8, 2048, 8192, 2), (8, 2048, 2048, 2), (3, 512, 4096, 4),
                                          (16, 256, 2048, 1), (1, 2048, 8192, 8)])
def test_fp8_partials_through_the_rmsnorm_equal_the_merged_linear(quantize_x, m, n, k, splits):
    """FP8 weights on epilogue 3: the consuming RMSNorm's sum of the partials
    times the row scale (1/x_s) and the weight's scale_inv is the merged
    linear's output bit for bit (same split count), and its residual sum,
    output and output amax match the RMSNorm of that tensor bit for bit."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    from fastdms_amd.layers.linear import linear_partials, linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(m * 13 + splits + quantize_x)
    x, w = _bf16((m, k), g).cuda(), _bf16((n, k), g, 0.02).cuda()
    w8, sinv = quantize_fp8_rows(w)
    merged = linear_small_m(x, w8, weight_scale_inv=sinv, quantize_x=quantize_x, k_splits=splits)
    part = linear_partials(x, w8, splits, weight_scale_inv=sinv, quantize_x=quantize_x)
    nw = (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16).cuda()
    res = _bf16((m, n), g).cuda()
    am_want = torch.empty(m, device="cuda", dtype=torch.float32)
    am_got = torch.empty(m, device="cuda", dtype=torch.float32)
    want_h, want_res = rms_norm(merged, nw, 1e-5, residual=res, amax_out=am_want)
    got_h, got_res = rms_norm(part, nw, 1e-5, residual=res, amax_out=am_got)
    torch.cuda.synchronize()
    assert torch.equal(got_res, want_res) and torch.equal(got_h, want_h)
    assert torch.equal(am_got, am_want) and torch.equal(am_want, want_h.float().abs().amax(dim=1))
    assert torch.equal(rms_norm(part, nw, 1e-5), rms_norm(merged, nw, 1e-5))


@pytest.mark.parametrize("quantize_x", [1, 2])
def test_fp8_rows_with_nan_or_inf(quantize_x):
    """A row holding a NaN or an inf: its amax is NaN / inf (NaN propagates
    through every amax), the scale follows the reference's where(amax > 0)
    rule and the row's outputs are NaN, as the oracle's; the other rows are
    unchanged.  Same through the statistics pass, a producer's amax and the
    RMSNorm's quantised codes."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    from fastdms_amd.layers.linear import linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(40 + quantize_x)
    m, n, k = 6, 512, 2048
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    x[1, 100] = float("nan")
    x[3, 7] = float("inf")
    x[4, 9] = -float("inf")
    w8, sinv = quantize_fp8_rows(w.cuda())
    xc = x.cuda()
    y = linear_small_m(xc, w8, weight_scale_inv=sinv, quantize_x=quantize_x).float().cpu()
    w8_t, sinv_ref = olin.quantize_weight_to_fp8(w.float().numpy())
    ref = olin.fp8_linear(x.float().numpy(), w8_t, sinv_ref, quantize_x=True, torch_form=quantize_x == 2)
    bad = [1, 3, 4]
    assert np.isnan(ref[bad]).all() and torch.isnan(y[bad]).all()
    good = [0, 2, 5]
    clean = linear_small_m(xc[good].contiguous(), w8, weight_scale_inv=sinv, quantize_x=quantize_x).float().cpu()
    assert torch.equal(y[good], clean)
    am = xc.float().abs().amax(dim=1, keepdim=True)
    assert torch.isnan(am[1]).all() and torch.isinf(am[3]).all()
    y2 = linear_small_m(xc, w8, weight_scale_inv=sinv, quantize_x=quantize_x, x_amax=am).float().cpu()
    assert torch.isnan(y2[bad]).all() and torch.equal(y2[good], clean)
    # through the RMSNorm: a NaN input row gives a NaN amax and NaN codes
    nw = torch.ones(k, device="cuda", dtype=torch.bfloat16)
    amn = torch.empty(m, device="cuda", dtype=torch.float32)
    q = torch.empty((m, k), device="cuda", dtype=torch.float8_e4m3fn)
    out = rms_norm(xc, nw, 1e-5, amax_out=amn, q_out=q, q_mode=quantize_x)
    assert torch.isnan(amn[1]) and torch.isnan(out[1].float()).all()
    y3 = linear_small_m(q, w8, weight_scale_inv=sinv, quantize_x=quantize_x, x_amax=amn.view(m, 1)).float().cpu()
    y4 = linear_small_m(out, w8, weight_scale_inv=sinv, quantize_x=quantize_x).float().cpu()
    assert torch.equal(torch.isnan(y3), torch.isnan(y4)) and torch.equal(y3.nan_to_num(), y4.nan_to_num())


def test_rmsnorm_amax_output():
    """fdms_rmsnorm's amax_out is each output row's max |value| (plain rows,
    with a residual, and the per-head QK-norm view)."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    g = torch.Generator().manual_seed(5)
    for rows, hidden in ((8, 2048), (1, 4096), (16, 8192), (3, 264)):
        x, r = _bf16((rows, hidden), g).cuda(), _bf16((rows, hidden), g).cuda()
        nw = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).cuda()
        am = torch.empty(rows, device="cuda", dtype=torch.float32)
        out = rms_norm(x, nw, 1e-5, amax_out=am)
        assert torch.equal(am, out.float().abs().amax(dim=1))
        out, _ = rms_norm(x, nw, 1e-5, residual=r, amax_out=am)
        assert torch.equal(am, out.float().abs().amax(dim=1))
    # the quantised output: the codes and scale of quantize_fp8_rows on the
    # bf16 output, bit for bit; bf16_out=False leaves only the codes
    from fastdms_amd.layers.linear import SplitPartials, quantize_fp8_rows
    for q_mode in (1, 2):
        x, r = _bf16((8, 2048), g).cuda(), _bf16((8, 2048), g).cuda()
        nw = (1.0 + 0.1 * torch.randn(2048, generator=g)).to(torch.bfloat16).cuda()
        am = torch.empty(8, device="cuda", dtype=torch.float32)
        codes = torch.empty((8, 2048), device="cuda", dtype=torch.float8_e4m3fn)
        out, _ = rms_norm(x, nw, 1e-5, residual=r, amax_out=am, q_out=codes, q_mode=q_mode)
        want, _ = quantize_fp8_rows(out, torch_form=q_mode == 2)
        assert torch.equal(codes.view(torch.uint8), want.view(torch.uint8))
        codes2 = torch.zeros_like(codes)
        none, _ = rms_norm(x, nw, 1e-5, residual=r, amax_out=am, q_out=codes2, q_mode=q_mode, bf16_out=False)
        assert none is None and torch.equal(codes2.view(torch.uint8), want.view(torch.uint8))
        part = torch.randn((2, 8, 2048), generator=g).cuda()
        codes3 = torch.empty_like(codes)
        out3, _ = rms_norm(SplitPartials(part), nw, 1e-5, residual=r, amax_out=am, q_out=codes3, q_mode=q_mode)
        want3, _ = quantize_fp8_rows(out3, torch_form=q_mode == 2)
        assert torch.equal(codes3.view(torch.uint8), want3.view(torch.uint8))
    q = _bf16((4, 6, 128), g).cuda()
    view = q[:, 1:5]   # strided per-head rows
    nw = (1.0 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).cuda()
    am = torch.empty(16, device="cuda", dtype=torch.float32)
    out = rms_norm(view, nw, 1e-6, amax_out=am)
    assert torch.equal(am, out.float().abs().reshape(16, 128).amax(dim=1))


def test_linear_small_m_argument_errors():
    require_gpu()
    from fastdms_amd.layers.linear import PRO_RMSNORM, linear_small_m
    x = torch.zeros((17, 256), device="cuda", dtype=torch.bfloat16)
    w = torch.zeros((32, 256), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        linear_small_m(x, w)                      # 17 rows
    with pytest.raises(ValueError):
        linear_small_m(x[:4, :200], w[:, :200])   # K not a multiple of 256
    with pytest.raises(RuntimeError):
        xx = x[:4]
        linear_small_m(xx, w, prologue=PRO_RMSNORM, norm_weight=torch.ones(256, device="cuda", dtype=torch.bfloat16),
                       residual=xx, residual_out=xx)   # residual_out aliases the input


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("m,n,k", [(1, 128256, 2048), (8, 4096, 2048), (3, 512, 256), (8, 2048, 8192)])
def test_linear_argmax_small_m(fp8, m, n, k):
    """C7: greedy head = argmax of bf16 logits (bf16 weights) or of fp32 FP8
    scores (embed_head.py:96-211), lowest index on ties; a mismatch is allowed
    only where the reference scores of the two picks are within accumulation
    noise."""
    require_gpu()
    from fastdms_amd.layers.linear import linear_argmax_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(m + n + k + fp8)
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    if fp8:
        w8, si = quantize_fp8_rows(w.cuda())
        tok = linear_argmax_small_m(x.cuda(), w8, weight_scale_inv=si).cpu()
        w8_t, sref = olin.quantize_weight_to_fp8(w.float().numpy())
        sc = torch.from_numpy(olin.fp8_linear(x.float().numpy(), w8_t, sref))
    else:
        tok = linear_argmax_small_m(x.cuda(), w.cuda()).cpu()
        sc = _ref_linear(x, w, None).double()
    want = sc.argmax(dim=1)
    for i in range(m):
        if int(tok[i]) != int(want[i]):
            gap = float(sc[i, want[i]] - sc[i, tok[i]])
            assert gap <= 1e-3 * float(sc[i].abs().max()), (i, int(tok[i]), int(want[i]), gap)


def test_linear_argmax_ties_and_nan():
    """Ties pick the lowest index; a NaN score wins (torch.argmax order)."""
    require_gpu()
    from fastdms_amd.layers.linear import linear_argmax_small_m
    k, n = 256, 4096
    w = torch.zeros((n, k), dtype=torch.bfloat16)
    w[100, 0] = w[3000, 0] = w[4000, 0] = 1.0     # row 0: three-way tie -> 100
    w[2000, 1] = 2.0                               # row 1: strict max at 2000
    x = torch.zeros((2, k), dtype=torch.bfloat16)
    x[0, 0] = 1.0
    x[1, 1] = 1.0
    assert linear_argmax_small_m(x.cuda(), w.cuda()).cpu().tolist() == [100, 2000]
    w[777, 2] = float("nan")                       # a NaN weight makes score 777 NaN for every row
    assert linear_argmax_small_m(x.cuda(), w.cuda()).cpu().tolist() == [777, 777]


@pytest.mark.parametrize("mode", ["symmetric", "asymmetric"])
@pytest.mark.parametrize("group", [32, 128, 256])
def test_quantize_int4_groups_bit_exact(mode, group):
    """C5 quantisation (linear.py:414-459): codes bit-exact vs the oracle,
    bf16 scale / zero bit-exact in the reference's scale_zeros layout [groups,
    N, 2] (linear.py:461-464); the packing puts q[2j] in the low nibble."""
    require_gpu()
    from fastdms_amd.layers.linear import quantize_int4_groups
    g = torch.Generator().manual_seed(group + len(mode))
    w = (torch.randn(48, 1024, generator=g) * 0.05 + (0.02 if mode == "asymmetric" else 0.0)).to(torch.bfloat16)
    w[3, :group] = 0.0
    packed, scale_zeros = quantize_int4_groups(w.cuda(), group, mode)
    assert scale_zeros.shape == (1024 // group, 48, 2) and scale_zeros.dtype == torch.bfloat16
    scale, zero = scale_zeros[:, :, 0].t(), scale_zeros[:, :, 1].t()
    q_ref, s_ref, z_ref = olin.quantize_weight_int4(w.float().numpy(), group, mode)
    p = packed.cpu().numpy()
    q = np.empty((48, 1024), np.uint8)
    q[:, 0::2] = p & 0xF
    q[:, 1::2] = p >> 4
    assert np.array_equal(q, q_ref)
    assert np.array_equal(scale.float().cpu().numpy(), s_ref)
    assert np.array_equal(zero.float().cpu().numpy(), z_ref)
    # the reference's torch expressions evaluated on this GPU agree too
    q_t, s_t, z_t = torch_int4_reference(w.cuda(), group, mode)
    assert np.array_equal(q, q_t) and np.array_equal(s_ref, s_t) and np.array_equal(z_ref, z_t)


@pytest.mark.parametrize("m,n,k,group,mode", [(1, 3072, 2048, 128, "symmetric"), (8, 2048, 8192, 256, "symmetric"),
                                              (5, 512, 256, 32, "symmetric"), (8, 1024, 2048, 128, "asymmetric"),
                                              (3, 512, 768, 64, "asymmetric")])
def test_linear_int4_small_m_matches_oracle(m, n, k, group, mode):
    """W4A16: x @ dequant(W)^T with dequant = bf16((q-8)*s + z) (the oracle's
    float64 dequant differs by the bf16 rounding of each weight only; with an
    asymmetric zero the kernel's q*s + (z - 8s) may round a weight the other
    way); K off a multiple of 128 per wave (the half k-block) included."""
    require_gpu()
    from fastdms_amd.layers.linear import EPI_SILU_MUL, linear_int4_small_m, quantize_int4_groups
    gen = torch.Generator().manual_seed(m + n + k)
    x, w = _bf16((m, k), gen), _bf16((n, k), gen, 0.05)
    if mode == "asymmetric":
        w = (w.float() + 0.03).to(torch.bfloat16)  # groups off zero: a nonzero zero point
    bias = _bf16((n,), gen, 0.1)
    packed, scale_zeros = quantize_int4_groups(w.cuda(), group, mode)
    q, s_ref, z_ref = olin.quantize_weight_int4(w.float().numpy(), group, mode)
    deq = torch.from_numpy(numerics.bf16_round(olin.int4_dequant(q, s_ref, z_ref, group).astype(np.float32)))
    y = linear_int4_small_m(x.cuda(), packed, scale_zeros, group, bias.cuda())
    want = (_ref_linear(x, deq, None).float() + bias.float()).to(torch.bfloat16)  # linear.py:475-477
    _close_bf16(y, want, "int4", ulps=2.0, atol=2e-3)
    tok = linear_int4_small_m(x.cuda(), packed, scale_zeros, group, greedy=True).cpu()
    sc = _ref_linear(x, deq, None).double()
    for i in range(m):
        if int(tok[i]) != int(sc[i].argmax()):
            assert float(sc[i].max() - sc[i, tok[i]]) <= 1e-3 * float(sc[i].abs().max())
    if n % 32 == 0:
        ye = linear_int4_small_m(x.cuda(), packed, scale_zeros, group, epilogue=EPI_SILU_MUL)
        gu = _ref_linear(x, deq, None).float()
        f = n // 2
        _close_bf16(ye, (torch.nn.functional.silu(gu[:, :f]) * gu[:, f:]).to(torch.bfloat16), "int4 silu",
                    ulps=2.0, atol=2e-3)


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_int4_partials_equal_the_merged_linear(splits):
    """W4A16 epilogue 3: the fp32 split partials summed in split order are the
    in-kernel merge at the same split count bit for bit, and the RMSNorm that
    sums them (the decode step's o_proj / down_proj consumer) gives the same
    rows as the RMSNorm of the finished linear."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    from fastdms_amd.layers.linear import linear_int4_partials, linear_int4_small_m, quantize_int4_groups
    gen = torch.Generator().manual_seed(splits)
    m, n, k = 8, 2048, 8192
    x, w = _bf16((m, k), gen), _bf16((n, k), gen, 0.05)
    res = _bf16((m, n), gen)
    nw = (1.0 + 0.2 * torch.randn(n, generator=gen)).to(torch.bfloat16).cuda()
    packed, scale_zeros = quantize_int4_groups(w.cuda(), 128)
    y = linear_int4_small_m(x.cuda(), packed, scale_zeros, 128, k_splits=splits)
    part = linear_int4_partials(x.cuda(), packed, scale_zeros, 128, k_splits=splits)
    acc = part.data[0].clone()
    for i in range(1, splits):
        acc = acc + part.data[i]
    assert torch.equal(acc.to(torch.bfloat16), y), "partials summed in split order"
    h_part, r_part = rms_norm(part, nw, 1e-5, residual=res.cuda())
    h_y, r_y = rms_norm(y, nw, 1e-5, residual=res.cuda())
    assert torch.equal(h_part, h_y) and torch.equal(r_part, r_y), "RMSNorm of the partials"


@pytest.mark.parametrize("m,n,k", [(9, 2048, 2048), (40, 768, 512), (16, 3072, 1000)])
def test_fp8_rows_gemm_prefill_rows(m, n, k):
    """_fp8_linear for prefill row counts (linear.py:635-662): torch-form
    activation quantisation, fp32 products, bf16 output, bias in bf16."""
    require_gpu()
    from fastdms_amd.layers.linear import QX_TORCH, fp8_rows_gemm, quantize_fp8_rows
    g = torch.Generator().manual_seed(m + n + k)
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    bias = _bf16((n,), g, 0.1)
    w8, sinv = quantize_fp8_rows(w.cuda())
    y = fp8_rows_gemm(x.cuda(), w8, sinv.reshape(1, -1), bias.cuda(), QX_TORCH)
    w8_t, sref = olin.quantize_weight_to_fp8(w.float().numpy())
    acc = olin.fp8_linear(x.float().numpy(), w8_t, sref, quantize_x=True, torch_form=True)
    pre = torch.from_numpy(numerics.bf16_round(acc.astype(np.float32)))
    want = (pre + bias.float()).to(torch.bfloat16)
    _close_bf16(y, want, "fp8 rows gemm", ulps=2.0, atol=1e-3, mag=pre)


@pytest.mark.parametrize("impl", ["fdms", "hipblaslt"])
@pytest.mark.parametrize("m,n,k,bias", [(1000, 3072, 2048, False), (300, 202, 272, True), (129, 130, 160, True),
                                         (17, 4096, 1024, False), (4096, 4096, 1024, False),
                                         (4100, 4098, 272, True), (1024, 2048, 8192, True)])
def test_fp8_gemm_matches_the_oracle(m, n, k, bias, impl):
    """The prefill FP8 GEMM (the _scaled_mm of _fp8_linear, linear.py:635-662)
    at prefill row counts, both implementations: fdms_fp8_gemm on the FP8
    matrix cores -- full and partial 128 x 128 tiles and, from 256 tiles of
    256 x 256 up, the LDS-staged kernel (full and partial tiles); a K tail
    (272 = 2 * 128 + 16), N not a multiple of 4 (per-element stores) -- and
    hipBLASLt's scaled GEMM (row counts padded to 16; N or K off 16 run
    fdms_fp8_gemm); bias
    or none; within 2 bf16 ulps of the oracle (fp32 accumulation in a
    different order)."""
    require_gpu()
    from fastdms_amd.layers.linear import fp8_gemm, quantize_fp8_rows
    g = torch.Generator().manual_seed(m * 7 + n + k)
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    b = _bf16((n,), g, 0.1) if bias else None
    w8, sinv = quantize_fp8_rows(w.cuda())
    y = fp8_gemm(x.cuda(), w8, sinv.reshape(1, -1), None if b is None else b.cuda(), impl=impl)
    w8_t, sref = olin.quantize_weight_to_fp8(w.float().numpy())
    acc = olin.fp8_linear(x.float().numpy(), w8_t, sref, quantize_x=True, torch_form=True)
    pre = torch.from_numpy(numerics.bf16_round(acc.astype(np.float32)))
    want = pre if b is None else pre + b.float()
    _close_bf16(y, want.to(torch.bfloat16), "fp8 gemm", ulps=2.0, atol=1e-3, mag=pre)


@pytest.mark.parametrize("m", [2, 8])
def test_linear_argmax_fp8_bf16_scores(m):
    """The FP8 head at more than one row: argmax of the _fp8_linear logits
    rounded to bf16 (forward().argmax(), embed_head.py:543-583); bf16 ties go to
    the lowest index, so the result equals the argmax of the fused logits."""
    require_gpu()
    from fastdms_amd.layers.linear import QX_TORCH, linear_argmax_small_m, linear_small_m, quantize_fp8_rows
    g = torch.Generator().manual_seed(31 + m)
    n, k = 32768, 2048
    x, w = _bf16((m, k), g), _bf16((n, k), g, 0.02)
    w8, si = quantize_fp8_rows(w.cuda())
    tok = linear_argmax_small_m(x.cuda(), w8, weight_scale_inv=si, quantize_x=QX_TORCH, bf16_scores=True).cpu()
    logits = linear_small_m(x.cuda(), w8, weight_scale_inv=si, quantize_x=QX_TORCH).cpu()
    assert tok.tolist() == olin.argmax_lowest(logits.float().numpy()).tolist()
    w8_t, sref = olin.quantize_weight_to_fp8(w.float().numpy())
    sc = numerics.bf16_round(olin.fp8_linear(x.float().numpy(), w8_t, sref, torch_form=True).astype(np.float32))
    for i in range(m):
        gap = float(sc[i].max() - sc[i, int(tok[i])])
        assert gap <= 2 ** -7 * float(np.abs(sc[i]).max()), (i, gap)


def test_fp8_rerank_topk_matches_oracle():
    """embed_head.py:214-302: FP8 re-scoring of candidate ids, lowest id on
    ties, invalid ids never chosen."""
    require_gpu()
    from fastdms_amd.layers.embed_head import fp8_rerank_topk
    from fastdms_amd.layers.linear import quantize_fp8_rows
    g = torch.Generator().manual_seed(5)
    n, k = 4096, 2048
    x, w = _bf16((3, k), g), _bf16((n, k), g, 0.02)
    w[17] = w[9]                                      # identical rows: a tie between ids 9 and 17
    w8, si = quantize_fp8_rows(w.cuda())
    cand = torch.randint(0, n, (3, 16), generator=g)
    cand[1, :2] = torch.tensor([17, 9])
    cand[2, 5] = n + 3                                # out of range: scores -inf
    x[1] = 0.0
    x[1, :k] = (w[9].float() * 10).to(torch.bfloat16)  # row 1 prefers the duplicated rows
    got = fp8_rerank_topk(x.cuda(), cand.cuda(), w8, si.reshape(1, -1)).cpu().tolist()
    w8_t, sref = olin.quantize_weight_to_fp8(w.float().numpy())
    want = [olin.fp8_rerank_topk(x[r].float().numpy(), cand[r].numpy(), w8_t, sref) for r in range(3)]
    assert got[1] == 9 and want[1] == 9
    for r in range(3):
        if got[r] != want[r]:     # accumulation order only: the two scores are within noise
            sc = olin.fp8_linear(x[r:r + 1].float().numpy(), w8_t[:, [got[r], want[r]]], sref[:, [got[r], want[r]]])
            assert abs(sc[0, 0] - sc[0, 1]) <= 1e-5 * abs(sc[0, 1]), (r, got[r], want[r])
