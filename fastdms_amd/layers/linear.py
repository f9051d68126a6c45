"""Linear layers (mirror of fastdms/layers/linear.py class names, single GPU).

Decode-shaped calls (at most 16 rows) run the HIP kernels
``fdms_linear_small_m`` (bf16 or FP8 weights, optional fused RMSNorm prologue
or SiLU*up epilogue) and ``fdms_linear_int4_small_m`` (INT4 weights).  FP8 /
INT4 weights are made by ``fdms_quantize_fp8_rows`` / ``fdms_quantize_int4_groups``
as the reference's ``quantize_weight_to_fp8`` makes them (linear.py:813-847,
414-459), and ``LinearBase.route`` picks the path in the reference's order
(linear.py:855-926) under the same environment switches.  Prefill row counts
use the ROCm GEMM library (hipBLASLt through torch) for bf16 weights.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F
from torch import nn

from .. import _native as nat
from . import quant_env as qe

PRO_NONE, PRO_RMSNORM, PRO_NORM_STATS = 0, 1, 2
EPI_NONE, EPI_SILU_MUL, EPI_PARTIALS, EPI_RESIDUAL_STATS = 0, 1, 3, 4
QX_NONE, QX_DIVIDE, QX_TORCH = 0, 1, 2   # activation quantisation: none / 448/amax / reciprocal(amax)*448
SMALL_M_MAX_ROWS = 16
_MAX_K_SPLITS = 8


def int4_max_rows() -> int:
    return qe.int4_max_rows()


def small_m_supported(rows: int, in_features: int, out_features: int) -> bool:
    """Shapes fdms_linear_small_m accepts (k-blocks of 64 per wave, 16-column strips)."""
    return 1 <= rows <= SMALL_M_MAX_ROWS and in_features % 256 == 0 and out_features % 16 == 0


# split-K workspace per device: grown on demand, never freed (captured graphs keep pointing at it)
_WS: dict[int, list] = {}
_RETIRED: list[torch.Tensor] = []
_NUM_CUS: dict[int, int] = {}


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _num_cus(device: torch.device) -> int:
    idx = _device_index(device)
    if idx not in _NUM_CUS:
        _NUM_CUS[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _NUM_CUS[idx]


def choose_k_splits(device: torch.device, strips: int, k: int) -> int:
    """Split K over workgroups when there are fewer 16-column strips than CUs
    and K is long: the merge costs about one memory round trip, which only a
    long per-workgroup K amortises.  Each split keeps at least 2048 columns in
    whole 256-column slices."""
    s = 1
    cus = _num_cus(device)
    while (s * 2 <= _MAX_K_SPLITS and strips * s < cus and k % (s * 2 * 256) == 0
           and k // (s * 2) >= 2048 and k >= 4096):
        s *= 2
    return s


def choose_partial_splits(device: torch.device, strips: int, k: int) -> int:
    """K splits of a linear whose merge the consumer does (no merge cost in the
    linear): enough workgroups to cover the CUs, each split a whole number of
    512-column slices.  FASTDMS_AMD_PARTIAL_SPLITS overrides (tuning)."""
    env = os.environ.get("FASTDMS_AMD_PARTIAL_SPLITS", "").strip()
    if env.isdigit() and int(env) >= 1 and k % (int(env) * 256) == 0:
        return int(env)
    s = 1
    cus = _num_cus(device)
    while s * 2 <= _MAX_K_SPLITS and strips * s < cus and k % (s * 2 * 512) == 0:
        s *= 2
    return s


class SplitPartials:
    """fp32 split-K partial sums [k_splits, rows, n] of a decode linear whose
    merge is left to the consuming RMSNorm (``rms_norm`` accepts this in place
    of x): x = bf16(sum over splits, in split order), times ``row_scale[row]``
    (an FP8 linear's 1/x_s) and ``col_scale[col]`` (its weight scale_inv) when
    present."""

    def __init__(self, data: torch.Tensor, row_scale: torch.Tensor | None = None,
                 col_scale: torch.Tensor | None = None):
        self.data = data
        self.row_scale = row_scale
        self.col_scale = col_scale

    @property
    def shape(self):
        return self.data.shape[1:]


_PARTIALS: dict[int, torch.Tensor] = {}
_ROW_SCALES: dict[int, torch.Tensor] = {}


def _amax_args(x_amax: torch.Tensor | None, rows: int) -> tuple[int, int, int]:
    """(pointer, partial maxima per row, row stride) of a producer's amax
    [rows, n] fp32 (n = 1 for an RMSNorm's, the strips for a linear's)."""
    if x_amax is None:
        return 0, 0, 0
    if x_amax.dtype != torch.float32 or x_amax.dim() != 2 or x_amax.shape[0] < rows or x_amax.stride(1) != 1:
        raise ValueError("x_amax must be fp32 [rows, n] with a contiguous last axis")
    return x_amax.data_ptr(), x_amax.shape[1], x_amax.stride(0)


def _partials_buffer(device: torch.device, k_splits: int, rows: int, n: int) -> torch.Tensor:
    """[k_splits, rows, n] fp32 view of the per-device split-partials buffer."""
    need = k_splits * rows * n
    idx = _device_index(device)
    buf = _PARTIALS.get(idx)
    if buf is None or buf.numel() < need:
        if buf is not None:
            _RETIRED.append(buf)
        buf = torch.empty(max(need, SMALL_M_MAX_ROWS * 4096 * 4), device=device, dtype=torch.float32)
        _PARTIALS[idx] = buf
    return buf[:need].view(k_splits, rows, n)


def linear_partials(x: torch.Tensor, weight: torch.Tensor, k_splits: int | None = None, *,
                    weight_scale_inv: torch.Tensor | None = None, quantize_x: int | None = None,
                    x_amax: torch.Tensor | None = None) -> SplitPartials:
    """y = x @ W^T (W [N, K] bf16, or FP8 e4m3fn with ``weight_scale_inv``; no
    bias, at most 16 rows) as fp32 split partials (fdms_linear_small_m epilogue
    3); for FP8 weights the row and column scales travel with them.  The
    partials live in a per-device buffer that the next call overwrites: consume
    them before the next linear_partials call."""
    fp8 = weight.dtype == torch.float8_e4m3fn
    if (weight.dtype != torch.bfloat16 and not fp8) or x.dtype != torch.bfloat16 or x.stride(-1) != 1:
        raise ValueError("linear_partials expects bf16 activations and bf16 or FP8 weights")
    if fp8 and weight_scale_inv is None:
        raise ValueError("FP8 weights need weight_scale_inv")
    qx = (QX_DIVIDE if fp8 else QX_NONE) if quantize_x is None else int(quantize_x)
    if qx not in (QX_NONE, QX_DIVIDE, QX_TORCH):
        raise ValueError(f"quantize_x must be one of 0, 1, 2; got {quantize_x!r}")
    n, k = weight.shape
    rows = x.shape[0]
    if not small_m_supported(rows, k, n) or x.shape[1] != k:
        raise ValueError(f"linear_partials does not support rows={rows}, K={k}, N={n}")
    am_ptr, am_n, am_s = _amax_args(x_amax if qx else None, rows)
    if k_splits is None:
        k_splits = choose_partial_splits(x.device, n // 16, k)
    part = _partials_buffer(x.device, k_splits, rows, n)
    idx = _device_index(x.device)
    sinv = row_scale = None
    if fp8:
        sinv = weight_scale_inv.reshape(-1)
        row_scale = _ROW_SCALES.get(idx)
        if row_scale is None:
            row_scale = torch.empty(SMALL_M_MAX_ROWS, device=x.device, dtype=torch.float32)
            _ROW_SCALES[idx] = row_scale
        row_scale = row_scale[:rows]
    nat.require_cuda(x, weight, what="linear_partials")
    nat.call("fdms_linear_small_m", x.data_ptr(), x.stride(0), rows, k, weight.data_ptr(),
             nat.DT_FP8 if fp8 else nat.DT_BF16, weight.stride(0), nat.ptr(sinv), None, n, PRO_NONE, None, 0.0,
             None, 0, None, 0, qx if fp8 else QX_NONE, EPI_PARTIALS, int(k_splits), part.data_ptr(), None,
             part.data_ptr(), n, am_ptr or None, am_n, am_s, None, nat.ptr(row_scale), nat.DT_BF16, nat.stream())
    return SplitPartials(part, row_scale, sinv)


def linear_residual_stats(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor, f_out: torch.Tensor,
                          ssq_out: torch.Tensor, *, weight_scale_inv: torch.Tensor | None = None,
                          k_splits: int | None = None) -> None:
    """A decode linear finished as the residual add of the RMSNorm that follows
    it (fdms_linear_small_m epilogue 4; layernorm.py:32-40): with v = bf16(x @
    W^T), f_out = fp32(v) + fp32(residual) ([rows, N] fp32), residual becomes
    bf16(f) in place, and ssq_out[rows, N / 16] holds each 16-column strip's
    sum of f^2 -- the statistic linear_norm_stats applies the norm from.  bf16
    activations (no quantisation), no bias."""
    n, k = weight.shape
    rows = x.shape[0]
    fp8 = weight.dtype == torch.float8_e4m3fn
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or x.shape[1] != k:
        raise ValueError("linear_residual_stats expects bf16 activations [rows, K] with a contiguous last axis")
    if (weight.dtype != torch.bfloat16 and not fp8) or (fp8 and weight_scale_inv is None):
        raise ValueError("linear_residual_stats expects bf16 weights, or FP8 with weight_scale_inv")
    if not small_m_supported(rows, k, n):
        raise ValueError(f"linear_residual_stats does not support rows={rows}, K={k}, N={n}")
    strips = n // 16
    # the kernel writes ssq_out[row * strips + strip]: exactly [rows, N/16]
    if (residual.dtype != torch.bfloat16 or residual.shape != (rows, n) or residual.stride(1) != 1
            or f_out.dtype != torch.float32 or f_out.shape != (rows, n) or f_out.stride(1) != 1
            or ssq_out.dtype != torch.float32 or not ssq_out.is_contiguous() or ssq_out.shape != (rows, strips)):
        raise ValueError("linear_residual_stats: residual bf16 [rows, N], f_out fp32 [rows, N], "
                         "ssq_out contiguous fp32 [rows, N/16]")
    if k_splits is None:
        env = os.environ.get("FASTDMS_AMD_RESID_SPLITS", "").strip()  # tuning override
        if env.isdigit() and 1 <= int(env) <= _MAX_K_SPLITS and k % (int(env) * 256) == 0:
            k_splits = int(env)
        else:
            k_splits = choose_k_splits(x.device, strips, k)
    ws = counters = None
    if k_splits > 1:
        ws, counters = linear_workspace(x.device, strips * k_splits * 256, strips)
    sinv = None if weight_scale_inv is None else weight_scale_inv.reshape(-1)
    nat.require_cuda(x, weight, residual, f_out, ssq_out, what="linear_residual_stats")
    nat.call("fdms_linear_small_m", x.data_ptr(), x.stride(0), rows, k, weight.data_ptr(),
             nat.DT_FP8 if fp8 else nat.DT_BF16, weight.stride(0), nat.ptr(sinv), None, n, PRO_NONE, None, 0.0,
             residual.data_ptr(), residual.stride(0), residual.data_ptr(), residual.stride(0), QX_NONE,
             EPI_RESIDUAL_STATS, int(k_splits), nat.ptr(ws), nat.ptr(counters), f_out.data_ptr(), f_out.stride(0),
             None, 0, 0, ssq_out.data_ptr(), None, nat.DT_BF16, nat.stream())


def linear_norm_stats(f: torch.Tensor, ssq: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                      weight_scale_inv: torch.Tensor | None = None, epilogue: int = EPI_NONE,
                      out: torch.Tensor | None = None, k_splits: int | None = None) -> torch.Tensor:
    """y = RMSNorm(f) @ W^T for the fp32 rows f of a linear_residual_stats
    producer (fdms_linear_small_m prologue 2): the norm's rsqrt(mean(f^2) +
    eps) comes from the producer's strip sums ``ssq`` [rows, strips], the
    normalised activation is bf16(bf16(f * rsqrt) * norm_weight) as the
    RMSNorm makes it (layernorm.py:32-40).  epilogue EPI_SILU_MUL: W = [gate;
    up] and the result is SiLU(gate) * up."""
    n, k = weight.shape
    rows = f.shape[0]
    fp8 = weight.dtype == torch.float8_e4m3fn
    if f.dtype != torch.float32 or f.stride(-1) != 1 or f.shape[1] != k:
        raise ValueError("linear_norm_stats expects fp32 rows [rows, K] with a contiguous last axis")
    # every column of ssq is summed into the row's norm: one per producer strip (K / 16)
    if (ssq.dtype != torch.float32 or ssq.dim() != 2 or ssq.shape[0] < rows or ssq.shape[1] != k // 16
            or ssq.stride(1) != 1):
        raise ValueError("ssq must be fp32 [rows, K/16] (the producer's strip sums) with a contiguous last axis")
    if (weight.dtype != torch.bfloat16 and not fp8) or (fp8 and weight_scale_inv is None):
        raise ValueError("linear_norm_stats expects bf16 weights, or FP8 with weight_scale_inv")
    if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != k or not norm_weight.is_contiguous():
        raise ValueError("norm_weight must be contiguous bf16 [K]")
    if epilogue not in (EPI_NONE, EPI_SILU_MUL):
        raise ValueError(f"linear_norm_stats: epilogue {epilogue} is not supported")
    n_out = n // 2 if epilogue == EPI_SILU_MUL else n
    if not small_m_supported(rows, k, n_out) or (epilogue == EPI_SILU_MUL and n % 2):
        raise ValueError(f"linear_norm_stats does not support rows={rows}, K={k}, N={n}")
    if out is None:
        out = torch.empty((rows, n_out), device=f.device, dtype=torch.bfloat16)
    strips = n_out // 16
    if k_splits is None:
        env = os.environ.get("FASTDMS_AMD_NORM_SPLITS", "").strip()  # tuning override
        if env.isdigit() and 1 <= int(env) <= _MAX_K_SPLITS and k % (int(env) * 256) == 0:
            k_splits = int(env)
        else:
            k_splits = choose_k_splits(f.device, strips, k)
    ws = counters = None
    if k_splits > 1:
        ws, counters = linear_workspace(f.device, strips * k_splits * 256 * (2 if epilogue else 1), strips)
    sinv = None if weight_scale_inv is None else weight_scale_inv.reshape(-1)
    nat.require_cuda(f, ssq, weight, norm_weight, out, what="linear_norm_stats")
    nat.call("fdms_linear_small_m", f.data_ptr(), f.stride(0), rows, k, weight.data_ptr(),
             nat.DT_FP8 if fp8 else nat.DT_BF16, weight.stride(0), nat.ptr(sinv), nat.ptr(bias), n, PRO_NORM_STATS,
             norm_weight.data_ptr(), float(eps), None, 0, None, 0, QX_NONE, int(epilogue), int(k_splits),
             nat.ptr(ws), nat.ptr(counters), out.data_ptr(), out.stride(0), ssq.data_ptr(), ssq.shape[1],
             ssq.stride(0), None, None, nat.DT_F32, nat.stream())
    return out


def linear_workspace(device: torch.device, n_floats: int, n_counters: int):
    idx = _device_index(device)
    entry = _WS.setdefault(idx, [None, None])
    if entry[0] is None or entry[0].numel() < n_floats:
        if entry[0] is not None:
            _RETIRED.append(entry[0])
        entry[0] = torch.empty(max(n_floats, 1), device=device, dtype=torch.float32)
    if entry[1] is None or entry[1].numel() < n_counters:
        if entry[1] is not None:
            _RETIRED.append(entry[1])
        entry[1] = torch.zeros(max(n_counters, 1), device=device, dtype=torch.int32)
    return entry[0], entry[1]


def reserve_linear_workspace(device: torch.device, max_out_features: int) -> None:
    """Size the split-K workspace (and the split-partials buffer) for any
    linear of at most max_out_features output columns (call before graph
    capture)."""
    idx = _device_index(device)
    need = _MAX_K_SPLITS * SMALL_M_MAX_ROWS * max_out_features
    if idx not in _PARTIALS or _PARTIALS[idx].numel() < need:
        if idx in _PARTIALS:
            _RETIRED.append(_PARTIALS[idx])
        _PARTIALS[idx] = torch.empty(need, device=device, dtype=torch.float32)
    strips = max_out_features // 16
    linear_workspace(device, strips * _MAX_K_SPLITS * 512, strips)


def quantize_fp8_rows(x: torch.Tensor, out: torch.Tensor | None = None, scale_inv: torch.Tensor | None = None,
                      *, torch_form: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row FP8 quantisation: (e4m3fn rows, scale_inv [rows] fp32) with
    s = 448/amax(row) (1 for an all-zero row), rows = fp8(x * s), scale_inv = 1/s
    (linear.py:386-388, 813-823; the activation form 514-523, 652-654, 683-694).
    torch_form rounds 448/amax as the reference's torch expressions do
    (reciprocal then multiply); False divides directly like its Triton kernels."""
    if x.dim() != 2 or x.stride(1) != 1 or x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("quantize_fp8_rows expects bf16/fp32 rows with a contiguous last axis")
    rows, k = x.shape
    if out is None:
        out = torch.empty((rows, k), device=x.device, dtype=torch.float8_e4m3fn)
    if scale_inv is None:
        scale_inv = torch.empty(rows, device=x.device, dtype=torch.float32)
    nat.require_cuda(x, out, scale_inv, what="quantize_fp8_rows")
    nat.call("fdms_quantize_fp8_rows", x.data_ptr(), nat.dtype_code(x.dtype), x.stride(0), rows, k, out.data_ptr(),
             out.stride(0), scale_inv.data_ptr(), int(bool(torch_form)), nat.stream())
    return out, scale_inv


def linear_small_m(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                   weight_scale_inv: torch.Tensor | None = None, prologue: int = PRO_NONE,
                   norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                   residual: torch.Tensor | None = None, residual_out: torch.Tensor | None = None,
                   quantize_x: bool | int | None = None, epilogue: int = EPI_NONE, k_splits: int | None = None,
                   out: torch.Tensor | None = None, x_amax: torch.Tensor | None = None,
                   amax_out: torch.Tensor | None = None) -> torch.Tensor:
    """y = a @ W^T for at most 16 rows.  ``weight`` is [N, K] bf16, or FP8
    e4m3fn with ``weight_scale_inv`` [N] (or [1, N]).  ``a`` is x, or RMSNorm of
    x (+ residual) with ``norm_weight`` (prologue 1; the bf16 sum goes to
    ``residual_out``).  epilogue 1: W = [gate; up] and the result is
    silu(gate) * up, [rows, N/2].  quantize_x: QX_DIVIDE (True; the default for
    FP8 weights, the row-1 / small-M kernels), QX_TORCH (_fp8_linear's form) or
    QX_NONE (False).  ``x_amax`` [rows, n]: x's row amax as partial maxima from
    its producer (used with activation quantisation and no prologue; same
    result, no pass over x).  ``amax_out`` [rows, N_out/16] receives the
    per-strip max |y| for an FP8 consumer of y."""
    if weight.dim() != 2:
        raise ValueError("weight must be [out_features, in_features]")
    n, k = weight.shape
    rows = x.shape[0]
    fp8 = weight.dtype == torch.float8_e4m3fn
    x_fp8 = x.dtype == torch.float8_e4m3fn   # codes its producer quantised with x_amax
    if (x.dtype != torch.bfloat16 and not x_fp8) or x.stride(-1) != 1:
        raise ValueError("linear_small_m expects bf16 (or pre-quantised e4m3fn) activations with a contiguous "
                         "last axis")
    if x_fp8 and (not fp8 or x_amax is None or prologue != PRO_NONE or quantize_x in (False, QX_NONE)):
        raise ValueError("e4m3fn activations need FP8 weights, x_amax and activation quantisation")
    if fp8 and weight_scale_inv is None:
        raise ValueError("FP8 weights need weight_scale_inv")
    if not fp8 and weight.dtype != torch.bfloat16:
        raise ValueError(f"unsupported weight dtype {weight.dtype}")
    n_out = n // 2 if epilogue == EPI_SILU_MUL else n
    if not small_m_supported(rows, k, n_out) or (epilogue == EPI_SILU_MUL and n % 2):
        raise ValueError(f"linear_small_m does not support rows={rows}, K={k}, N={n}")
    if x.shape[1] != k:
        raise ValueError(f"activation width {x.shape[1]} does not match K={k}")
    qx = (QX_DIVIDE if fp8 else QX_NONE) if quantize_x is None else int(quantize_x)
    if qx not in (QX_NONE, QX_DIVIDE, QX_TORCH):
        raise ValueError(f"quantize_x must be one of 0, 1, 2; got {quantize_x!r}")
    if out is None:
        out = torch.empty((rows, n_out), device=x.device, dtype=torch.bfloat16)
    strips = n_out // 16
    if k_splits is None:
        k_splits = choose_k_splits(x.device, strips, k)
    ws = counters = None
    if k_splits > 1:
        ws, counters = linear_workspace(x.device, strips * k_splits * 256 * (2 if epilogue else 1), strips)
    sinv = None if weight_scale_inv is None else weight_scale_inv.reshape(-1)
    am_ptr, am_n, am_s = _amax_args(x_amax if (qx and prologue == PRO_NONE) else None, rows)
    if amax_out is not None and (amax_out.dtype != torch.float32 or not amax_out.is_contiguous()
                                 or amax_out.numel() < rows * strips):
        raise ValueError("amax_out must be contiguous fp32 [rows, N_out/16]")
    nat.require_cuda(x, weight, out, what="linear_small_m")
    nat.call("fdms_linear_small_m", x.data_ptr(), x.stride(0), rows, k, weight.data_ptr(),
             nat.DT_FP8 if fp8 else nat.DT_BF16, weight.stride(0), nat.ptr(sinv), nat.ptr(bias), n, int(prologue),
             nat.ptr(norm_weight), float(eps), nat.ptr(residual), 0 if residual is None else residual.stride(0),
             nat.ptr(residual_out), 0 if residual_out is None else residual_out.stride(0), qx,
             int(epilogue), int(k_splits), nat.ptr(ws), nat.ptr(counters), out.data_ptr(), out.stride(0),
             am_ptr or None, am_n, am_s, nat.ptr(amax_out), None, nat.DT_FP8 if x_fp8 else nat.DT_BF16,
             nat.stream())
    return out


def linear_argmax_small_m(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                          weight_scale_inv: torch.Tensor | None = None, quantize_x: bool | int | None = None,
                          bf16_scores: bool | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy head for at most 16 rows: int64 token ids argmax_n (x @ W^T)[m, n]
    in torch.argmax order.  bf16 weights score bf16 logits (F.linear + argmax).
    FP8 weights score the x-quantised products in fp32 (the row-1 argmax,
    embed_head.py:96-211; the default), or with ``bf16_scores`` as the bf16
    logits of forward() (quantize_x=QX_TORCH for its _fp8_linear)."""
    n, k = weight.shape
    rows = x.shape[0]
    fp8 = weight.dtype == torch.float8_e4m3fn
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or x.shape[1] != k:
        raise ValueError("linear_argmax_small_m expects bf16 activations [rows, K] with a contiguous last axis")
    if fp8 and weight_scale_inv is None:
        raise ValueError("FP8 weights need weight_scale_inv")
    if not small_m_supported(rows, k, n):
        raise ValueError(f"linear_argmax_small_m does not support rows={rows}, K={k}, N={n}")
    qx = (QX_DIVIDE if fp8 else QX_NONE) if quantize_x is None else int(quantize_x)
    if qx not in (QX_NONE, QX_DIVIDE, QX_TORCH):
        raise ValueError(f"quantize_x must be one of 0, 1, 2; got {quantize_x!r}")
    if bf16_scores is None:
        bf16_scores = not fp8
    strips = n // 16
    k_splits = choose_k_splits(x.device, strips, k)
    ws = counters = None
    if k_splits > 1:
        ws, counters = linear_workspace(x.device, strips * k_splits * 256, strips)
    part_val = torch.empty((rows, strips), device=x.device, dtype=torch.float32)
    part_idx = torch.empty((rows, strips), device=x.device, dtype=torch.int32)
    if out is None:
        out = torch.empty(rows, device=x.device, dtype=torch.int64)
    sinv = None if weight_scale_inv is None else weight_scale_inv.reshape(-1)
    nat.require_cuda(x, weight, out, what="linear_argmax_small_m")
    nat.call("fdms_linear_argmax_small_m", x.data_ptr(), x.stride(0), rows, k, weight.data_ptr(),
             nat.DT_FP8 if fp8 else nat.DT_BF16, weight.stride(0), nat.ptr(sinv), nat.ptr(bias), n,
             qx, int(bool(bf16_scores)), int(k_splits), nat.ptr(ws), nat.ptr(counters), part_val.data_ptr(),
             part_idx.data_ptr(), out.data_ptr(), nat.stream())
    return out


def quantize_int4_groups(w: torch.Tensor, group_size: int, mode: str = "symmetric"):
    """INT4 group quantisation of weight rows [N, K] (linear.py:414-459).
    Returns (packed [N, K/2] uint8: q[2j] low nibble, q[2j+1] high nibble,
    scale_zeros [K/group, N, 2] bf16: the reference's layout, linear.py:461-464,
    scale in [..., 0], zero in [..., 1]); dequant (q - 8) * scale + zero."""
    mode = mode.strip().lower()
    if mode not in {"sym", "symmetric", "asym", "asymmetric", "affine"}:
        raise ValueError("int4 quant_mode must be symmetric or asymmetric")
    if w.dim() != 2 or w.stride(1) != 1 or w.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("quantize_int4_groups expects bf16/fp32 rows with a contiguous last axis")
    n, k = w.shape
    if group_size not in (32, 64, 128, 256) or k % group_size:
        raise ValueError(f"group size {group_size} must be one of 32/64/128/256 and divide K={k}")
    packed = torch.empty((n, k // 2), device=w.device, dtype=torch.uint8)
    scale_zeros = torch.empty((k // group_size, n, 2), device=w.device, dtype=torch.bfloat16)
    nat.require_cuda(w, what="quantize_int4_groups")
    nat.call("fdms_quantize_int4_groups", w.data_ptr(), nat.dtype_code(w.dtype), w.stride(0), n, k, group_size,
             int(mode in {"asym", "asymmetric", "affine"}), packed.data_ptr(), packed.stride(0),
             scale_zeros.data_ptr(), n, nat.stream())
    return packed, scale_zeros


def linear_int4_small_m(x: torch.Tensor, packed: torch.Tensor, scale_zeros: torch.Tensor, group_size: int,
                        bias: torch.Tensor | None = None, *, epilogue: int = EPI_NONE,
                        out: torch.Tensor | None = None, greedy: bool = False,
                        k_splits: int | None = None) -> torch.Tensor:
    """W4A16 for at most 16 rows (linear.py:462-478 semantics): y = x @
    dequant(W)^T, or SiLU*up (epilogue 1), or greedy token ids (greedy=True);
    scale_zeros is bf16 [K/group, N, 2] (the reference's layout)."""
    n, k = packed.shape[0], packed.shape[1] * 2
    rows = x.shape[0]
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or x.shape[1] != k:
        raise ValueError("linear_int4_small_m expects bf16 activations [rows, K]")
    if (scale_zeros.dtype != torch.bfloat16 or scale_zeros.shape != (k // group_size, n, 2)
            or not scale_zeros.is_contiguous()):
        raise ValueError("scale_zeros must be contiguous bf16 [K/group, N, 2]")
    n_out = n // 2 if epilogue == EPI_SILU_MUL else n
    if not small_m_supported(rows, k, n_out):
        raise ValueError(f"linear_int4_small_m does not support rows={rows}, K={k}, N={n}")
    strips = n_out // 16
    if k_splits is None:
        k_splits = choose_k_splits(x.device, strips, k)
    ws = counters = None
    if k_splits > 1:
        ws, counters = linear_workspace(x.device, strips * k_splits * 256 * (2 if epilogue else 1), strips)
    pv = pi = tok = None
    if greedy:
        pv = torch.empty((rows, strips), device=x.device, dtype=torch.float32)
        pi = torch.empty((rows, strips), device=x.device, dtype=torch.int32)
        tok = out if out is not None else torch.empty(rows, device=x.device, dtype=torch.int64)
        y = None
    else:
        y = out if out is not None else torch.empty((rows, n_out), device=x.device, dtype=torch.bfloat16)
    nat.require_cuda(x, packed, scale_zeros, what="linear_int4_small_m")
    nat.call("fdms_linear_int4_small_m", x.data_ptr(), x.stride(0), rows, k, packed.data_ptr(), packed.stride(0),
             scale_zeros.data_ptr(), int(group_size), n, nat.ptr(bias), n,
             2 if greedy else int(epilogue), int(k_splits), nat.ptr(ws), nat.ptr(counters), nat.ptr(pv), nat.ptr(pi),
             nat.ptr(tok), nat.ptr(y), 0 if y is None else y.stride(0), nat.stream())
    return tok if greedy else y


def linear_int4_partials(x: torch.Tensor, packed: torch.Tensor, scale_zeros: torch.Tensor, group_size: int,
                         k_splits: int | None = None) -> SplitPartials:
    """W4A16 y = x @ dequant(W)^T (no bias, at most 16 rows) as fp32 split
    partials (fdms_linear_int4_small_m epilogue 3) for the next RMSNorm to sum,
    in the same per-device buffer as linear_partials (consume before the next
    call)."""
    n, k = packed.shape[0], packed.shape[1] * 2
    rows = x.shape[0]
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or x.shape[1] != k:
        raise ValueError("linear_int4_partials expects bf16 activations [rows, K]")
    if (scale_zeros.dtype != torch.bfloat16 or scale_zeros.shape != (k // group_size, n, 2)
            or not scale_zeros.is_contiguous()):
        raise ValueError("scale_zeros must be contiguous bf16 [K/group, N, 2]")
    if not small_m_supported(rows, k, n):
        raise ValueError(f"linear_int4_partials does not support rows={rows}, K={k}, N={n}")
    if k_splits is None:
        k_splits = choose_partial_splits(x.device, n // 16, k)
    part = _partials_buffer(x.device, k_splits, rows, n)
    nat.require_cuda(x, packed, scale_zeros, what="linear_int4_partials")
    nat.call("fdms_linear_int4_small_m", x.data_ptr(), x.stride(0), rows, k, packed.data_ptr(), packed.stride(0),
             scale_zeros.data_ptr(), int(group_size), n, None, n, EPI_PARTIALS, int(k_splits), part.data_ptr(),
             None, None, None, None, None, 0, nat.stream())
    return SplitPartials(part)


def fp8_gemm_impl() -> str:
    """The FP8 GEMM of prefill row counts: "hipblaslt" (default; torch's
    _scaled_mm with row-wise scales, the call the reference makes in
    _fp8_linear, linear.py:652-659: a plain library GEMM, 1.8-2.2 PFLOP/s at
    the Llama-3.2-1B prefill shapes on MI355X) or "fdms" (fdms_fp8_gemm, this
    library's FP8 matrix-core kernel, 0.6-0.8 PFLOP/s there).
    FASTDMS_AMD_FP8_GEMM selects; shapes hipBLASLt does not take (K or N not
    multiples of 16) run fdms_fp8_gemm, row counts are padded to 16."""
    impl = os.environ.get("FASTDMS_AMD_FP8_GEMM", "hipblaslt").strip().lower()
    if impl not in ("hipblaslt", "fdms"):
        raise ValueError(f"FASTDMS_AMD_FP8_GEMM must be 'hipblaslt' or 'fdms', got {impl!r}")
    return impl


def fp8_gemm(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale_inv: torch.Tensor,
             bias: torch.Tensor | None = None, *, torch_form: bool = True,
             out: torch.Tensor | None = None, impl: str | None = None) -> torch.Tensor:
    """_fp8_linear for prefill row counts on the FP8 matrix cores
    (linear.py:635-662): rows quantised per row (fdms_quantize_fp8_rows), then
    y = bf16(sum_k xq * w8 * x_scale_inv * w_scale_inv) with fp32 accumulation
    (fp8_gemm_impl: hipBLASLt's scaled GEMM or fdms_fp8_gemm), bias added in
    bf16.  x [M, K] bf16 / fp32, weight_fp8 [N, K] e4m3fn, K a multiple of
    16."""
    if x.dim() != 2 or weight_fp8.dim() != 2 or x.shape[1] != weight_fp8.shape[1]:
        raise ValueError(f"fp8_gemm shape mismatch: x {tuple(x.shape)}, weight {tuple(weight_fp8.shape)}")
    rows, k = x.shape
    n = weight_fp8.shape[0]
    if k % 16 or weight_fp8.stride(1) != 1 or weight_fp8.stride(0) % 16 or weight_fp8.data_ptr() % 16:
        raise ValueError("fp8_gemm needs K a multiple of 16 and 16-byte aligned weight rows")
    nat.require_cuda(x, weight_fp8, weight_scale_inv, what="fp8_gemm")
    sinv = weight_scale_inv.reshape(-1).float().contiguous()
    if sinv.numel() != n:
        raise ValueError(f"weight_scale_inv has {sinv.numel()} entries for {n} rows")
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    impl = impl or fp8_gemm_impl()
    if impl == "hipblaslt" and n % 16 == 0 and k % 16 == 0 and out is None:
        # hipBLASLt takes row counts in multiples of 16: the quantised rows
        # are padded with zero rows (scale 1), whose outputs are dropped
        rows16 = -(-rows // 16) * 16
        xq = torch.empty((rows16, k), device=x.device, dtype=torch.float8_e4m3fn)
        xsi = torch.empty(rows16, device=x.device, dtype=torch.float32)
        if rows16 > rows:
            xq[rows:].view(torch.uint8).zero_()
            xsi[rows:].fill_(1.0)
        quantize_fp8_rows(x.contiguous(), out=xq[:rows], scale_inv=xsi[:rows], torch_form=torch_form)
        y = torch._scaled_mm(xq, weight_fp8.t(), scale_a=xsi.reshape(-1, 1), scale_b=sinv.reshape(1, -1),
                             out_dtype=torch.bfloat16, use_fast_accum=False)[:rows]
        return y if b is None else y + b
    xq, xsi = quantize_fp8_rows(x.contiguous(), torch_form=torch_form)
    if out is None:
        out = torch.empty((rows, n), device=x.device, dtype=torch.bfloat16)
    nat.call("fdms_fp8_gemm", xq.data_ptr(), xq.stride(0), xsi.data_ptr(), weight_fp8.data_ptr(),
             weight_fp8.stride(0), sinv.data_ptr(), nat.ptr(b), out.data_ptr(), out.stride(0), rows, n, k,
             nat.stream())
    return out


def fp8_rows_gemm(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale_inv: torch.Tensor,
                  bias: torch.Tensor | None, quantize_x: int) -> torch.Tensor:
    """FP8 linear for any row count, the reference's _fp8_linear semantics
    (linear.py:635-662; QX_TORCH) or its Triton kernels' (QX_DIVIDE / QX_NONE):
    y = bf16(sum_k xq*w8 / x_s * scale_inv), bias added in bf16.  Rows <= 16 of a
    supported shape run fdms_linear_small_m; larger row counts run fp8_gemm (the
    FP8 matrix cores).  Unquantised activations (QX_NONE) or K not a multiple
    of 16 multiply the decoded FP8 values in fp32 with torch."""
    rows, k = x.shape
    n = weight_fp8.shape[0]
    if small_m_supported(rows, k, n):
        return linear_small_m(x.contiguous(), weight_fp8, bias, weight_scale_inv=weight_scale_inv,
                              quantize_x=quantize_x)
    if quantize_x != QX_NONE and k % 16 == 0:
        return fp8_gemm(x, weight_fp8, weight_scale_inv, bias, torch_form=quantize_x == QX_TORCH)
    sinv = weight_scale_inv.reshape(1, -1).float()
    w = weight_fp8.float()
    if quantize_x == QX_NONE:
        acc = x.float() @ w.t()
    else:
        xq, xsi = quantize_fp8_rows(x.contiguous(), torch_form=quantize_x == QX_TORCH)
        acc = (xq.float() @ w.t()) * xsi.reshape(-1, 1)
    y = (acc * sinv).to(torch.bfloat16)
    return y if bias is None else y + bias.to(torch.bfloat16)


class LinearBase(nn.Module):
    """Weights [out_features, in_features] bf16, optionally shadowed or replaced
    by FP8 rows (``weight_fp8`` [N, K] = the reference's column-major
    ``weight_fp8_t``, ``weight_scale_inv`` [1, N]) and INT4 groups
    (``weight_int4`` [N, K/2], ``weight_int4_scale_zeros`` [K/group, N, 2], the
    reference's name and layout)."""

    def __init__(self, input_size: int, output_size: int, bias: bool = False):
        super().__init__()
        self.input_size = input_size
        self.output_size = output_size
        self.weight = nn.Parameter(torch.empty(output_size, input_size), requires_grad=False)
        if bias:
            self.bias = nn.Parameter(torch.zeros(output_size), requires_grad=False)
        else:
            self.register_parameter("bias", None)
        self._fp8_weight_enabled = False
        self._fp8_module_name = ""
        self._fp8_row1_only = False
        self._fp8_min_rows = 1
        self._int4_enabled = False
        self._int4_group_size = 0

    # -- weight conversion ----------------------------------------------------
    def quantize_weight_to_fp8(self, *, keep_bf16_weight: bool = False, module_name: str | None = None,
                               row1_only: bool = False) -> None:
        """linear.py:813-847: per-output-channel FP8 weights, plus the INT4
        shadow when FASTDMS_INT4_ROW1_WEIGHTS is on and the module is in
        FASTDMS_INT4_ROW1_SCOPE (829-836)."""
        if row1_only and not keep_bf16_weight:
            raise ValueError("row1-only FP8 shadow requires keeping the BF16 weight")
        w8, sinv = quantize_fp8_rows(self.weight.detach())
        self._set_buffer("weight_fp8", w8)
        self._set_buffer("weight_scale_inv", sinv.reshape(1, -1))
        if qe.int4_weights_enabled() and qe.int4_module_in_scope(module_name):
            self.quantize_weight_to_int4()
        self._fp8_min_rows = qe.fp8_module_min_rows(module_name)
        self._fp8_module_name = module_name or ""
        if not keep_bf16_weight:
            self._drop_bf16_weight()
        self._fp8_weight_enabled = True
        self._fp8_row1_only = bool(row1_only)

    def quantize_weight_to_int4(self, *, group_size: int | None = None, mode: str | None = None) -> bool:
        """The INT4 row-1 shadow (linear.py:414-459) with FASTDMS_INT4_ROW1_GROUP_SIZE /
        _QUANT_MODE by default.  Like the reference it is skipped (False) for a
        shape the INT4 kernel does not take."""
        group = qe.int4_group_size() if group_size is None else int(group_size)
        mode = qe.int4_quant_mode() if mode is None else mode
        k, n = self.input_size, self.output_size
        if self.weight.numel() == 0 or k % group or not small_m_supported(1, k, n):
            return False
        packed, scale_zeros = quantize_int4_groups(self.weight.detach(), group, mode)
        self._set_buffer("weight_int4", packed)
        self._set_buffer("weight_int4_scale_zeros", scale_zeros)
        self._int4_group_size = group
        self._int4_enabled = True
        return True

    def _set_buffer(self, name: str, value: torch.Tensor) -> None:
        if name in self._buffers:
            self._buffers[name] = value
        else:
            self.register_buffer(name, value, persistent=False)

    def _drop_bf16_weight(self) -> None:
        dev = self.weight.device
        del self._parameters["weight"]
        self.register_buffer("weight", torch.empty(0, device=dev, dtype=torch.bfloat16), persistent=False)

    @property
    def weight_fp8_t(self) -> torch.Tensor:
        return self.weight_fp8.t()

    # -- dispatch ---------------------------------------------------------------
    def _row1_mode(self) -> str:
        """linear.py:860-868: the module's row-1 kernel mode."""
        name = self._fp8_module_name
        if name.endswith(".down_proj") and self.weight.numel() == 0:
            return qe.fp8_down_row1_mode()
        if name.endswith(".gate_up_proj"):
            return qe.fp8_gate_up_row1_mode()
        if ".self_attn." in name:
            return qe.fp8_attention_row1_mode()
        return qe.fp8_row1_mode()

    def route(self, rows: int) -> tuple[str, int]:
        """(path, activation quantisation) for a call of ``rows`` rows, in the
        reference's order (linear.py:855-926): "int4" (rows <= the INT4 row
        limit, row-1 mode on), "fp8" row 1 (mode on; quantised or raw
        activation), "bf16" for a row-1-only shadow, "fp8" small-M (2 <= rows <=
        FASTDMS_FP8_SMALL_M_TRITON_MAX_ROWS, N % 16 == 0) or "fp8" _fp8_linear
        (QX_TORCH) once rows >= the module's FP8 minimum or the bf16 weight is
        gone ("fp8_dequant" when FASTDMS_FP8_LINEAR_IMPL=dequant or K % 16), else "bf16"."""
        if not self._fp8_weight_enabled:
            return "bf16", QX_NONE
        mode = self._row1_mode()
        if self._int4_enabled and 1 <= rows <= qe.int4_max_rows() and mode != "off":
            return "int4", QX_NONE
        if rows == 1 and mode != "off":
            return "fp8", QX_DIVIDE if mode == "quantized" else QX_NONE
        if self._fp8_row1_only:
            return "bf16", QX_NONE
        if self.weight.numel() == 0 or rows >= self._fp8_min_rows:
            if (qe.fp8_small_m_enabled() and 1 < rows <= qe.fp8_small_m_max_rows()
                    and self.output_size % 16 == 0):
                return "fp8", QX_DIVIDE
            if (os.environ.get("FASTDMS_FP8_LINEAR_IMPL", "").strip().lower() == "dequant"
                    or self.input_size % 16):
                return "fp8_dequant", QX_NONE
            return "fp8", QX_TORCH
        return "bf16", QX_NONE

    def small_m_fused(self, rows: int, epilogue: int = EPI_NONE) -> bool:
        """True when a call of ``rows`` rows runs fdms_linear_small_m (bf16 or
        FP8 route on a supported shape; contiguous rows assumed)."""
        n_out = self.output_size // 2 if epilogue == EPI_SILU_MUL else self.output_size
        return self.route(rows)[0] in ("bf16", "fp8") and small_m_supported(rows, self.input_size, n_out)

    def x_quant_mode(self, rows: int) -> int:
        """The activation quantisation (QX_DIVIDE / QX_TORCH) when this linear
        quantises its activation on the small-M kernel -- its producer may then
        hand over the row amax, or the quantised codes -- else QX_NONE."""
        path, qx = self.route(rows)
        if path == "fp8" and small_m_supported(rows, self.input_size, self.output_size):
            return qx
        return QX_NONE

    def wants_x_amax(self, rows: int) -> bool:
        return self.x_quant_mode(rows) != QX_NONE

    def run_quantized(self, xq: torch.Tensor, x_amax: torch.Tensor, *, epilogue: int = EPI_NONE,
                      amax_out: torch.Tensor | None = None) -> torch.Tensor:
        """The small-M FP8 path on an activation its producer already quantised
        (e4m3fn codes ``xq`` with the row amax ``x_amax``, as rms_norm's q_out
        with q_mode = x_quant_mode(rows))."""
        qx = self.x_quant_mode(xq.shape[0])
        if qx == QX_NONE:
            raise ValueError("run_quantized needs the small-M FP8 route with activation quantisation")
        return linear_small_m(xq, self.weight_fp8, self.bias, weight_scale_inv=self.weight_scale_inv, quantize_x=qx,
                              epilogue=epilogue, x_amax=x_amax, amax_out=amax_out)

    def run(self, x2: torch.Tensor, bias: torch.Tensor | None, *, epilogue: int = EPI_NONE,
            route: tuple[str, int] | None = None, x_amax: torch.Tensor | None = None,
            amax_out: torch.Tensor | None = None) -> torch.Tensor:
        """Execute ``route`` (default: self.route) on rows x2 [rows, K].  With
        epilogue EPI_SILU_MUL the weight is [gate; up] and the result is the
        SiluAndMul of the linear's output (fused into the decode kernels).
        ``x_amax`` / ``amax_out`` as linear_small_m (small-M paths only;
        amax_out on another path is an error)."""
        rows = x2.shape[0]
        path, qx = self.route(rows) if route is None else route
        n_out = self.output_size // 2 if epilogue == EPI_SILU_MUL else self.output_size
        fused = small_m_supported(rows, self.input_size, n_out) and x2.stride(-1) == 1
        if amax_out is not None and not (fused and path in ("fp8", "bf16")):
            raise ValueError("amax_out needs the small-M kernel path")
        if path == "int4":
            return linear_int4_small_m(x2.contiguous(), self.weight_int4, self.weight_int4_scale_zeros,
                                       self._int4_group_size, bias, epilogue=epilogue)
        if path == "fp8" and fused:
            return linear_small_m(x2.contiguous(), self.weight_fp8, bias, weight_scale_inv=self.weight_scale_inv,
                                  quantize_x=qx, epilogue=epilogue, x_amax=x_amax, amax_out=amax_out)
        if path == "bf16" and fused:
            return linear_small_m(x2, self.weight, bias, epilogue=epilogue, amax_out=amax_out)
        if path == "fp8":
            y = fp8_rows_gemm(x2, self.weight_fp8, self.weight_scale_inv, bias, qx)
        elif path == "fp8_dequant":  # linear.py:645-647: the weight dequantised in the activation dtype
            w = (self.weight_fp8.to(x2.dtype) * self.weight_scale_inv.reshape(-1, 1).to(x2.dtype))
            y = F.linear(x2, w, bias)
        else:
            y = F.linear(x2, self.weight, bias)
        if epilogue == EPI_SILU_MUL:
            g, u = y.float().chunk(2, -1)
            y = (F.silu(g) * u).to(y.dtype)
        return y

    def int4_applies(self, rows: int) -> bool:
        return self.route(rows)[0] == "int4"

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        """Dispatch (linear.py:855-926) through ``route``."""
        y = self.run(x.reshape(-1, x.shape[-1]), bias)
        return y.reshape(*x.shape[:-1], self.output_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._linear(x, self.bias)


class ReplicatedLinear(LinearBase):
    pass


class ColumnParallelLinear(LinearBase):
    pass


class MergedColumnParallelLinear(ColumnParallelLinear):
    def __init__(self, input_size: int, output_sizes: list[int], bias: bool = False):
        self.output_sizes = output_sizes
        super().__init__(input_size, sum(output_sizes), bias=bias)


class QKVParallelLinear(ColumnParallelLinear):
    def __init__(self, hidden_size: int, head_size: int, total_num_heads: int, total_num_kv_heads: int | None = None,
                 bias: bool = False):
        self.head_size = head_size
        self.total_num_heads = total_num_heads
        self.total_num_kv_heads = total_num_kv_heads or total_num_heads
        out = (self.total_num_heads + 2 * self.total_num_kv_heads) * head_size
        super().__init__(hidden_size, out, bias=bias)


class RowParallelLinear(LinearBase):
    pass


def convert_linear_modules_to_fp8(module: nn.Module) -> int:
    """linear.py:1076-1095: FP8 weights for every LinearBase in
    FASTDMS_FP8_WEIGHT_SCOPE, attention modules as a row-1-only shadow
    (FASTDMS_FP8_ATTENTION_ROW1_SHADOW) unless FASTDMS_FP8_ATTENTION_FULL;
    returns the number of converted modules."""
    scope = qe.fp8_weight_scope()
    shadow = qe.fp8_attention_row1_shadow_enabled()
    full = qe.fp8_attention_full_enabled()
    converted = 0
    for name, child in module.named_modules():
        # the LM head is not a LinearBase in the reference (embed_head.py:450):
        # it is converted only by FASTDMS_FP8_LM_HEAD (model_runner.py:76-93)
        if not isinstance(child, LinearBase) or getattr(child, "is_lm_head", False):
            continue
        is_attn = ".self_attn." in name
        use_shadow = shadow and is_attn and not full
        force_full = full and is_attn
        if not use_shadow and not force_full and not qe.fp8_module_in_scope(name, scope):
            continue
        keep = True if use_shadow else qe.fp8_module_keep_bf16_weight(name)
        child.quantize_weight_to_fp8(keep_bf16_weight=keep, module_name=name, row1_only=use_shadow)
        converted += 1
    return converted
