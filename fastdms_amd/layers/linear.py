"""Linear layers (mirror of fastdms/layers/linear.py class names, single GPU).

Decode-shaped calls (at most 16 rows) run the HIP kernel
``fdms_linear_small_m`` for bf16 or FP8 weights, optionally with a fused
RMSNorm(+residual) or SiLU*up prologue.  Larger row counts (prefill) use the
ROCm GEMM library (hipBLASLt through torch) for bf16 weights; FP8 weights are
quantised per output channel by ``fdms_quantize_fp8_rows`` exactly as the
reference's ``quantize_weight_to_fp8`` (linear.py:813-847).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import _native as nat

PRO_NONE, PRO_RMSNORM = 0, 1
EPI_NONE, EPI_SILU_MUL = 0, 1
SMALL_M_MAX_ROWS = 16
_MAX_K_SPLITS = 8


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
    """Size the split-K workspace for any linear of at most max_out_features
    output columns (call before graph capture)."""
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
                   quantize_x: bool | None = None, epilogue: int = EPI_NONE, k_splits: int | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """y = a @ W^T for at most 16 rows.  ``weight`` is [N, K] bf16, or FP8
    e4m3fn with ``weight_scale_inv`` [N] (or [1, N]).  ``a`` is x, or RMSNorm of
    x (+ residual) with ``norm_weight`` (prologue 1; the bf16 sum goes to
    ``residual_out``).  epilogue 1: W = [gate; up] and the result is
    silu(gate) * up, [rows, N/2].  FP8 weights quantise the activation per row
    unless ``quantize_x`` is False."""
    if weight.dim() != 2:
        raise ValueError("weight must be [out_features, in_features]")
    n, k = weight.shape
    rows = x.shape[0]
    fp8 = weight.dtype == torch.float8_e4m3fn
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1:
        raise ValueError("linear_small_m expects bf16 activations with a contiguous last axis")
    if fp8 and weight_scale_inv is None:
        raise ValueError("FP8 weights need weight_scale_inv")
    if not fp8 and weight.dtype != torch.bfloat16:
        raise ValueError(f"unsupported weight dtype {weight.dtype}")
    n_out = n // 2 if epilogue == EPI_SILU_MUL else n
    if not small_m_supported(rows, k, n_out) or (epilogue == EPI_SILU_MUL and n % 2):
        raise ValueError(f"linear_small_m does not support rows={rows}, K={k}, N={n}")
    if x.shape[1] != k:
        raise ValueError(f"activation width {x.shape[1]} does not match K={k}")
    if quantize_x is None:
        quantize_x = fp8
    if out is None:
        out = torch.empty((rows, n_out), device=x.device, dtype=torch.bfloat16)
    strips = n_out // 16
    if k_splits is None:
        k_splits = choose_k_splits(x.device, strips, k)
    ws = counters = None
    if k_splits > 1:
        ws, counters = linear_workspace(x.device, strips * k_splits * 256 * (2 if epilogue else 1), strips)
    sinv = None if weight_scale_inv is None else weight_scale_inv.reshape(-1)
    nat.require_cuda(x, weight, out, what="linear_small_m")
    nat.call("fdms_linear_small_m", x.data_ptr(), x.stride(0), rows, k, weight.data_ptr(),
             nat.DT_FP8 if fp8 else nat.DT_BF16, weight.stride(0), nat.ptr(sinv), nat.ptr(bias), n, int(prologue),
             nat.ptr(norm_weight), float(eps), nat.ptr(residual), 0 if residual is None else residual.stride(0),
             nat.ptr(residual_out), 0 if residual_out is None else residual_out.stride(0), int(bool(quantize_x)),
             int(epilogue), int(k_splits), nat.ptr(ws), nat.ptr(counters), out.data_ptr(), out.stride(0),
             nat.stream())
    return out


def linear_argmax_small_m(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                          weight_scale_inv: torch.Tensor | None = None, quantize_x: bool | None = None,
                          out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy head for at most 16 rows: int64 token ids argmax_n (x @ W^T)[m, n]
    in torch.argmax order.  bf16 weights score bf16 logits (F.linear + argmax);
    FP8 weights score fp32 x-quantised products (embed_head.py:96-211)."""
    n, k = weight.shape
    rows = x.shape[0]
    fp8 = weight.dtype == torch.float8_e4m3fn
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or x.shape[1] != k:
        raise ValueError("linear_argmax_small_m expects bf16 activations [rows, K] with a contiguous last axis")
    if fp8 and weight_scale_inv is None:
        raise ValueError("FP8 weights need weight_scale_inv")
    if not small_m_supported(rows, k, n):
        raise ValueError(f"linear_argmax_small_m does not support rows={rows}, K={k}, N={n}")
    if quantize_x is None:
        quantize_x = fp8
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
             int(bool(quantize_x)), int(k_splits), nat.ptr(ws), nat.ptr(counters), part_val.data_ptr(),
             part_idx.data_ptr(), out.data_ptr(), nat.stream())
    return out


class LinearBase(nn.Module):

    def __init__(self, input_size: int, output_size: int, bias: bool = False):
        super().__init__()
        self.input_size = input_size
        self.output_size = output_size
        self.weight = nn.Parameter(torch.empty(output_size, input_size), requires_grad=False)
        if bias:
            self.bias = nn.Parameter(torch.zeros(output_size), requires_grad=False)
        else:
            self.register_parameter("bias", None)
        self.quant = None
        self._fp8_weight_enabled = False
        self._fp8_module_name = ""

    def quantize_weight_to_fp8(self, *, keep_bf16_weight: bool = False, module_name: str | None = None,
                               row1_only: bool = False) -> None:
        """linear.py:813-847: per-output-channel FP8 weights.  ``weight_fp8``
        is [N, K] row-major, i.e. the reference's column-major ``weight_fp8_t``
        [K, N] (exposed as that view); ``weight_scale_inv`` is [1, N] fp32."""
        if row1_only and not keep_bf16_weight:
            raise ValueError("row1-only FP8 shadow requires keeping the BF16 weight")
        w8, sinv = quantize_fp8_rows(self.weight.detach())
        self.register_buffer("weight_fp8", w8, persistent=False)
        self.register_buffer("weight_scale_inv", sinv.reshape(1, -1), persistent=False)
        if not keep_bf16_weight:
            del self._parameters["weight"]
            self.register_buffer("weight", torch.empty(0, device=w8.device, dtype=torch.bfloat16), persistent=False)
        self._fp8_weight_enabled = True
        self._fp8_row1_only = bool(row1_only)
        self._fp8_module_name = module_name or ""

    @property
    def weight_fp8_t(self) -> torch.Tensor:
        return self.weight_fp8.t()

    def _linear(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        """Dispatch (linear.py:855-926): decode rows -> fdms_linear_small_m (FP8 or
        bf16 weights); prefill rows -> dequantised or bf16 library GEMM."""
        x2 = x.reshape(-1, x.shape[-1])
        rows = x2.shape[0]
        if self._fp8_weight_enabled:
            if small_m_supported(rows, self.input_size, self.output_size):
                y = linear_small_m(x2.contiguous(), self.weight_fp8, bias, weight_scale_inv=self.weight_scale_inv)
                return y.reshape(*x.shape[:-1], self.output_size)
            if self.weight.numel() == 0:
                w = (self.weight_fp8.to(torch.bfloat16) * self.weight_scale_inv.reshape(-1, 1).to(torch.bfloat16))
                return F.linear(x, w, bias)
            return F.linear(x, self.weight, bias)
        if small_m_supported(rows, self.input_size, self.output_size) and x2.stride(-1) == 1:
            y = linear_small_m(x2, self.weight, bias)
            return y.reshape(*x.shape[:-1], self.output_size)
        return F.linear(x, self.weight, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.quant is not None:
            return self.quant(x, self.bias)
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
