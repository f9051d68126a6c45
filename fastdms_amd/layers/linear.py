"""Linear layers (mirror of fastdms/layers/linear.py class names, single GPU).

bf16 weights run through the ROCm GEMM library (hipBLASLt via torch) — plain
dense GEMMs.  FP8 / INT4 weight paths are hand-written HIP kernels in
``fastdms_amd.layers.quant``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


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
        self.quant = None  # set by fastdms_amd.layers.quant.quantize_linear

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.quant is not None:
            return self.quant(x, self.bias)
        return F.linear(x, self.weight, self.bias)


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
