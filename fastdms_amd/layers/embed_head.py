"""Token embedding and LM head (mirror of fastdms/layers/embed_head.py, single GPU).

``ParallelLMHead.forward`` / ``greedy_token_ids`` take the last token of
every prefill sequence (embed_head.py:491-495, 545-549) and pick the kernel
in the reference's order (embed_head.py:491-598): with FP8 weights, one row
uses the INT4 shadow (optionally re-ranked in FP8) or the FP8 row-1 GEMV with
fp32 scores; more rows score the _fp8_linear logits in bf16.  Argmax ties go
to the lowest index (embed_head.py:142, 160).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import _native as nat
from ..utils.context import get_context
from . import quant_env as qe
from .linear import (QX_DIVIDE, QX_TORCH, LinearBase, fp8_rows_gemm, linear_argmax_small_m, linear_int4_small_m,
                     quantize_fp8_rows, small_m_supported)


class VocabParallelEmbedding(nn.Module):
    _fp8_embedding_enabled = False

    def __init__(self, num_embeddings: int, embedding_dim: int):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim), requires_grad=False)
        self._fp8_embedding_weight: torch.Tensor | None = None
        self._fp8_embedding_scale_inv: torch.Tensor | None = None

    def quantize_embedding_to_fp8(self, *, keep_bf16_weight: bool = False) -> None:
        """embed_head.py:379-387: per-row FP8 table, scale_inv [V, 1]."""
        w8, sinv = quantize_fp8_rows(self.weight.detach())
        self._set_fp8_embedding(w8, sinv.reshape(-1, 1), keep_bf16_weight)

    def enable_fp8_embedding_from_lm_head(self, lm_head: "ParallelLMHead", *, keep_bf16_weight: bool = False) -> None:
        """embed_head.py:389-402: share the FP8 head rows as the table."""
        if not getattr(lm_head, "_fp8_weight_enabled", False):
            raise RuntimeError("FP8 embedding sharing requires an FP8-quantized lm_head")
        self._set_fp8_embedding(lm_head.weight_fp8, lm_head.weight_scale_inv.reshape(-1, 1), keep_bf16_weight)

    def _set_fp8_embedding(self, w8: torch.Tensor, sinv: torch.Tensor, keep_bf16_weight: bool) -> None:
        self._fp8_embedding_weight, self._fp8_embedding_scale_inv = w8, sinv
        self._fp8_embedding_dtype = self.weight.dtype if self.weight.numel() else torch.bfloat16
        if not keep_bf16_weight and "weight" in self._parameters:
            dev = self.weight.device
            del self._parameters["weight"]
            self.register_buffer("weight", torch.empty(0, device=dev, dtype=torch.bfloat16), persistent=False)
        self._fp8_embedding_enabled = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._fp8_embedding_enabled:
            # embed_head.py:422-432: fp8 row and its scale_inv, each in bf16,
            # multiplied -- the fdms_embedding_fp8 gather
            if self._fp8_embedding_dtype != torch.bfloat16:
                raise ValueError("the FP8 embedding gather produces bf16 rows")
            flat = x.reshape(-1).to(torch.long).contiguous()
            w8 = self._fp8_embedding_weight
            out = torch.empty((flat.numel(), w8.shape[1]), device=w8.device, dtype=torch.bfloat16)
            nat.require_cuda(flat, w8, out, what="fp8 embedding")
            nat.call("fdms_embedding_fp8", flat.data_ptr(), flat.numel(), w8.data_ptr(), w8.stride(0),
                     self._fp8_embedding_scale_inv.data_ptr(), w8.shape[0], out.data_ptr(), out.stride(0),
                     w8.shape[1], nat.stream())
            return out.reshape(*x.shape, w8.shape[1])
        return F.embedding(x, self.weight)


def embedding_rms_norm(ids: torch.Tensor, table: torch.Tensor, norm_weight: torch.Tensor,
                       eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(RMSNorm(table[ids]), table[ids]) in one launch (fdms_embedding_rmsnorm):
    the decode step's bf16 embedding gather (embed_head.py:87-104) and the
    first decoder layer's input_layernorm without residual (layernorm.py:
    16-28), whose input rows are the step's first residual.  Bit-identical to
    rms_norm(F.embedding(ids, table)); an id outside the table gives NaN rows."""
    if table.dtype != torch.bfloat16 or table.dim() != 2 or table.stride(1) != 1:
        raise ValueError("embedding_rms_norm expects a bf16 [vocab, hidden] table with a contiguous last axis")
    if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != table.shape[1]:
        raise ValueError("norm_weight must be bf16 [hidden]")
    flat = ids.reshape(-1).to(torch.long).contiguous()
    n, hidden = flat.numel(), table.shape[1]
    out = torch.empty((n, hidden), device=table.device, dtype=torch.bfloat16)
    rows = torch.empty((n, hidden), device=table.device, dtype=torch.bfloat16)
    nat.require_cuda(flat, table, norm_weight, what="embedding_rms_norm")
    nat.call("fdms_embedding_rmsnorm", flat.data_ptr(), n, table.data_ptr(), table.stride(0), table.shape[0],
             norm_weight.data_ptr(), float(eps), out.data_ptr(), out.stride(0), rows.data_ptr(), rows.stride(0),
             hidden, nat.stream())
    return out, rows


def fp8_rerank_topk(x: torch.Tensor, candidates: torch.Tensor, weight_fp8: torch.Tensor,
                    weight_scale_inv: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """embed_head.py:214-302: per row, FP8 scores (448/amax activation
    quantisation, fp32) of the candidate token ids; the best candidate, lowest
    id on ties.  candidates [rows, topk] int64, topk in {2, 4, 8, 16, 32}."""
    rows, k = x.shape
    topk = candidates.shape[1]
    if topk not in (2, 4, 8, 16, 32):
        raise ValueError(f"topk must be one of 2, 4, 8, 16, 32, got {topk}")
    if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or weight_fp8.shape[1] != k or k % 16:
        raise ValueError("fp8_rerank_topk expects bf16 rows [rows, K], K % 16 == 0, and FP8 weight rows [N, K]")
    cand = candidates.to(torch.int64).contiguous()
    if out is None:
        out = torch.empty(rows, device=x.device, dtype=torch.int64)
    nat.require_cuda(x, cand, weight_fp8, what="fp8_rerank_topk")
    nat.call("fdms_fp8_rerank_topk", x.data_ptr(), x.stride(0), rows, k, weight_fp8.data_ptr(), weight_fp8.stride(0),
             weight_scale_inv.data_ptr(), weight_fp8.shape[0], cand.data_ptr(), topk, out.data_ptr(), nat.stream())
    return out


class ParallelLMHead(VocabParallelEmbedding, LinearBase):
    """The LM head as a bias-free linear [vocab, hidden] (LinearBase's FP8 /
    INT4 weights and kernels) that also serves as the tied embedding table."""

    is_lm_head = True

    def __init__(self, num_embeddings: int, embedding_dim: int, bias: bool = False):
        assert not bias
        LinearBase.__init__(self, embedding_dim, num_embeddings, bias=False)
        self.num_embeddings = num_embeddings
        self.last_logits: torch.Tensor | None = None

    def quantize_weight_to_fp8(self, *, keep_bf16_weight: bool = True, module_name: str | None = None,
                               row1_only: bool = False) -> None:
        """embed_head.py:466-489: FP8 rows (+ the INT4 shadow when
        FASTDMS_INT4_ROW1_SCOPE includes the head), FASTDMS_FP8_LM_HEAD_MIN_ROWS."""
        w8, sinv = quantize_fp8_rows(self.weight.detach())
        self._set_buffer("weight_fp8", w8)
        self._set_buffer("weight_scale_inv", sinv.reshape(1, -1))
        if qe.int4_lm_head_enabled():
            self.quantize_weight_to_int4()
        self._fp8_min_rows = qe.fp8_lm_head_min_rows()
        if not keep_bf16_weight:
            self._drop_bf16_weight()
        self._fp8_weight_enabled = True

    def _last_rows(self, x: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        if ctx.is_prefill:
            x = x[ctx.cu_seqlens_q[1:] - 1].contiguous()
        return x

    def _row1_allowed(self, rows: int) -> bool:
        """embed_head.py:88-93."""
        return rows == 1 and (self.weight.numel() == 0 or rows >= self._fp8_min_rows) and \
            qe.fp8_lm_head_row1_enabled()

    def route(self, rows: int) -> tuple[str, int]:
        """forward()'s kernel choice (embed_head.py:550-583)."""
        if not self._fp8_weight_enabled:
            return "bf16", 0
        if self._row1_allowed(rows) and self._int4_enabled and qe.int4_lm_head_rerank_topk() == 0:
            return "int4", 0
        if self._row1_allowed(rows):
            return "fp8", QX_DIVIDE
        if self.weight.numel() == 0 or rows >= self._fp8_min_rows:
            return "fp8", QX_TORCH
        return "bf16", 0

    def greedy_route(self, rows: int) -> tuple[str, int, bool]:
        """greedy_token_ids' choice (embed_head.py:491-543): (path, activation
        quantisation, bf16 scores)."""
        if self._fp8_weight_enabled and self._row1_allowed(rows):
            if self._int4_enabled:
                return ("int4_rerank" if qe.int4_lm_head_rerank_topk() else "int4"), 0, True
            return "fp8", QX_DIVIDE, False
        path, qx = self.route(rows)
        return path, qx, True

    def logits(self, x2: torch.Tensor) -> torch.Tensor:
        path, qx = self.route(x2.shape[0])
        if path == "fp8" and not small_m_supported(x2.shape[0], self.input_size, self.output_size):
            return fp8_rows_gemm(x2, self.weight_fp8, self.weight_scale_inv, None, qx)
        return self.run(x2, None, route=(path, qx))

    def greedy_into(self, x2: torch.Tensor, out: torch.Tensor) -> None:
        """Greedy token ids of rows x2 [rows, K] into ``out`` (int64 [rows])
        without leaving the device: the head's GEMV fused with the argmax."""
        rows = x2.shape[0]
        path, qx, bf16_scores = self.greedy_route(rows)
        fused = small_m_supported(rows, self.input_size, self.output_size)
        if path == "int4" and fused:
            linear_int4_small_m(x2, self.weight_int4, self.weight_int4_scale_zeros, self._int4_group_size, None,
                                greedy=True, out=out)
        elif path == "int4_rerank":
            logits = linear_int4_small_m(x2, self.weight_int4, self.weight_int4_scale_zeros, self._int4_group_size,
                                         None)
            cand = logits.topk(qe.int4_lm_head_rerank_topk(), dim=-1, sorted=False).indices
            fp8_rerank_topk(x2, cand, self.weight_fp8, self.weight_scale_inv, out=out)
        elif path == "fp8" and fused:
            linear_argmax_small_m(x2, self.weight_fp8, None, weight_scale_inv=self.weight_scale_inv,
                                  quantize_x=qx, bf16_scores=bf16_scores, out=out)
        elif path == "bf16" and fused:
            linear_argmax_small_m(x2, self.weight, None, out=out)
        else:
            logits = self.logits(x2)
            nat.call("fdms_argmax_rows", logits.data_ptr(), nat.dtype_code(logits.dtype), logits.stride(0), rows,
                     logits.shape[1], out.data_ptr(), nat.stream())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.logits(self._last_rows(x))

    def greedy_token_ids(self, x: torch.Tensor) -> torch.Tensor:
        x = self._last_rows(x).contiguous()
        out = torch.empty(x.shape[0], device=x.device, dtype=torch.int64)
        self.greedy_into(x, out)
        return out
