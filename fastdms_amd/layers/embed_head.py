"""Token embedding and LM head (mirror of fastdms/layers/embed_head.py, single GPU).

``ParallelLMHead.greedy_token_ids`` takes the last token of every prefill
sequence (embed_head.py:491-495) and returns the argmax id, lowest index on
ties (embed_head.py:142, 160).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from ..utils.context import get_context


class VocabParallelEmbedding(nn.Module):
    def __init__(self, num_embeddings: int, embedding_dim: int):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.embedding(x, self.weight)


class ParallelLMHead(VocabParallelEmbedding):
    def __init__(self, num_embeddings: int, embedding_dim: int, bias: bool = False):
        super().__init__(num_embeddings, embedding_dim)
        self.quant = None
        self.last_logits: torch.Tensor | None = None
        assert not bias
        # linear-layer view of the head (the decode step runs it as a fused linear)
        self.input_size, self.output_size = embedding_dim, num_embeddings
        self.bias = None
        self._fp8_weight_enabled = False

    def _last_rows(self, x: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        if ctx.is_prefill:
            x = x[ctx.cu_seqlens_q[1:] - 1].contiguous()
        return x

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self._last_rows(x)
        if self.quant is not None:
            return self.quant(x, None)
        return F.linear(x, self.weight)

    def greedy_token_ids(self, x: torch.Tensor) -> torch.Tensor:
        x = self._last_rows(x)
        if self.quant is not None and hasattr(self.quant, "argmax"):
            return self.quant.argmax(x)
        logits = self.quant(x, None) if self.quant is not None else F.linear(x, self.weight)
        self.last_logits = logits  # the rows the ids came from (kept for inspection; no copy)
        return logits.argmax(dim=-1)
