"""Llama / Qwen3 decoder glue (mirror of fastdms/models/llama.py:40-330 and
qwen3.py:82-197).

Per layer, the order of operations is the reference's: qkv projection ->
[Qwen3: per-head q/k RMSNorm] -> DMS decision capture (prefill: extract on q;
decode: fused decision + RoPE + compact append) -> RoPE (prefill) -> streaming
pack of post-RoPE k / v into compact spans (prefill) -> attention -> o_proj.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import torch
from torch import nn

from ..engine.chunked_prefill import attend_and_pack
from ..engine.dms import extract_dms_eviction_decisions
from ..layers.activation import silu_and_mul
from ..layers.attention import Attention
from ..layers.compact_attention import (compact_attention_inline_q_rope_enabled, compact_attention_splitk_enabled,
                                        dms_decode_store_transient_k_enabled, dms_fused_decode_preprocess_enabled,
                                        fused_decode_attention_supported, fused_dms_rope_store_compact_decode)
from ..layers.embed_head import ParallelLMHead, VocabParallelEmbedding, embedding_rms_norm
from ..layers.layernorm import RMSNorm
from ..layers.linear import (EPI_NONE, EPI_SILU_MUL, LinearBase, MergedColumnParallelLinear, QKVParallelLinear,
                             RowParallelLinear, linear_int4_partials, linear_norm_stats, linear_partials,
                             linear_residual_stats, small_m_supported)
from ..layers.rotary_embedding import get_rope
from ..utils.context import get_context


@dataclass
class ModelConfig:
    """The HF config fields the model reads (names as in transformers)."""
    model_type: str = "llama"
    vocab_size: int = 128256
    hidden_size: int = 2048
    intermediate_size: int = 8192
    num_hidden_layers: int = 16
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 64
    rope_theta: float = 500000.0
    rope_scaling: dict | None = field(default_factory=lambda: {
        "rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 8192})
    rms_norm_eps: float = 1e-5
    max_position_embeddings: int = 131072
    tie_word_embeddings: bool = True
    attention_bias: bool = False
    qk_norm: bool = False
    hidden_act: str = "silu"
    dtype: str = "bfloat16"
    # synthetic-weights option (no checkpoint counterpart): > 0 plants a
    # previous-token attention head and a successor table in an untied LM head
    # (the greedy token at position p is succ[token at p - 1]), so that greedy
    # decisions carry a wide logit margin that depends on the attention
    # (models/synthetic.py)
    successor_margin: float = 0.0


def _deferred_linear(lin: LinearBase, x: torch.Tensor, x_amax: torch.Tensor | None = None):
    """A linear whose only consumer is an RMSNorm: on the bf16 / FP8 / INT4
    small-M decode path its split-K merge (and the FP8 row / column scaling)
    moves into that RMSNorm (SplitPartials), which saves the linear's merge
    round trips; other paths return the finished tensor.  ``x_amax``: x's row
    amax from its producer, for an FP8 linear's activation quantisation."""
    rows = x.shape[0]
    path, qx = lin.route(rows)
    if (_defer_splitk_enabled() and lin.bias is None and path in ("bf16", "fp8", "int4")
            and small_m_supported(rows, lin.input_size, lin.output_size) and x.stride(-1) == 1):
        if path == "int4":
            return linear_int4_partials(x, lin.weight_int4, lin.weight_int4_scale_zeros, lin._int4_group_size)
        if path == "bf16":
            return linear_partials(x, lin.weight)
        return linear_partials(x, lin.weight_fp8, weight_scale_inv=lin.weight_scale_inv, quantize_x=qx,
                               x_amax=x_amax)
    return lin.run(x, lin.bias, x_amax=x_amax)


def _norm_into(norm: RMSNorm, x, res: torch.Tensor | None, lin: LinearBase, rows: int):
    """RMSNorm (+ residual add) whose output feeds ``lin``.  When ``lin``
    quantises its activation to FP8 on the small-M kernel, the norm does that
    quantisation once and hands over the e4m3fn codes and the row amax instead
    of the bf16 rows (the linear's workgroups then skip quantising).  Returns
    (activation, residual, row amax or None)."""
    qx = lin.x_quant_mode(rows)
    if not qx:
        if res is None:
            return norm(x), x, None
        h, res = norm(x, res)
        return h, res, None
    dev = res.device if res is not None else x.device
    am = torch.empty((rows, 1), device=dev, dtype=torch.float32)
    q = torch.empty((rows, lin.input_size), device=dev, dtype=torch.float8_e4m3fn)
    quant = dict(amax_out=am, q_out=q, q_mode=qx, bf16_out=False)
    if res is None:
        norm(x, **quant)
        return q, x, am
    _, res = norm(x, res, **quant)
    return q, res, am


def _linear_from_norm(lin: LinearBase, h: torch.Tensor, am: torch.Tensor | None, *, epilogue: int = EPI_NONE,
                      amax_out: torch.Tensor | None = None) -> torch.Tensor:
    """The linear after _norm_into: on the pre-quantised codes when it handed
    them over, else on the bf16 rows."""
    if am is not None:
        return lin.run_quantized(h, am, epilogue=epilogue, amax_out=amax_out)
    return lin.run(h, lin.bias, epilogue=epilogue, amax_out=amax_out)


def _defer_splitk_enabled() -> bool:
    return os.environ.get("FASTDMS_AMD_DEFER_SPLITK", "1").strip() != "0"


def _norm_stats_enabled(hidden_size: int) -> bool:
    """RMSNorms split between the linears around them on the bf16 decode path
    (LlamaModel._forward_decode_norm_stats).  Default: at hidden sizes from
    4096 (measured on MI355X, Qwen3-8B shape c=8: 1 927 against 1 850 decode
    tok/s); not at 2048 (Llama-3.2-1B shape c=8: 7 720 against 7 758 -- the
    fp32 activation rows and the norm prologue cost qkv and gate_up 2.3 and
    3.3 us, the in-kernel split merge o_proj and down_proj 1.8 us each,
    about what the two RMSNorm launches per layer cost).
    FASTDMS_AMD_NORM_STATS=1 / 0 forces it on / off."""
    env = os.environ.get("FASTDMS_AMD_NORM_STATS", "").strip()
    if env in ("0", "1"):
        return env == "1"
    return hidden_size >= 4096


class LlamaAttention(nn.Module):

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim or config.hidden_size // self.num_heads
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.scaling = self.head_dim ** -0.5
        self.qkv_proj = QKVParallelLinear(config.hidden_size, self.head_dim, self.num_heads, self.num_kv_heads,
                                          bias=config.attention_bias)
        self.o_proj = RowParallelLinear(self.num_heads * self.head_dim, config.hidden_size, bias=False)
        self.rotary_emb = get_rope(self.head_dim, self.head_dim, config.max_position_embeddings, config.rope_theta,
                                   config.rope_scaling)
        self.attn = Attention(self.num_heads, self.head_dim, self.scaling, self.num_kv_heads)
        self.qk_norm = config.qk_norm
        if self.qk_norm:
            self.q_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
            self.k_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)

    def forward(self, positions: torch.Tensor, hidden_states: torch.Tensor) -> torch.Tensor:
        qkv = self.qkv_proj(hidden_states)
        return self.o_proj(self.attend(positions, qkv))

    def attend(self, positions: torch.Tensor, qkv: torch.Tensor) -> torch.Tensor:
        """Everything between the qkv and o projections; returns [T, Hq*D]."""
        q = qkv[:, :self.q_size].view(-1, self.num_heads, self.head_dim)
        k = qkv[:, self.q_size:self.q_size + self.kv_size].view(-1, self.num_kv_heads, self.head_dim)
        v = qkv[:, self.q_size + self.kv_size:].view(-1, self.num_kv_heads, self.head_dim)
        ctx = get_context()
        fused = False
        inline_q_rope = False
        evict_mask = None
        layer_id = self.attn.layer_id
        can_fuse = (ctx.dms_capture_enabled and dms_fused_decode_preprocess_enabled() and not ctx.is_prefill
                    and ctx.compact_kv_enabled and ctx.compact_slot_mapping is not None
                    and self.attn.compact_k_cache.numel() > 0)
        one_launch = (can_fuse and not dms_decode_store_transient_k_enabled()
                      and fused_decode_attention_supported(q, k, v, self.attn.compact_k_cache))
        if self.qk_norm and not one_launch:  # Qwen3: QK-norm before DMS extraction (qwen3.py:92-94)
            q = self.q_norm(q)
            k = self.k_norm(k)
        if ctx.dms_capture_enabled:
            if ctx.dms_layer_evictions is None and ctx.dms_layer_evictions_buffer is None and not can_fuse:
                raise RuntimeError("DMS capture requires a layer eviction recorder")
            if layer_id < 0:
                raise RuntimeError("DMS capture requires assigned attention layer ids")
            evict_out = None
            if ctx.dms_layer_evictions_buffer is not None:
                evict_out = ctx.dms_layer_evictions_buffer[layer_id]
            if one_launch:
                # (QK-norm +) decision + RoPE + append + attention in one launch
                if evict_out is None:
                    evict_out = torch.empty((q.shape[0], self.num_kv_heads), device=q.device, dtype=torch.bool)
                o = self.attn.forward_fused_decode(q, k, v, positions, self.rotary_emb.cos_sin_cache, evict_out,
                                                   ctx.dms_alpha_scale, ctx.dms_alpha_offset,
                                                   *((self.q_norm, self.k_norm) if self.qk_norm else ()))
                if ctx.dms_layer_evictions is not None:
                    ctx.dms_layer_evictions[layer_id] = evict_out
                return o.view(o.shape[0], -1)
            if can_fuse:
                inline_q_rope = (compact_attention_inline_q_rope_enabled() and compact_attention_splitk_enabled()
                                 and q.shape[0] == 1 and self.head_dim % 2 == 0 and self.head_dim >= 32)
                slot = ctx.compact_slot_mapping
                if slot.ndim == 3:
                    slot = slot[layer_id]
                if evict_out is None:
                    evict_out = torch.empty((q.shape[0], self.num_kv_heads), device=q.device, dtype=torch.bool)
                fused_dms_rope_store_compact_decode(
                    q, k, v, self.rotary_emb.cos_sin_cache, self.attn.compact_k_cache, self.attn.compact_v_cache,
                    slot, evict_out, positions, num_kv_heads=self.num_kv_heads, alpha_scale=ctx.dms_alpha_scale,
                    alpha_offset=ctx.dms_alpha_offset, store_q=not inline_q_rope,
                    store_transient_k=dms_decode_store_transient_k_enabled(), k_scale=self.attn.compact_k_scale,
                    v_scale=self.attn.compact_v_scale)
                evict_mask = evict_out
                fused = True
            else:
                q, evict_mask = extract_dms_eviction_decisions(
                    q, num_kv_heads=self.num_kv_heads, num_qo_heads=self.num_heads, head_dim=self.head_dim,
                    alpha_scale=ctx.dms_alpha_scale, alpha_offset=ctx.dms_alpha_offset, inplace=True, out=evict_out)
            if ctx.dms_layer_evictions is not None:
                ctx.dms_layer_evictions[layer_id] = evict_mask
        if not fused:
            q, k = self.rotary_emb(positions, q, k)
        if ctx.is_prefill and ctx.prefill_chunk is not None:  # a long prompt's chunk over its retained prefix
            o = attend_and_pack(self.attn, layer_id, q, k, v, evict_mask, ctx, self.attn.scale)
            return o.view(o.shape[0], -1)
        if (ctx.is_prefill and ctx.streaming_pack_manager is not None and ctx.streaming_pack_seq_ids
                and ctx.dms_capture_enabled):
            ctx.streaming_pack_manager.streaming_pack_layer(
                layer_id=layer_id, k=k, v=v, evict_mask=evict_mask, cu_seqlens_q=ctx.cu_seqlens_q,
                seq_ids=ctx.streaming_pack_seq_ids, window_size=ctx.streaming_pack_window_size,
                cu_seqlens_host=ctx.cu_seqlens_q_host)
        o = self.attn(q, k, v, compact_append_stored=fused, compact_q_rope=fused and inline_q_rope,
                      positions=positions, cos_sin_cache=self.rotary_emb.cos_sin_cache)
        return o.view(o.shape[0], -1)


class LlamaMLP(nn.Module):

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        assert config.hidden_act == "silu"
        self.gate_up_proj = MergedColumnParallelLinear(config.hidden_size, [config.intermediate_size] * 2)
        self.down_proj = RowParallelLinear(config.intermediate_size, config.hidden_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(silu_and_mul(self.gate_up_proj(x)))


class LlamaDecoderLayer(nn.Module):

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.self_attn = LlamaAttention(config)
        self.mlp = LlamaMLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, positions, hidden_states, residual):
        if residual is None:
            hidden_states, residual = self.input_layernorm(hidden_states), hidden_states
        else:
            hidden_states, residual = self.input_layernorm(hidden_states, residual)
        hidden_states = self.self_attn(positions, hidden_states)
        hidden_states, residual = self.post_attention_layernorm(hidden_states, residual)
        return self.mlp(hidden_states), residual


class LlamaModel(nn.Module):

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.embed_tokens = VocabParallelEmbedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([LlamaDecoderLayer(config) for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        hidden_states = self.embed_tokens(input_ids)
        residual = None
        for layer in self.layers:
            hidden_states, residual = layer(positions, hidden_states, residual)
        hidden_states, _ = self.norm(hidden_states, residual)
        return hidden_states

    def forward_decode_fused(self, input_ids: torch.Tensor, positions: torch.Tensor, lm_head: LinearBase,
                             greedy_out: torch.Tensor | None = None) -> torch.Tensor | None:
        """The decode step (same math as forward + LM head) on the decode-shaped
        linear kernel: per layer RMSNorm(+residual add), qkv, attention, o_proj,
        RMSNorm(+add), gate_up with SiLU*up as its epilogue, down_proj; then the
        final RMSNorm(+add) and the LM head.  Returns the logits [rows, vocab], or
        with ``greedy_out`` writes the greedy token ids there (the head's GEMV
        fused with the argmax) and returns None.

        With bf16 linears (``_norm_stats_path``) the RMSNorms between layers are
        no kernels of their own: o_proj and down_proj finish as the residual
        add (fp32 rows f, the residual in place, per-strip sums of f^2) and
        qkv / gate_up apply the norm from those sums as they load their
        activation (fdms_linear_small_m epilogue 4 / prologue 2).  Otherwise
        (FP8 / INT4 routes, which quantise the normalised activation) each
        RMSNorm is a kernel that merges its producer's split partials."""
        rows = input_ids.shape[0]
        x, h0 = self._embed_first_norm(input_ids, rows)
        dev = x.device
        if self._norm_stats_path(rows):
            return self._forward_decode_norm_stats(x, h0, positions, lm_head, greedy_out)
        res = None
        for i, layer in enumerate(self.layers):
            attn, mlp = layer.self_attn, layer.mlp
            # an FP8 linear's activation statistics come from its producer: the
            # RMSNorms quantise qkv's / gate_up's input themselves, gate_up hands
            # down_proj its per-strip output amax
            if i == 0 and h0 is not None:
                h, res, am = h0, x, None  # the first norm came with the embedding rows
            else:
                h, res, am = _norm_into(layer.input_layernorm, x, res, attn.qkv_proj, rows)
            qkv = _linear_from_norm(attn.qkv_proj, h, am)
            o = _deferred_linear(attn.o_proj, attn.attend(positions, qkv))
            h, res, am = _norm_into(layer.post_attention_layernorm, o, res, mlp.gate_up_proj, rows)
            am_act = None
            if mlp.down_proj.wants_x_amax(rows) and mlp.gate_up_proj.small_m_fused(rows, EPI_SILU_MUL):
                am_act = torch.empty((rows, mlp.gate_up_proj.output_size // 32), device=dev, dtype=torch.float32)
            act = _linear_from_norm(mlp.gate_up_proj, h, am, epilogue=EPI_SILU_MUL, amax_out=am_act)
            x = _deferred_linear(mlp.down_proj, act, x_amax=am_act)
        h, _ = self.norm(x, res)
        if greedy_out is not None:
            lm_head.greedy_into(h, greedy_out)
            return None
        return lm_head.logits(h)

    def _norm_stats_path(self, rows: int) -> bool:
        if not _norm_stats_enabled(self.norm.weight.numel()) or len(self.layers) < 2:
            return False
        for layer in self.layers:
            attn, mlp = layer.self_attn, layer.mlp
            lins = (attn.qkv_proj, attn.o_proj, mlp.gate_up_proj, mlp.down_proj)
            if any(lin.route(rows)[0] != "bf16" for lin in lins):
                return False
            if attn.o_proj.bias is not None or mlp.down_proj.bias is not None:
                return False
        return True

    def _embed_first_norm(self, input_ids: torch.Tensor, rows: int) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(embedding rows, the first input_layernorm of them or None).  With a
        bf16 table and a first qkv that takes bf16 rows, one launch gathers the
        rows and normalises them (fdms_embedding_rmsnorm); otherwise the gather
        alone (the FP8 table's kernel, or F.embedding), normalised later."""
        emb, norm = self.embed_tokens, self.layers[0].input_layernorm
        if (not emb._fp8_embedding_enabled and emb.weight.dtype == torch.bfloat16 and emb.weight.numel() > 0
                and self.layers[0].self_attn.qkv_proj.x_quant_mode(rows) == 0):
            h, x = embedding_rms_norm(input_ids, emb.weight, norm.weight, norm.eps)
            return x, h
        return emb(input_ids), None

    def _forward_decode_norm_stats(self, x: torch.Tensor, h0: torch.Tensor | None, positions: torch.Tensor,
                                   lm_head: LinearBase, greedy_out: torch.Tensor | None) -> torch.Tensor | None:
        """forward_decode_fused on bf16 linears: the first layer's input RMSNorm
        and the final one are kernels, every RMSNorm in between is split
        between the linear before it (the residual add and the row sums of
        squares) and the one after it (the scaling)."""
        rows, hidden = x.shape
        f = torch.empty((rows, hidden), device=x.device, dtype=torch.float32)
        ssq = torch.empty((rows, hidden // 16), device=x.device, dtype=torch.float32)
        res = x  # the embedding rows are the first residual, updated in place from here on
        h = h0 if h0 is not None else self.layers[0].input_layernorm(x)
        last = len(self.layers) - 1
        for i, layer in enumerate(self.layers):
            attn, mlp = layer.self_attn, layer.mlp
            if i == 0:
                qkv = attn.qkv_proj.run(h, attn.qkv_proj.bias)
            else:
                norm = layer.input_layernorm
                qkv = linear_norm_stats(f, ssq, norm.weight, norm.eps, attn.qkv_proj.weight, attn.qkv_proj.bias)
            linear_residual_stats(attn.attend(positions, qkv), attn.o_proj.weight, res, f, ssq)
            norm = layer.post_attention_layernorm
            act = linear_norm_stats(f, ssq, norm.weight, norm.eps, mlp.gate_up_proj.weight, mlp.gate_up_proj.bias,
                                    epilogue=EPI_SILU_MUL)
            if i < last:
                linear_residual_stats(act, mlp.down_proj.weight, res, f, ssq)
            else:
                h, _ = self.norm(_deferred_linear(mlp.down_proj, act), res)
        if greedy_out is not None:
            lm_head.greedy_into(h, greedy_out)
            return None
        return lm_head.logits(h)

    def decode_fused_supported(self, rows: int, lm_head: LinearBase) -> bool:
        mods = [lm_head]
        for layer in self.layers:
            mods += [layer.self_attn.qkv_proj, layer.self_attn.o_proj, layer.mlp.gate_up_proj, layer.mlp.down_proj]
        return all(small_m_supported(rows, m.input_size, m.output_size) for m in mods) and all(
            layer.mlp.gate_up_proj.output_size % 32 == 0 for layer in self.layers)


class LlamaForCausalLM(nn.Module):
    packed_modules_mapping = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"),
                              "v_proj": ("qkv_proj", "v"), "gate_proj": ("gate_up_proj", 0),
                              "up_proj": ("gate_up_proj", 1)}

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.config = config
        self.model = LlamaModel(config)
        self.lm_head = ParallelLMHead(config.vocab_size, config.hidden_size)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        return self.model(input_ids, positions)

    def compute_logits(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return self.lm_head(hidden_states)

    def compute_greedy_token_ids(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return self.lm_head.greedy_token_ids(hidden_states)

    def decode_fused_supported(self, rows: int) -> bool:
        return self.model.decode_fused_supported(rows, self.lm_head)

    def forward_decode_fused(self, input_ids: torch.Tensor, positions: torch.Tensor,
                             greedy_out: torch.Tensor | None = None) -> torch.Tensor | None:
        """Decode step through the decode-shaped linear kernels; returns the
        logits, or writes greedy token ids into ``greedy_out``."""
        return self.model.forward_decode_fused(input_ids, positions, self.lm_head, greedy_out)


Qwen3ForCausalLM = LlamaForCausalLM  # the same glue with config.qk_norm = True
