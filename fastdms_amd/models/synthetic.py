"""Random-init model shapes for the benchmarks (no checkpoints are available).

Presets follow the BASELINE configurations: Llama-3.2-1B shape (16 layers,
hidden 2048, 32 q / 8 kv heads, head_dim 64, FFN 8192, vocab 128256, RoPE theta
500000 with llama3 scaling) and Qwen3-8B shape (36 layers, hidden 4096, 32 / 8
heads, head_dim 128, FFN 12288, vocab 151936, QK-norm).

Weights are N(0, 0.02) from a generator seeded per parameter, on the model's device.  The DMS decision of kv
head h is q channel D-1 of query head h*G (dms.py:163-168); its projection row
is drawn N(0, 1/hidden) and given a bias so that, for RMS-normalised inputs,
P(decision > threshold) = 1 - survive_fraction, i.e. about 1/8 of the tokens
outside the window survive.
"""
from __future__ import annotations

import math
from dataclasses import replace
from statistics import NormalDist

import torch

from .llama import LlamaForCausalLM, ModelConfig

PRESETS: dict[str, ModelConfig] = {
    "llama-3.2-1b": ModelConfig(),
    "qwen3-8b": ModelConfig(model_type="qwen3", vocab_size=151936, hidden_size=4096, intermediate_size=12288,
                            num_hidden_layers=36, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                            rope_theta=1000000.0, rope_scaling=None, rms_norm_eps=1e-6,
                            max_position_embeddings=40960, tie_word_embeddings=False, qk_norm=True),
    "tiny-llama": ModelConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                              num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                              max_position_embeddings=4096),
    "tiny-qwen3": ModelConfig(model_type="qwen3", vocab_size=512, hidden_size=256, intermediate_size=512,
                              num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                              rope_theta=1000000.0, rope_scaling=None, rms_norm_eps=1e-6,
                              max_position_embeddings=4096, tie_word_embeddings=False, qk_norm=True),
}


def model_config(name_or_config) -> ModelConfig:
    if isinstance(name_or_config, ModelConfig):
        return name_or_config
    if isinstance(name_or_config, dict):
        return ModelConfig(**name_or_config)
    try:
        return replace(PRESETS[str(name_or_config)])
    except KeyError:
        raise ValueError(f"unknown synthetic model {name_or_config!r}; presets: {sorted(PRESETS)}") from None


def dms_decision_rows(config: ModelConfig) -> list[int]:
    """Rows of the fused qkv weight that produce the borrowed decision channel."""
    g = config.num_attention_heads // config.num_key_value_heads
    d = config.head_dim
    return [(h * g) * d + d - 1 for h in range(config.num_key_value_heads)]


@torch.no_grad()
def build_synthetic_model(config: ModelConfig, *, seed: int = 0, device: str | torch.device = "cuda",
                          dms_threshold: float = 0.5, survive_fraction: float = 0.125,
                          std: float = 0.02) -> LlamaForCausalLM:
    """Instantiate the model on ``device`` in bf16 with seeded random weights."""
    config = replace(config, attention_bias=True)  # carries the decision-channel bias
    if config.successor_margin > 0:
        config = replace(config, tie_word_embeddings=False)
    model = LlamaForCausalLM(config)
    # drawn on the target device (a 1B-parameter model in well under a second
    # on the GPU); the same seed gives the same weights on the same device type
    device = torch.device(device)
    gen = torch.Generator(device=device)
    for i, (name, p) in enumerate(sorted(model.named_parameters(), key=lambda kv: kv[0])):
        gen.manual_seed(seed * 1000003 + i)
        if name.endswith("norm.weight"):
            data = torch.ones(p.shape, device=device)
        elif name.endswith(".bias"):
            data = torch.zeros(p.shape, device=device)
        else:
            data = torch.randn(p.shape, generator=gen, device=device) * std
        p.data = data.to(dtype=torch.bfloat16)
        del data
    if config.tie_word_embeddings:
        model.lm_head.weight = model.model.embed_tokens.weight
    # decision channel: v ~ N(mu, 1) for RMS-normalised inputs, P(v > thr) = 1 - survive_fraction
    z = NormalDist().inv_cdf(1.0 - survive_fraction)
    mu = dms_threshold + z
    rows = dms_decision_rows(config)
    for li, layer in enumerate(model.model.layers):
        gen.manual_seed(seed * 7919 + li)
        w = layer.self_attn.qkv_proj.weight
        r = torch.randn((len(rows), config.hidden_size), generator=gen, device=device) / math.sqrt(config.hidden_size)
        w.data[rows] = r.to(device=device, dtype=torch.bfloat16)
        layer.self_attn.qkv_proj.bias.data[rows] = mu
    if config.successor_margin > 0:
        _plant_successor_table(model, config, seed, device, std)
    for module in model.modules():  # RoPE tables go with the model
        if hasattr(module, "cos_sin_cache"):
            module.cos_sin_cache = module.cos_sin_cache.to(device)
    return model.eval()


# The previous-token plant: query head 1 of kv head 1 in layer 0 attends to the
# token one position back, through RoPE.  Its q and k are constants (weight
# rows zero, biases set) in the first _PLANT_PLANES rotary planes, plane i
# weighted _PLANT_DECAY**i, with k rotated one position ahead of q, so the
# score at distance delta is A * sum_i w_i cos(theta_i (delta - 1)): A at
# delta = 1 and at least 0.149 A (Llama-3.2-1B RoPE; 0.20 A Qwen3-8B) below
# that at every other distance up to 16 384.  A = _PLANT_SCORE nats after the
# 1/sqrt(head_dim) scale, so the head's softmax puts all but ~e^-15 of its
# mass on the previous token, whatever else the compact KV holds.
_PLANT_LAYER = 0
_PLANT_PLANES = 16
_PLANT_DECAY = 0.8
_PLANT_SCORE = 100.0
# RMS of the planted head's output in the residual stream (about that of the
# rest of the final residual of these random models)
_PLANT_RESIDUAL_RMS = 3.0


def _plant_heads(config: ModelConfig) -> tuple[int, int]:
    """(kv head, query head) of the planted previous-token head."""
    g = config.num_attention_heads // config.num_key_value_heads
    if g < 2:
        raise ValueError("the previous-token plant needs at least two query heads per kv head")
    kv = 1 if config.num_key_value_heads > 1 else 0
    return kv, kv * g + 1  # query head kv*g carries the DMS decision channel


@torch.no_grad()
def _plant_successor_table(model, config: ModelConfig, seed: int, device, std: float) -> None:
    """Random weights give nearly flat logits: at the Llama-3.2-1B shape the
    top two of 128 256 logits are typically 1-2 bf16 ulps apart, so two
    correct implementations that round differently disagree on greedy tokens
    within a few steps.  This plants the margin a trained model has, through
    attention: a previous-token head in layer 0 (constants above) copies its
    value row of the previous token, W_v RMSNorm(e[prev]), through its o_proj
    block (scaled so its output has RMS _PLANT_RESIDUAL_RMS) into the
    residual stream as c[prev]; LM-head row succ[t] gets successor_margin *
    unit(c[t]) added for a seeded permutation succ.  The greedy token at
    position p is then succ[token at p - 1] by a wide margin, and it is
    retrieved by the decode attention from the compact FP8 K/V rows appended
    in the previous step (with RoPE of q and k at their positions): an
    engine whose attention, RoPE, appends or K/V addressing are wrong loses
    the previous token and with it the planted margin."""
    kv, qh = _plant_heads(config)
    d, hidden = config.head_dim, config.hidden_size
    attn = model.model.layers[_PLANT_LAYER].self_attn
    # RoPE angle per position step of each plane, from the model's own table
    cos_sin = attn.rotary_emb.cos_sin_cache if hasattr(attn, "rotary_emb") else None
    if cos_sin is None:
        cos_sin = next(m.cos_sin_cache for m in model.modules() if hasattr(m, "cos_sin_cache"))
    row1 = cos_sin[1].reshape(-1).float().to(device)
    theta = torch.atan2(row1[d // 2:], row1[:d // 2])[:_PLANT_PLANES]
    w = _PLANT_DECAY ** torch.arange(_PLANT_PLANES, dtype=torch.float32, device=device)
    w = w / w.sum()
    raw = _PLANT_SCORE * math.sqrt(d)  # q.k at distance 1, before the 1/sqrt(d) scale
    qkv = attn.qkv_proj
    q_rows = slice(qh * d, (qh + 1) * d)
    k0 = config.num_attention_heads * d
    k_rows = slice(k0 + kv * d, k0 + (kv + 1) * d)
    qv = torch.zeros(d, device=device)
    kv_vec = torch.zeros(d, device=device)
    planes = torch.arange(_PLANT_PLANES, device=device)
    if config.qk_norm:
        # the per-head RMSNorm fixes |q| = |k| = sqrt(d) * gain on the planted
        # dims: sqrt(w_i) per plane before the norm, the gain in the norm
        # weights (shared by the layer's heads; the other dims keep weight 1)
        amp = torch.sqrt(w)
        gain = math.sqrt(raw / d)
        for norm in (attn.q_norm, attn.k_norm):
            nw = norm.weight.data.float()
            nw[planes] = gain
            nw[planes + d // 2] = gain
            norm.weight.data = nw.to(torch.bfloat16)
    else:
        amp = torch.sqrt(raw * w)
    qv[planes] = amp
    kv_vec[planes] = amp * torch.cos(theta)
    kv_vec[planes + d // 2] = amp * torch.sin(theta)
    for rows, vec in ((q_rows, qv), (k_rows, kv_vec)):
        qkv.weight.data[rows] = 0
        qkv.bias.data[rows] = vec.to(torch.bfloat16)
    # c[t]: what the head writes into the residual stream for previous token t
    v_rows = slice(k0 + config.num_key_value_heads * d + kv * d, k0 + config.num_key_value_heads * d + (kv + 1) * d)
    w_v = qkv.weight.data[v_rows].float()
    o = attn.o_proj.weight
    w_o = o.data[:, qh * d:(qh + 1) * d].float()
    emb = model.model.embed_tokens.weight.data
    unit_c = torch.empty((config.vocab_size, hidden), device=device, dtype=torch.float32)
    rms_sum = 0.0
    for t0 in range(0, config.vocab_size, 16384):
        e = emb[t0:t0 + 16384].float()
        x = e * torch.rsqrt(e.pow(2).mean(dim=1, keepdim=True) + config.rms_norm_eps)
        c = (x @ w_v.T) @ w_o.T
        n = c.norm(dim=1, keepdim=True)
        rms_sum += float((n / math.sqrt(hidden)).sum())
        unit_c[t0:t0 + 16384] = c / n.clamp_min(1e-12)
    beta = _PLANT_RESIDUAL_RMS / (rms_sum / config.vocab_size)
    o.data[:, qh * d:(qh + 1) * d] = (w_o * beta).to(torch.bfloat16)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 104729 + 17)
    succ = torch.randperm(config.vocab_size, generator=gen, device=device)
    head = model.lm_head.weight.data.float()
    head[succ] += float(config.successor_margin) * unit_c
    model.lm_head.weight.data = head.to(torch.bfloat16)
    del unit_c, head


def successor_table(config: ModelConfig, seed: int, device) -> torch.Tensor:
    """The planted successor permutation of a model built with successor_margin:
    the greedy token at position p is succ[token at p - 1]."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 104729 + 17)
    return torch.randperm(config.vocab_size, generator=gen, device=device)
