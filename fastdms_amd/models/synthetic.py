"""Random-init model shapes for the benchmarks (no checkpoints are available).

Presets follow the BASELINE configurations: Llama-3.2-1B shape (16 layers,
hidden 2048, 32 q / 8 kv heads, head_dim 64, FFN 8192, vocab 128256, RoPE theta
500000 with llama3 scaling) and Qwen3-8B shape (36 layers, hidden 4096, 32 / 8
heads, head_dim 128, FFN 12288, vocab 151936, QK-norm).

Weights are N(0, 0.02) from a seeded CPU generator.  The DMS decision of kv
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
    model = LlamaForCausalLM(config)
    gen = torch.Generator(device="cpu")
    for i, (name, p) in enumerate(sorted(model.named_parameters(), key=lambda kv: kv[0])):
        gen.manual_seed(seed * 1000003 + i)
        if name.endswith("norm.weight"):
            data = torch.ones(p.shape)
        elif name.endswith(".bias"):
            data = torch.zeros(p.shape)
        else:
            data = torch.randn(p.shape, generator=gen) * std
        p.data = data.to(device=device, dtype=torch.bfloat16)
    if config.tie_word_embeddings:
        model.lm_head.weight = model.model.embed_tokens.weight
    # decision channel: v ~ N(mu, 1) for RMS-normalised inputs, P(v > thr) = 1 - survive_fraction
    z = NormalDist().inv_cdf(1.0 - survive_fraction)
    mu = dms_threshold + z
    rows = dms_decision_rows(config)
    for li, layer in enumerate(model.model.layers):
        gen.manual_seed(seed * 7919 + li)
        w = layer.self_attn.qkv_proj.weight
        r = torch.randn((len(rows), config.hidden_size), generator=gen) / math.sqrt(config.hidden_size)
        w.data[rows] = r.to(device=device, dtype=torch.bfloat16)
        layer.self_attn.qkv_proj.bias.data[rows] = mu
    for module in model.modules():  # RoPE tables go with the model
        if hasattr(module, "cos_sin_cache"):
            module.cos_sin_cache = module.cos_sin_cache.to(device)
    return model.eval()
