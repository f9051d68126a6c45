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


# Final residual RMS of the random model above (measured at the Llama-3.2-1B
# shape: 3.8 after 16 layers); the planted embedding matches it.
_EMBED_RMS = 4.0


@torch.no_grad()
def _plant_successor_table(model, config: ModelConfig, seed: int, device, std: float) -> None:
    """Random weights give nearly flat logits: at the Llama-3.2-1B shape the
    top two of 128 256 logits are typically 1-2 bf16 ulps apart, so any two
    correct implementations that round differently disagree on greedy tokens
    within a few steps.  This plants the margin a trained model has: the token
    embeddings are scaled to the residual stream's size (so the current
    token stays a large part of the final hidden state) and LM-head row
    succ[t] gets successor_margin * unit(e_t) added, for a seeded permutation
    succ.  The greedy token after t is then succ[t] by a wide margin (about
    successor_margin * 0.7 * sqrt(hidden) logits against a random maximum
    near 4), whatever the context contributes to the other logits."""
    emb = model.model.embed_tokens.weight
    e = emb.data.float() * (_EMBED_RMS / std)
    emb.data = e.to(torch.bfloat16)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 104729 + 17)
    succ = torch.randperm(config.vocab_size, generator=gen, device=device)
    unit = e / e.norm(dim=1, keepdim=True)
    head = model.lm_head.weight.data.float()
    head[succ] += float(config.successor_margin) * unit
    model.lm_head.weight.data = head.to(torch.bfloat16)
    del e, unit, head


def successor_table(config: ModelConfig, seed: int, device) -> torch.Tensor:
    """The planted successor permutation of a model built with successor_margin."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed * 104729 + 17)
    return torch.randperm(config.vocab_size, generator=gen, device=device)
