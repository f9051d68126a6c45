"""Pins the model-level oracle (oracle/model.py) against an independent
restatement of the reference's Llama / Qwen3 layer (llama.py:87-330,
qwen3.py:82-197, layernorm.py:16-40, activation.py:8-11, dms.py:152-262,
rotary_embedding.py:7-15) written with torch library routines instead of the
oracle's own building blocks:

* RMSNorm through ``torch.nn.functional.rms_norm`` (fp32) then bf16 and the
  bf16 weight product;
* the DMS decision read from the grouped ``[T, Hkv, G, D]`` view (dms.py:222-230);
* RoPE as ``x*cos + rotate_half(x)*sin`` in fp32 (decode keys go to FP8
  from fp32, compact_attention.py:177-194; prefill keys through bf16);
* prefill attention through ``scaled_dot_product_attention(is_causal=True)``;
* decode attention over the token set the DMS rule keeps, recomputed from the
  per-token decisions (``~evict | cur - t <= W``, compact_kv.py:1263-1337),
  on FP8 values from torch's own float8_e4m3fn cast;
* SiLU through ``torch.nn.functional.silu``.

Prefill logits, per-head live counts and a few decode steps' logits must agree
with the oracle run with the exact expiry every step.  A dropped residual, a
decode RoPE position off by one, a window edge off by one, swapped k/v
columns or a decision lane left in q each moves the logits by far more than
the tolerance (checked by planting such mistakes in the restatement: see
test_planted_mistakes_are_caught).
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

W = 16
ALPHA = (10.0, 5.0)


def _model(preset: str, layers: int):
    from fastdms_amd.models.synthetic import PRESETS, build_synthetic_model
    from oracle.model import weights_from_model
    cfg = replace(PRESETS[preset], num_hidden_layers=layers)
    model = build_synthetic_model(cfg, seed=3, device="cpu", dms_threshold=ALPHA[1] / ALPHA[0])
    return weights_from_model(model), model.config if hasattr(model, "config") else cfg


class Restated:
    """A straightforward re-derivation of the compact-DMS forward, one
    sequence, exact expiry every step."""

    def __init__(self, w, cfg, mistake: str | None = None):
        from oracle import attention as oatt
        self.w, self.cfg, self.mistake = w, cfg, mistake
        self.H, self.Hkv, self.D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.G = self.H // self.Hkv
        # the cos/sin table is pinned against the reference formula in test_oracle_attention
        self.cs = torch.from_numpy(oatt.rope_cos_sin_cache(self.D, cfg.max_position_embeddings, cfg.rope_theta,
                                                           cfg.rope_scaling))
        L = cfg.num_hidden_layers
        self.k8 = [None] * L  # [t, Hkv, D] fp32 values of the FP8 post-RoPE keys
        self.v8 = [None] * L
        self.evict = [None] * L  # [t, Hkv] bool

    def norm(self, x32, weight):
        y = F.rms_norm(x32, (x32.shape[-1],), eps=self.cfg.rms_norm_eps).to(torch.bfloat16)
        return (y * weight.to(torch.bfloat16)).float()

    def lin(self, x, name, bias=False):
        b = self.w.get(name + ".bias") if bias else None
        return F.linear(x, self.w[name + ".weight"], b).to(torch.bfloat16).float()

    def rope(self, x, pos):
        cs = self.cs[pos][:, 0]  # [t, D]
        cos, sin = cs[:, None, :self.D // 2].repeat(1, 1, 2), cs[:, None, self.D // 2:].repeat(1, 1, 2)
        x1, x2 = x[..., :self.D // 2], x[..., self.D // 2:]
        rot = torch.cat((-x2, x1), dim=-1)  # rotate_half
        return x * cos + rot * sin  # fp32

    def fp8(self, x):
        return x.to(torch.float8_e4m3fn).float()

    def decide(self, q):
        """q [t, H, D] -> (q with the decision lanes zeroed, evict [t, Hkv])."""
        grouped = q.reshape(q.shape[0], self.Hkv, self.G, self.D).clone()
        val = grouped[:, :, 0, -1]
        evict = val * ALPHA[0] - ALPHA[1] > 0
        if self.mistake != "no_zero":
            grouped[:, :, 0, -1] = 0
        return grouped.reshape(q.shape), evict

    def layer(self, l, x, residual, pos, prefill):
        pre = f"model.layers.{l}."
        if residual is None:
            residual, h = x, self.norm(x, self.w[pre + "input_layernorm.weight"])
        else:
            s = x + residual
            residual = s.to(torch.bfloat16).float()
            h = self.norm(s, self.w[pre + "input_layernorm.weight"])
        qkv = self.lin(h, pre + "self_attn.qkv_proj", bias=True)
        t = qkv.shape[0]
        qs, ks = self.H * self.D, self.Hkv * self.D
        q = qkv[:, :qs].reshape(t, self.H, self.D)
        k = qkv[:, qs:qs + ks].reshape(t, self.Hkv, self.D)
        v = qkv[:, qs + ks:].reshape(t, self.Hkv, self.D)
        if self.cfg.qk_norm:
            q = self.norm(q, self.w[pre + "self_attn.q_norm.weight"])
            k = self.norm(k, self.w[pre + "self_attn.k_norm.weight"])
        bf = lambda x: x.to(torch.bfloat16).float()
        if self.mistake == "swap_kv":
            k, v = v, k
        cur = int(pos[-1])
        if self.mistake == "pos_shift" and not prefill:
            pos = pos + 1
        q, evict = self.decide(q)
        q = bf(self.rope(q, pos))
        # prefill: RotaryEmbedding returns bf16 keys, packed to FP8 from them;
        # decode: the fused preprocess stores its fp32 RoPE output as FP8
        # (compact_attention.py:177-194)
        k = self.rope(k, pos)
        k8, v8 = self.fp8(bf(k) if prefill else k), self.fp8(v)
        k = bf(k)
        if prefill:
            self.k8[l], self.v8[l], self.evict[l] = k8, v8, evict
            kq = k.repeat_interleave(self.G, dim=1).transpose(0, 1).double()
            vq = v.repeat_interleave(self.G, dim=1).transpose(0, 1).double()
            att = F.scaled_dot_product_attention(q.transpose(0, 1).double(), kq, vq, is_causal=True)
            att = att.transpose(0, 1).float()
        else:
            self.k8[l] = torch.cat([self.k8[l], k8])
            self.v8[l] = torch.cat([self.v8[l], v8])
            self.evict[l] = torch.cat([self.evict[l], evict])
            tok = torch.arange(cur + 1)
            att = torch.empty(1, self.H, self.D)
            for h in range(self.Hkv):
                win = W + 1 if self.mistake == "window" else W
                keep = (~self.evict[l][:, h]) | (cur - tok <= win)
                kk = self.k8[l][keep, h].double()
                vv = self.v8[l][keep, h].double()
                qh = q[0, h * self.G:(h + 1) * self.G].double()
                p = torch.softmax(qh @ kk.T * self.D ** -0.5, dim=-1)
                att[0, h * self.G:(h + 1) * self.G] = (p @ vv).float()
        att = att.to(torch.bfloat16).float()
        o = self.lin(att.reshape(t, -1), pre + "self_attn.o_proj")
        s = o + residual
        residual = s.to(torch.bfloat16).float()
        if self.mistake == "no_residual":
            residual = o
        h = self.norm(s, self.w[pre + "post_attention_layernorm.weight"])
        gu = self.lin(h, pre + "mlp.gate_up_proj")
        f = gu.shape[1] // 2
        act = (F.silu(gu[:, :f]) * gu[:, f:]).to(torch.bfloat16).float()
        return self.lin(act, pre + "mlp.down_proj"), residual

    def forward(self, ids, pos, prefill):
        x = self.w["model.embed_tokens.weight"][torch.as_tensor(ids)]
        residual = None
        for l in range(self.cfg.num_hidden_layers):
            x, residual = self.layer(l, x, residual, pos, prefill)
        s = x + residual
        h = self.norm(s, self.w["model.norm.weight"])
        head = self.w["lm_head.weight"]
        return (h[-1:] @ head.T).to(torch.bfloat16).float()

    def live_counts(self, cur):
        tok = torch.arange(self.evict[0].shape[0])
        return np.array([[int(((~ev[:, h]) | (cur - tok <= W)).sum()) for h in range(self.Hkv)]
                         for ev in self.evict])


def _compare(preset, layers, prompt_len, steps, mistake=None):
    from oracle.model import OracleModel
    w, cfg = _model(preset, layers)
    orc = OracleModel(w, cfg, window_size=W, alpha_scale=ALPHA[0], alpha_offset=ALPHA[1], capacity_tokens=8192,
                      max_model_len=1024)
    rs = Restated(w, cfg, mistake)
    rng = np.random.default_rng(7)
    ids = rng.integers(0, cfg.vocab_size, prompt_len).tolist()
    first = orc.prefill([(0, ids, steps + 1)])[0]
    got = rs.forward(ids, torch.arange(prompt_len), prefill=True)
    errs = [float((got[0] - orc.last_logits[0]).abs().max() / orc.last_logits.abs().max())]
    live_ok = np.array_equal(rs.live_counts(prompt_len - 1), orc.mgr.seq_states[0].live_counts)
    tok = first
    for i in range(steps):
        p = prompt_len + i
        nxt = orc.decode([0], [tok], [p], expiry_mode="0")[0]
        got = rs.forward([tok], torch.tensor([p]), prefill=False)
        errs.append(float((got[0] - orc.last_logits[0]).abs().max() / orc.last_logits.abs().max()))
        live_ok = live_ok and np.array_equal(rs.live_counts(p), orc.mgr.seq_states[0].live_counts)
        tok = nxt
    return errs, live_ok


@pytest.mark.parametrize("preset,layers", [("tiny-llama", 1), ("tiny-llama", 2), ("tiny-qwen3", 2)])
def test_oracle_model_matches_restatement(preset, layers):
    errs, live_ok = _compare(preset, layers, prompt_len=90, steps=6)
    assert live_ok, "per-head live counts differ"
    assert max(errs) <= 1e-3, errs  # observed: 0 (bit-identical logits)


@pytest.mark.parametrize("mistake", ["no_residual", "swap_kv", "pos_shift", "window", "no_zero"])
def test_planted_mistakes_are_caught(mistake):
    """Each plausible composition mistake, planted in the restatement, breaks
    the agreement the test above asserts."""
    errs, live_ok = _compare("tiny-llama", 2, prompt_len=90, steps=6, mistake=mistake)
    assert (not live_ok) or max(errs) > 2e-3, (mistake, errs)
