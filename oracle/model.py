"""Model-level oracle — TEST INFRASTRUCTURE / CPU BASELINE ONLY.

A CPU restatement of the compact-DMS Llama / Qwen3 step in torch fp32 (the
"fp32 PyTorch CPU restatement" the benchmark times beside the GPU), rounding
to bf16 at the points the GPU path stores bf16 tensors.  The order of
operations follows fastdms/models/llama.py:87-330 (qwen3.py:82-197 for
QK-norm), fastdms/engine/model_runner.py:594-772 (prefill / decode
preparation) and fastdms/engine/compact_kv.py (pack, expiry, append, record).

Linear layers accumulate in fp32 in a different order than the GPU GEMMs, so
model-level agreement is checked on greedy tokens, not bits (parity unpinned
at the bit level for whole-model outputs; every kernel it composes is pinned
individually in tests/test_oracle_*.py).
"""
from __future__ import annotations

import numpy as np
import torch

from . import attention as oatt
from . import compact_kv as ock
from . import dms as odms
from . import linear as olin
from . import numerics


def bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


class OracleModel:
    """weights: name -> fp32 CPU tensor (values of the bf16 GPU weights), with
    the names of fastdms_amd.models.llama.LlamaForCausalLM.state_dict()."""

    def __init__(self, weights: dict, cfg, *, window_size: int, alpha_scale: float, alpha_offset: float,
                 capacity_tokens: int, max_model_len: int, kv_code: int = numerics.DT_FP8,
                 manager: ock.OracleCompactKVManager | None = None, fp8_linear: dict | None = None,
                 fp8_torch_form_min_rows: int | None = None, int4_linear: dict | None = None,
                 int4_max_rows: int = 0, embed_fp8: tuple | None = None, route=None, fp8_scales: str = "unit"):
        self.w = weights
        self.cfg = cfg
        self.window = int(window_size)
        self.alpha_scale = float(alpha_scale)
        self.alpha_offset = float(alpha_offset)
        self.kv_code = kv_code
        self.L = cfg.num_hidden_layers
        self.Hq = cfg.num_attention_heads
        self.Hkv = cfg.num_key_value_heads
        self.D = cfg.head_dim
        self.cos_sin = oatt.rope_cos_sin_cache(self.D, cfg.max_position_embeddings, cfg.rope_theta,
                                               cfg.rope_scaling)
        self.mgr = manager or ock.OracleCompactKVManager(self.L, self.Hkv, capacity_tokens, max_model_len,
                                                         head_dim=self.D, dtype_code=kv_code)
        # name -> (W8^T e4m3 bits [K, N], scale_inv [1, N]); rows at or above
        # fp8_torch_form_min_rows quantise the activation in _fp8_linear's torch
        # form (linear.py:652-654), fewer rows as the Triton kernels do
        self.fp8_linear = fp8_linear or {}
        self.fp8_torch_form_min_rows = fp8_torch_form_min_rows
        # name -> dequantised INT4 weight [N, K] (bf16 values), used for calls
        # of at most int4_max_rows rows (linear.py:855-870)
        self.int4_linear = int4_linear or {}
        self.int4_max_rows = int(int4_max_rows)
        # (e4m3 bits [V, D], scale_inv [V]): the FP8 token table (embed_head.py:424-434)
        self.embed_fp8 = embed_fp8
        # optional (name, rows) -> "int4" | "fp8" | "fp8_torch" | "bf16": the
        # dispatch decision of LinearBase._linear (linear.py:855-926) for a
        # module with several weight forms; None = the defaults above
        self.route = route
        # per-(layer, kv head) FP8 KV scales (the manager's "calibrate" mode:
        # amax / 224 of the layer's first packed K / V, fp32), None = unit
        self.kv_scales = None if fp8_scales == "unit" else np.ones((self.L, 2, self.Hkv), np.float32)
        self._calibrated = [False] * self.L

    # -- building blocks ------------------------------------------------------
    def rmsnorm(self, x, weight, residual=None):
        """fdms_rmsnorm: fp32 sum of squares, bf16 normalised value, bf16 product."""
        eps = self.cfg.rms_norm_eps
        if residual is not None:
            x = x + residual
            residual = bf16(x)
        var = (x * x).mean(dim=-1, keepdim=True)
        xn = bf16(x * torch.rsqrt(var + eps))  # layernorm.py:24, 37-38
        return bf16(xn * weight), residual

    def embed(self, ids):
        """embed_head.py:424-434: with an FP8 table, bf16(fp8 row) * bf16(scale_inv)."""
        ids = torch.as_tensor(ids)
        if self.embed_fp8 is None:
            return self.w["model.embed_tokens.weight"][ids]
        codes, sinv = self.embed_fp8
        rows = torch.from_numpy(numerics.e4m3fn_decode(codes[ids.numpy()]).astype(np.float32))
        s = torch.from_numpy(np.asarray(sinv, np.float32).reshape(-1)[ids.numpy()]).reshape(-1, 1)
        return bf16(bf16(rows) * bf16(s))

    def linear(self, x, name, bias=True):
        """bf16 F.linear: one rounding of the fp32 sum incl. the bias (the GEMM
        epilogue adds it); the FP8 and INT4 paths round the matmul to bf16 and
        add the bias in bf16 (linear.py:475-477, 659-661)."""
        quantised = True
        rows = x.shape[0]
        if self.route is not None:
            path = self.route(name, rows)
        elif name in self.int4_linear and rows <= self.int4_max_rows:
            path = "int4"
        elif name in self.fp8_linear:
            tf = self.fp8_torch_form_min_rows is not None and rows >= self.fp8_torch_form_min_rows
            path = "fp8_torch" if tf else "fp8"
        else:
            path = "bf16"
        if path == "int4":
            y = bf16(x @ self.int4_linear[name].T)
        elif path in ("fp8", "fp8_torch"):
            w8_t, scale_inv = self.fp8_linear[name]
            cache = self.__dict__.setdefault("_fp8_decoded", {})  # float64 weights, decoded once per name
            if cache.get(name, (None,))[0] is not w8_t:
                cache[name] = (w8_t, numerics.e4m3fn_decode(w8_t).astype(np.float64))
            y = bf16(torch.from_numpy(olin.fp8_linear(x.numpy(), w8_t, scale_inv, quantize_x=True,
                                                      torch_form=path == "fp8_torch",
                                                      w_decoded=cache[name][1]).astype(np.float32)))
        else:
            quantised = False
            y = x @ self.w[name + ".weight"].T
        b = self.w.get(name + ".bias") if bias else None
        if b is not None:
            y = y + (bf16(b) if quantised else b)
        return bf16(y)

    def qkv_split(self, qkv):
        qs, ks = self.Hq * self.D, self.Hkv * self.D
        t = qkv.shape[0]
        return (qkv[:, :qs].reshape(t, self.Hq, self.D), qkv[:, qs:qs + ks].reshape(t, self.Hkv, self.D),
                qkv[:, qs + ks:].reshape(t, self.Hkv, self.D))

    def qk_norm(self, layer, q, k):
        if not self.cfg.qk_norm:
            return q, k
        pre = f"model.layers.{layer}.self_attn."
        q, _ = self.rmsnorm(q, self.w[pre + "q_norm.weight"])
        k, _ = self.rmsnorm(k, self.w[pre + "k_norm.weight"])
        return q, k

    def mlp(self, layer, h):
        gu = self.linear(h, f"model.layers.{layer}.mlp.gate_up_proj", bias=False)
        f = gu.shape[1] // 2
        g, u = gu[:, :f], gu[:, f:]
        act = bf16(torch.nn.functional.silu(g) * u)  # activation.py:8-11, one rounding (compiled)
        return self.linear(act, f"model.layers.{layer}.mlp.down_proj", bias=False)

    def logits(self, x):
        name = "lm_head" if "lm_head.weight" in self.w else "model.embed_tokens"
        if name in self.fp8_linear:
            return self.linear(x, name, bias=False)
        return bf16(x @ self.w[name + ".weight"].T)

    def lm_head(self, x):
        self.last_logits = self.logits(x)
        return olin.argmax_lowest(self.last_logits.numpy())

    def _layer_scales(self, layer, k=None, v=None):
        if self.kv_scales is None:
            return None, None
        if not self._calibrated[layer] and k is not None:
            for i, x in enumerate((k, v)):
                amax = np.abs(np.asarray(x, np.float32)).max(axis=(0, 2))
                self.kv_scales[layer, i] = np.where(amax > 0, (amax / np.float32(224.0)).astype(np.float32),
                                                    np.float32(1.0))
            self._calibrated[layer] = True
        return self.kv_scales[layer, 0], self.kv_scales[layer, 1]

    # -- prefill (model_runner.py:594-679, llama.py:87-202) --------------------
    def prefill(self, seqs: list[tuple[int, list[int], int]]) -> list[int]:
        """seqs: (seq_id, prompt token ids, max_tokens).  Returns each sequence's first token."""
        for sid, prompt, max_tokens in seqs:
            self.mgr.allocate(sid, len(prompt), max_tokens)
        ids = torch.tensor([t for _, p, _ in seqs for t in p])
        cu = np.concatenate([[0], np.cumsum([len(p) for _, p, _ in seqs])]).astype(np.int64)
        pos = np.concatenate([np.arange(len(p)) for _, p, _ in seqs])
        cs = self.cos_sin[pos][:, None, 0]
        cos, sin = cs[..., :self.D // 2], cs[..., self.D // 2:]
        x = self.embed(ids)
        residual = None
        for layer in range(self.L):
            pre = f"model.layers.{layer}."
            if residual is None:
                h, _ = self.rmsnorm(x, self.w[pre + "input_layernorm.weight"])
                residual = x
            else:
                h, residual = self.rmsnorm(x, self.w[pre + "input_layernorm.weight"], residual)
            q, k, v = self.qkv_split(self.linear(h, pre + "self_attn.qkv_proj"))
            q, k = self.qk_norm(layer, q, k)
            qn, evict = odms.extract_dms_eviction_decisions(q.numpy(), num_kv_heads=self.Hkv, num_qo_heads=self.Hq,
                                                            head_dim=self.D, alpha_scale=self.alpha_scale,
                                                            alpha_offset=self.alpha_offset)
            qr = oatt.apply_rotary_emb(qn, cos, sin, numerics.DT_BF16)
            kr = oatt.apply_rotary_emb(k.numpy(), cos, sin, numerics.DT_BF16)
            vn = v.numpy()
            ks, vs = self._layer_scales(layer, kr, vn)
            self.mgr.streaming_pack_layer(layer_id=layer, k=kr, v=vn, evict_mask=evict, cu_seqlens_q=cu,
                                          seq_ids=[s for s, _, _ in seqs], window_size=self.window, k_scale=ks,
                                          v_scale=vs)
            att = numerics.bf16_round(oatt.causal_prefill_attention(qr, kr, vn, cu).astype(np.float32))
            o = self.linear(torch.from_numpy(att.reshape(att.shape[0], -1)), pre + "self_attn.o_proj", bias=False)
            h, residual = self.rmsnorm(o, self.w[pre + "post_attention_layernorm.weight"], residual)
            x = self.mlp(layer, h)
        x, _ = self.rmsnorm(x, self.w["model.norm.weight"], residual)
        return self.lm_head(x[torch.from_numpy(cu[1:] - 1)]).tolist()

    # -- decode (model_runner.py:713-772, 1055-1084; llama.py:121-156) ---------
    def decode(self, seq_ids: list[int], last_tokens: list[int], positions: list[int],
               expiry_mode: str = "auto") -> list[int]:
        self.mgr.apply_dms_evictions(seq_ids, positions, window_size=self.window, triton_mode=expiry_mode)
        base, live, slot, _ = self.mgr.prepare_decode_metadata(seq_ids)
        b = len(seq_ids)
        x = self.embed(last_tokens)
        residual = None
        pos = np.asarray(positions)
        evict_all = np.zeros((self.L, b, self.Hkv), dtype=bool)
        for layer in range(self.L):
            pre = f"model.layers.{layer}."
            if residual is None:
                h, _ = self.rmsnorm(x, self.w[pre + "input_layernorm.weight"])
                residual = x
            else:
                h, residual = self.rmsnorm(x, self.w[pre + "input_layernorm.weight"], residual)
            q, k, v = self.qkv_split(self.linear(h, pre + "self_attn.qkv_proj"))
            q, k = self.qk_norm(layer, q, k)
            qn, kn = q.numpy().copy(), k.numpy().copy()
            ck, cv = self.mgr.compact_k_per_layer[layer], self.mgr.compact_v_per_layer[layer]
            evict_all[layer] = oatt.fused_dms_rope_store_compact_decode(
                q=qn, k=kn, v=v.numpy(), cos_sin_cache=self.cos_sin, compact_k=ck, compact_v=cv,
                slot_mapping=slot[layer], positions=pos, num_kv_heads=self.Hkv, alpha_scale=self.alpha_scale,
                alpha_offset=self.alpha_offset, q_dtype_code=numerics.DT_BF16, k_dtype_code=numerics.DT_BF16,
                compact_dtype_code=self.kv_code, store_q=True, store_transient_k=False,
                k_scale=self._layer_scales(layer)[0], v_scale=self._layer_scales(layer)[1])
            ks, vs = self._layer_scales(layer)
            att = oatt.compact_decode_attention_storage(qn, ck, cv, self.kv_code, base[layer], live[layer],
                                                        k_scale=ks, v_scale=vs)
            att = numerics.bf16_round(att.astype(np.float32))
            o = self.linear(torch.from_numpy(att.reshape(b, -1)), pre + "self_attn.o_proj", bias=False)
            h, residual = self.rmsnorm(o, self.w[pre + "post_attention_layernorm.weight"], residual)
            x = self.mlp(layer, h)
        x, _ = self.rmsnorm(x, self.w["model.norm.weight"], residual)
        tokens = self.lm_head(x).tolist()
        self.mgr.record_appended_dms_decisions(seq_ids, positions, evict_all)
        return tokens


def weights_from_model(model) -> dict:
    """fp32 CPU copies of a fastdms_amd model's (bf16) parameters and buffers by name."""
    out = {}
    for name, p in model.state_dict().items():
        if name.endswith("cos_sin_cache"):
            continue
        out[name] = p.detach().float().cpu()
    if "lm_head.weight" not in out:
        out["lm_head.weight"] = out["model.embed_tokens.weight"]
    return out
