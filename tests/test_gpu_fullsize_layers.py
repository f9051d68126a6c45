"""Layer-local parity at the BASELINE sizes: one decode step of the engine at
configs[2] (Llama-3.2-1B shape, all 16 layers, c=8 prompts U[4096, 8192]) and
configs[3] (Qwen3-8B shape, all 36 layers, c=8 prompts of 8192 tokens), FP8
compact KV with calibrated per-head scales on the paged layout, checked layer
by layer against the oracle on the GPU's own inputs.

The prefill runs on the GPU; in the first decode step every layer's fused
decode launch (DMS decision, RoPE, FP8 append, attention) is captured: the
raw q / k / v rows it was given, and after it the decisions, the output and
the span's rows gathered through the block table (rank live - 1 is the row
the launch appended).  For each layer the oracle (oracle/attention.py) takes
the same raw rows and the span's earlier rows and must give
* the same DMS decisions, bit for bit (Qwen3: its decision lane is
  normalised by the per-head QK-norm, whose sum of squares the kernel adds in
  another order, so a decision may differ only where the oracle's value lies
  within a bf16 step of the threshold);
* the same appended FP8 K and V rows, bit for bit (Qwen3: at most two K
  bytes per layer one e4m3 step apart, for the same reason);
* an attention output within 2e-2 max-abs-relative (the north star's bound).
At the Llama shape the step's logits are also checked against the full
16-layer oracle decoding from the GPU's compact state (5 % relative RMS: the
random network's depth amplifies rounding, see test_gpu_engine_shapes.py).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import require_gpu

pytestmark = pytest.mark.gpu

DMS = dict(dms_window_size=256, dms_alpha_scale=10.0, dms_alpha_offset=5.0)
CASES = {
    "l1b_c8": ("llama-3.2-1b", np.random.default_rng(0).integers(4096, 8193, 8).tolist(), True),
    "q8b_c8": ("qwen3-8b", [8192] * 8, False),
}
PAGE = 16


def _gather_spans(arena, bt, live):
    """[B, H, max live, D] bytes of every span's ranks 0 .. live-1 (rows past
    live are zero), through the block table."""
    maxl = int(live.max())
    r = torch.arange(maxl, device=live.device)
    rows = bt[:, :, r // PAGE].long() * PAGE + (r % PAGE)
    valid = r < live[..., None]
    rows = torch.where(valid, rows, torch.zeros_like(rows))
    out = arena.view(torch.uint8)[rows]
    out[~valid] = 0
    return out.cpu().numpy()


class _Capture:
    def __init__(self):
        self.armed = False
        self.layers = []

    def install(self, monkeypatch):
        from fastdms_amd.layers.attention import Attention
        from fastdms_amd.utils.context import get_context
        orig = Attention.forward_fused_decode
        cap = self

        def hook(self, q, k, v, positions, cos_sin_cache, evict_out, alpha_scale, alpha_offset, q_norm=None,
                 k_norm=None):
            if not cap.armed:
                return orig(self, q, k, v, positions, cos_sin_cache, evict_out, alpha_scale, alpha_offset, q_norm,
                            k_norm)
            _, bt, live, slot = self._layer_metadata(get_context())
            raw = [x.float().cpu().numpy() for x in (q, k, v)]
            o = orig(self, q, k, v, positions, cos_sin_cache, evict_out, alpha_scale, alpha_offset, q_norm, k_norm)
            rec = dict(layer=self.layer_id, q=raw[0], k=raw[1], v=raw[2], pos=positions.cpu().numpy(),
                       live=live.cpu().numpy().copy(), slot=slot.cpu().numpy().copy(),
                       evict=evict_out.cpu().numpy().copy(), out=o.float().cpu().numpy(),
                       krows=_gather_spans(self.compact_k_cache, bt, live),
                       vrows=_gather_spans(self.compact_v_cache, bt, live),
                       k_scale=None if self.compact_k_scale is None else self.compact_k_scale.cpu().numpy(),
                       v_scale=None if self.compact_v_scale is None else self.compact_v_scale.cpu().numpy(),
                       q_norm=None if q_norm is None else q_norm.weight.float().cpu().numpy(),
                       k_norm=None if k_norm is None else k_norm.weight.float().cpu().numpy(),
                       eps=None if q_norm is None else q_norm.eps, scale=self.scale)
            cap.layers.append(rec)
            return o

        monkeypatch.setattr(Attention, "forward_fused_decode", hook)


def _head_norm(x, w, eps):
    """layernorm.py:19-40 per head, as the RMSNorm entry points round it."""
    xt = torch.from_numpy(x.astype(np.float32))
    inv = torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + eps)
    xn = (xt * inv).to(torch.bfloat16).float()
    return (xn * torch.from_numpy(w.astype(np.float32))).to(torch.bfloat16).float().numpy()


def _check_layer(rec, cache, hkv, thresh):
    """Oracle decision / append / attention for one captured layer; returns
    (max-abs-rel error, decisions on the threshold edge, differing K bytes)."""
    from oracle import attention as oatt
    from oracle import numerics
    q, k, v = rec["q"], rec["k"], rec["v"]
    b, hq, d = q.shape
    live = rec["live"]
    assert (rec["slot"] >= 0).all(), "every pair appends in a decode step"
    cap = int(live.max())
    base = (np.arange(b * hkv).reshape(b, hkv) * cap).astype(np.int32)
    ck = np.zeros((b * hkv * cap, d), np.uint8)
    cv = np.zeros_like(ck)
    for bi in range(b):
        for h in range(hkv):
            n = int(live[bi, h]) - 1  # the rows before this step's append
            ck[base[bi, h]:base[bi, h] + n] = rec["krows"][bi, h, :n]
            cv[base[bi, h]:base[bi, h] + n] = rec["vrows"][bi, h, :n]
    if rec["q_norm"] is not None:
        q, k = _head_norm(q, rec["q_norm"], rec["eps"]), _head_norm(k, rec["k_norm"], rec["eps"])
    qo = q.copy()
    ev = oatt.fused_dms_rope_store_compact_decode(
        q=qo, k=k.copy(), v=v, cos_sin_cache=cache, compact_k=ck, compact_v=cv, slot_mapping=base + live - 1,
        positions=rec["pos"], num_kv_heads=hkv, alpha_scale=DMS["dms_alpha_scale"],
        alpha_offset=DMS["dms_alpha_offset"], q_dtype_code=numerics.DT_BF16, k_dtype_code=numerics.DT_BF16,
        compact_dtype_code=numerics.DT_FP8, store_q=True, store_transient_k=False, k_scale=rec["k_scale"],
        v_scale=rec["v_scale"])
    g = hq // hkv
    edge = 0
    diff = np.argwhere(ev != rec["evict"])
    for bi, h in diff:
        val = float(q[bi, h * g, d - 1])
        # a decision may differ only on the threshold edge, and only with QK-norm
        assert rec["q_norm"] is not None and abs(val - thresh) <= abs(thresh) * 2.0 ** -7, \
            f"layer {rec['layer']}: DMS decision of (seq {bi}, head {h}) differs (value {val})"
        edge += 1
    app = base + live - 1
    kbytes = 0
    for bi in range(b):
        for h in range(hkv):
            n = int(live[bi, h]) - 1
            got_k, got_v = rec["krows"][bi, h, n], rec["vrows"][bi, h, n]
            assert np.array_equal(got_v, cv[app[bi, h]]), f"layer {rec['layer']}: appended V row ({bi}, {h})"
            kd = got_k != ck[app[bi, h]]
            if kd.any():
                assert rec["q_norm"] is not None, f"layer {rec['layer']}: appended K row ({bi}, {h})"
                assert (np.abs(got_k[kd].astype(int) - ck[app[bi, h]][kd].astype(int)) == 1).all()
            kbytes += int(kd.sum())
    assert kbytes <= 2, f"layer {rec['layer']}: {kbytes} appended K bytes differ"
    ref = oatt.compact_decode_attention_storage(qo, ck, cv, numerics.DT_FP8, base, live, scale=rec["scale"],
                                                k_scale=rec["k_scale"], v_scale=rec["v_scale"])
    err = float(np.abs(rec["out"].reshape(ref.shape) - ref).max() / np.abs(ref).max())
    assert err <= 2e-2, f"layer {rec['layer']}: attention max-abs-rel error {err:.3e}"
    return err, edge, kbytes


@pytest.mark.parametrize("case", sorted(CASES))
def test_decode_layers_follow_the_oracle_at_full_size(monkeypatch, case):
    require_gpu()
    from engine_oracle import oracle_for
    from oracle import attention as oatt
    from oracle_sync import sync_oracle_state
    from fastdms_amd import LLM, SamplingParams
    from fastdms_amd.models.synthetic import PRESETS
    name, lens, with_logits = CASES[case]
    for k, v in {"FASTDMS_AMD_DECODE_LOOKAHEAD": "0", "FASTDMS_COMPACT_GREEDY_FAST_LOOP": "0"}.items():
        monkeypatch.setenv(k, v)
    cap = _Capture()
    cap.install(monkeypatch)
    cfg = PRESETS[name]
    llm = LLM(cfg, max_model_len=max(lens) + 16, max_num_seqs=8, max_num_batched_tokens=sum(lens),
              enforce_eager=True, fused_greedy_head=not with_logits, compact_kv_fp8_scales="calibrate", seed=7,
              **DMS)
    runner, mgr = llm.model_runner, llm.model_runner.compact_kv_manager
    rng = np.random.default_rng(1)
    sp = SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True)
    seqs = [llm.add_request(rng.integers(0, cfg.vocab_size, n).tolist(), sp) for n in lens]
    llm.step()  # prefill
    torch.cuda.synchronize()
    print(f"{case}: prefill of {sum(lens)} tokens done", flush=True)
    orc = None
    if with_logits:
        orc = oracle_for(runner, llm.config, quant=False, dms=DMS)
        sync_oracle_state(orc, mgr, [s.seq_id for s in seqs])
        orc.kv_scales = mgr.kv_scales.cpu().numpy().copy()
        orc._calibrated = [True] * orc.L
    cap.armed = True
    llm.step()  # the decode step under test (the first: it runs the exact expiry before)
    cap.armed = False
    torch.cuda.synchronize()
    assert [r["layer"] for r in cap.layers] == list(range(cfg.num_hidden_layers))
    cache = oatt.rope_cos_sin_cache(cfg.head_dim, max(lens) + 16, cfg.rope_theta, cfg.rope_scaling)
    thresh = DMS["dms_alpha_offset"] / DMS["dms_alpha_scale"]
    errs, edges, kbytes = [], 0, 0
    for rec in cap.layers:
        e, ed, kb = _check_layer(rec, cache, cfg.num_key_value_heads, thresh)
        errs.append(e)
        edges += ed
        kbytes += kb
    live = np.stack([r["live"] for r in cap.layers])
    print(f"{case}: {len(errs)} layers, live rows per (seq, head) mean {live.mean():.0f} max {live.max()}; "
          f"attention max-abs-rel error max {max(errs):.2e}; decisions on the edge {edges}; "
          f"appended K bytes one step apart {kbytes}", flush=True)
    if with_logits:
        # the step under test fed each sequence its prefill token at position len(prompt)
        orc.decode([s.seq_id for s in seqs], [s.token_ids[-2] for s in seqs], [len(s) - 2 for s in seqs])
        got = runner.model.lm_head.last_logits.float().cpu()
        want = orc.last_logits
        rms = float((got - want).pow(2).mean().sqrt()) / float(want.pow(2).mean().sqrt())
        print(f"{case}: 16-layer decode logits rel-RMS {rms:.3e}", flush=True)
        assert rms <= 5e-2
    llm.exit()
