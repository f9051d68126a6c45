#!/usr/bin/env python3
"""Compact-DMS decode throughput on one MI355X.

Default workload (--config l1b-c8): Llama-3.2-1B-shaped
model with random bf16 weights, DMS window 256 / threshold 0.5 (~1/8 of tokens
outside the window survive), FP8 compact KV; 8 requests with prompt lengths
uniform in [4096, 8192] and uniform-random token ids, 128 greedy tokens each.
--config l1b-c1 and q8b-c8 (configs[3], Qwen3-8B shape) run the
same harness.  After a warm-up generation of the same prompt lengths, the
prompts are prefilled together (timed separately as prefill_tok_s), then one
"step" is one decode step of the batch: expiry policy, DMS decision + RoPE +
FP8 append, compact attention and the full model forward, greedy argmax and
decision recording.

Prints one JSON line:
  value            decode tok/s over the K timed steps (inputs resident in HBM)
  roofline         the compact decode attention kernel: algorithmic bytes per
                   launch / average launch time, measured with HIP events around
                   graph replays of that kernel on the live decode state
  cpu_baseline     the fp32 torch-CPU oracle (oracle/model.py) decoding the same
                   batch from the same compact state on the host cores, plus a
                   labelled CPU prefill figure and the host CPU model
  q8b_c8           (default run) the same decode harness on configs[3], the
                   Qwen3-8B shape the metric also names: decode tok/s, prefill
                   tok/s, greedy loop and its attention roofline (--no-8b skips)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E bandwidth

# BASELINE.json configs[1..3]: model preset, sequences, prompt-length range
CONFIGS = {
    "l1b-c1": ("llama-3.2-1b", 1, 8192, 8192,
               "BASELINE configs[1]: Llama-3.2-1B shape, c=1, one 8192-token prompt, 128 greedy tokens, "
               "DMS window 256 thr 0.5"),
    "l1b-c8": ("llama-3.2-1b", 8, 4096, 8192,
               "BASELINE configs[2]: Llama-3.2-1B shape, c=8 ragged prompts U[4096,8192], 128 greedy tokens, "
               "DMS window 256 thr 0.5"),
    "q8b-c8": ("qwen3-8b", 8, 8192, 8192,
               "BASELINE configs[3]: Qwen3-8B shape (QK-norm), c=8, 8192-token prompts, 128 greedy tokens, "
               "DMS window 256 thr 0.5"),
    "multitenant": ("llama-3.2-1b", 16, 512, 16384,
                    "BASELINE configs[4]: Llama-3.2-1B shape, W4A16 INT4 linears (group 128, symmetric), 32 requests "
                    "with Poisson(4/s) arrivals, prompts log-uniform [512,16384], generation U[64,256], compact KV "
                    "capped (deferred admission, spans overcommitted by a 32-token decode reserve, preemption)"),
}


def run_multitenant(args):
    """BASELINE configs[4] on one GPU: requests arrive on a Poisson clock and
    join the running engine; the compact KV arena is capped below the offered
    load, so prefills are deferred, spans grow during decode and sequences are
    preempted and re-admitted (re-prefill).  Reports generated tokens per
    second of wall time, the split into prefill / decode steps, time to first
    token and the admission / preemption counts.  No int4 KV: the reference's
    "int4 shadow" is its INT4 weight path (used here), it has no int4 KV."""
    import numpy as np
    import torch
    # the INT4 row-1 weights are applied by the FP8 weight conversion (as in
    # model_runner.py:72-113): FP8 rows for prefill, INT4 for decode rows
    os.environ.setdefault("FASTDMS_FP8_WEIGHTS", "1")
    os.environ.setdefault("FASTDMS_FP8_WEIGHT_SCOPE", "all")
    os.environ.setdefault("FASTDMS_FP8_LM_HEAD", "0")
    os.environ.setdefault("FASTDMS_INT4_ROW1_WEIGHTS", "1")
    os.environ.setdefault("FASTDMS_INT4_ROW1_SCOPE", "all")
    os.environ.setdefault("FASTDMS_INT4_ROW1_GROUP_SIZE", "128")
    os.environ.setdefault("FASTDMS_INT4_ROW1_QUANT_MODE", "symmetric")
    os.environ.setdefault("FASTDMS_INT4_ROW1_MAX_ROWS", "16")
    from fastdms_amd import LLM, SamplingParams

    rng = np.random.default_rng(args.seed)
    n_req = args.requests
    arrivals = np.cumsum(rng.exponential(1.0 / args.rate, n_req))
    lens = np.exp(rng.uniform(np.log(512), np.log(16384), n_req)).astype(int).tolist()
    gens = rng.integers(64, 257, n_req).tolist()
    cap = args.kv_cap_tokens
    progress(f"multitenant: {n_req} requests, prompts {min(lens)}..{max(lens)}, compact capacity {cap} tokens/layer")
    llm = LLM("llama-3.2-1b", max_model_len=16384 + 256, max_num_seqs=16, max_num_batched_tokens=16384 + 256,
              dms_window_size=256, dms_alpha_scale=10.0, dms_alpha_offset=5.0, kv_cache_dtype="float8_e4m3fn",
              seed=args.seed, compact_kv_capacity_tokens=cap, compact_admission="preempt",
              compact_decode_reserve_tokens=32)
    vocab = llm.config.hf_config.vocab_size
    prompts = [rng.integers(0, vocab, n).tolist() for n in lens]
    # warm-up: one short request (library set-up, decode graph capture)
    llm.generate([prompts[0][:512]], SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True))
    torch.cuda.synchronize()
    seqs, first_token = [], {}
    t_start = time.perf_counter()
    nxt = 0
    prefill_s = decode_s = 0.0
    prefill_tokens = decode_tokens = 0
    while nxt < n_req or not llm.is_finished():
        now = time.perf_counter() - t_start
        while nxt < n_req and arrivals[nxt] <= now:
            sp = SamplingParams(temperature=0.0, max_tokens=gens[nxt], ignore_eos=True)
            seqs.append((llm.add_request(prompts[nxt], sp), arrivals[nxt]))
            nxt += 1
        if llm.is_finished():
            time.sleep(max(0.0, arrivals[nxt] - now))
            continue
        t0 = time.perf_counter()
        _, num = llm.step()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        if num > 0:
            prefill_s += dt
            prefill_tokens += num
        else:
            decode_s += dt
            decode_tokens += -num
        for seq, arr in seqs:
            if seq.seq_id not in first_token and seq.num_completion_tokens > 0:
                first_token[seq.seq_id] = time.perf_counter() - t_start - arr
    wall = time.perf_counter() - t_start
    generated = sum(len(s.completion_token_ids) for s, _ in seqs)
    assert all(len(s.completion_token_ids) == g for (s, _), g in zip(seqs, gens)), "a request did not finish"
    ttft = np.array([first_token[s.seq_id] for s, _ in seqs])
    sched = llm.scheduler
    mgr = llm.model_runner.compact_kv_manager
    out = {
        "metric": "multitenant generated tok/s (wall clock, Poisson arrivals)",
        "value": round(generated / wall, 2), "unit": "tok/s", "n_gpus": 1, "steps": None, "warmup": 1,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 activations, int4 (W4A16, g128 symmetric) linears, fp8_e4m3 compact KV",
        "data": "synthetic",
        "config": {"workload": CONFIGS["multitenant"][4], "model": "llama-3.2-1b", "requests": n_req,
                   "rate_per_s": args.rate, "kv_cap_tokens_per_layer": cap, "parallelism": "single GPU"},
        "decode_tok_s": round(decode_tokens / decode_s, 1) if decode_s else None,
        "prefill_tok_s": round(prefill_tokens / prefill_s, 1) if prefill_s else None,
        "wall_s": round(wall, 3), "generated_tokens": generated,
        "ttft_s": {"p50": round(float(np.percentile(ttft, 50)), 3), "p99": round(float(np.percentile(ttft, 99)), 3)},
        "preemptions": sched.num_preemptions, "deferred_prefills": sched.num_deferrals,
        "span_moves": mgr.num_span_moves, "kv_layout": "paged" if mgr.paged else "span",
        "int4_linears": sum(1 for m in llm.model_runner.model.modules() if getattr(m, "_int4_enabled", False)),
        "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(out))
    llm.exit()


def progress(msg: str) -> None:
    """One progress line on stderr (stdout carries only the JSON result)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--config", choices=sorted(CONFIGS), default="l1b-c8",
                   help="BASELINE workload preset (model, batch, prompt lengths)")
    p.add_argument("--batch", type=int, default=None)
    p.add_argument("--min-prompt", type=int, default=None)
    p.add_argument("--max-prompt", type=int, default=None)
    p.add_argument("--gen", type=int, default=128)
    p.add_argument("--model", default=None)
    p.add_argument("--attn-replays", type=int, default=50)
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-scaling", action="store_true", help="skip the attention batch-scaling points")
    p.add_argument("--no-8b", action="store_true",
                   help="l1b-c8: skip the Qwen3-8B-shape (configs[3]) decode run of the same line")
    p.add_argument("--no-fast-loop", action="store_true",
                   help="skip the device-side greedy loop over the rest of the generation (counter runs)")
    p.add_argument("--requests", type=int, default=32, help="multitenant: number of requests")
    p.add_argument("--rate", type=float, default=4.0, help="multitenant: Poisson arrival rate (requests/s)")
    p.add_argument("--kv-cap-tokens", type=int, default=19000,
                   help="multitenant: compact KV capacity per layer (tokens); at the default seed the largest "
                        "request needs just under 19000 alone, so prefills are deferred and sequences preempted")
    p.add_argument("--eager", action="store_true", help="decode without HIP graphs")
    p.add_argument("--kv-scales", choices=["calibrate", "unit"], default="calibrate",
                   help="per-(layer, kv head) FP8 KV scales (BASELINE configs[1]-[3]) or unit scales (the "
                        "reference's bare cast)")
    return p.parse_args()


def attention_roofline(llm, seqs, replays: int, config: str = "l1b-c8"):
    """Average duration and algorithmic HBM bytes of the decode attention kernel
    the step runs, on the live decode state: one graph holds the kernel of
    every layer with the decode step's arguments; HIP events on the capture
    stream bracket `replays` replays.  With the fused decode path this is
    fdms_fused_decode_attention (DMS decision + RoPE + FP8 append + attention;
    each replay re-appends the step's row at rank live-1), else the plain
    compact attention.  Bytes per launch: FP8 K/V rows read from the spans,
    q / k / v rows read (bf16), the appended FP8 rows and the output written,
    and the int32 / int64 metadata."""
    import torch
    from fastdms_amd.layers.compact_attention import (attention_split_plan, attention_waves, mfma_heavy_rows,
                                                      compact_decode_attention, fused_decode_attention_planned,
                                                      compact_decode_attention_paged,
                                                      fused_decode_attention_supported,
                                                      fused_dms_rope_store_compact_decode_attention,
                                                      mfma_attention_path)

    runner = llm.model_runner
    mgr = runner.compact_kv_manager
    cfg = llm.config.hf_config
    md = runner.dms_metadata
    states = [mgr.seq_states[s.seq_id] for s in seqs]
    start = mgr._contiguous_active_slot_start(states)
    b = len(seqs)
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    live = mgr.layer_major_live_counts[:, start:start + b]
    if mgr.paged:  # the row the last decode step appended: rank live-1 through the block table
        bt = mgr.block_tables[:, start:start + b]
        last = (live - 1).long().clamp(min=0)
        page = torch.gather(bt, 3, (last // 16).unsqueeze(-1)).squeeze(-1)
        slot = (page * 16 + last % 16).to(torch.int32).contiguous()
        base = None
    else:
        bt = None
        base = mgr.layer_major_base_offsets[:, start:start + b]
        slot = (base + live - 1).contiguous()
    hint = runner.attention_hint(seqs)  # the bound (and so the split count) the decode step uses
    gen = torch.Generator(device="cpu").manual_seed(1)
    qkv = (torch.randn((b, (hq + 2 * hkv) * d), generator=gen) * 4).to(device="cuda", dtype=torch.bfloat16)
    q = qkv[:, :hq * d].view(b, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(b, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
    positions = torch.tensor([len(s) - 1 for s in seqs], device="cuda", dtype=torch.int64)
    evict = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
    layers = list(range(cfg.num_hidden_layers))
    arenas = [(mgr.compact_k_per_layer[l], mgr.compact_v_per_layer[l]) for l in layers]
    cos_sin = runner.model.model.layers[0].self_attn.rotary_emb.cos_sin_cache
    fused = fused_decode_attention_supported(q, k, v, arenas[0][0])
    out = torch.empty_like(q)
    plan = runner.decode_plan if (mgr.paged and fused) else None
    if plan is not None:
        # the step's work plan for this state: the plan kernel on copies of the
        # pool state with live - 1, so it re-derives the last step's append
        # rows (no page pops: those pages are already held) and the engine's
        # state is left as it is
        from fastdms_amd import _native as nat
        lv1 = (live - 1).contiguous()
        held = mgr.pages_held[:, start:start + b].clone()
        bt_c = bt.clone()
        stack, top = mgr.page_stack.clone(), mgr.page_top.clone()
        ovf = torch.zeros(1, dtype=torch.int32, device="cuda")
        slot_c = torch.empty_like(lv1)
        p_rows, p_heavy, p_splits = plan.partition(b * hkv)
        nat.call("fdms_paged_prepare_decode_plan", lv1.data_ptr(), *lv1.stride(), slot_c.data_ptr(),
                 *slot_c.stride(), bt_c.data_ptr(), *bt_c.stride()[:3], held.data_ptr(), *held.stride(),
                 stack.data_ptr(), stack.stride(0), top.data_ptr(), mgr.max_pages, ovf.data_ptr(),
                 positions.data_ptr(), plan.items.data_ptr(), plan.items.stride(0), p_rows, p_heavy, p_splits,
                 cfg.num_hidden_layers, b, hkv, nat.stream())
        torch.cuda.synchronize()
        if int(ovf.item()) or not torch.equal(slot_c, slot) or not torch.equal(lv1, live):
            raise RuntimeError("attention roofline: the plan does not reproduce the decode state")

    def launch(l):
        if plan is not None:
            ks, vs = mgr.layer_kv_scales(l)
            fused_decode_attention_planned(q, k, v, cos_sin, arenas[l][0], arenas[l][1], evict, positions, plan, l,
                                           num_kv_heads=hkv, alpha_scale=md.alpha_scale,
                                           alpha_offset=md.alpha_offset, out=out, k_scale=ks, v_scale=vs)
        elif fused:
            ks, vs = mgr.layer_kv_scales(l)
            fused_dms_rope_store_compact_decode_attention(
                q, k, v, cos_sin, arenas[l][0], arenas[l][1], slot[l], evict, positions,
                None if base is None else base[l], live[l], num_kv_heads=hkv, alpha_scale=md.alpha_scale,
                alpha_offset=md.alpha_offset, max_live_count=hint, out=out,
                block_tables=None if bt is None else bt[l], k_scale=ks, v_scale=vs)
        elif bt is not None:
            compact_decode_attention_paged(q, arenas[l][0], arenas[l][1], bt[l], live[l], 16, max_live_count=hint)
        else:
            compact_decode_attention(q, arenas[l][0], arenas[l][1], base[l], live[l], max_live_count=hint)

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.inference_mode(), torch.cuda.stream(s):  # the engine's tensors are inference tensors
        for l in layers:  # warm-up outside capture
            launch(l)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for l in layers:
                launch(l)
        g.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(s)
        for _ in range(replays):
            g.replay()
        t1.record(s)
        torch.cuda.synchronize()
    per_launch_s = t0.elapsed_time(t1) / 1e3 / (replays * len(layers))
    lv = live.to(torch.int64).cpu()
    elem = arenas[0][0].element_size()
    nl = len(layers)
    # paged: one int32 block-table entry per 16-row page read in place of the
    # span's base offset
    meta = 4 * int(((lv + 15) // 16).sum()) if bt is not None else 4 * nl * b * hkv
    if fused:
        kv_bytes = int((lv - 1).clamp(min=0).sum()) * d * 2 * elem     # span rows read (all but the appended one)
        io_bytes = nl * b * ((hq + 2 * hkv) * d * 2                     # raw q, k, v rows (bf16)
                             + 2 * hkv * d * elem                        # appended K and V rows (FP8)
                             + hq * d * 2                                # output (bf16)
                             + hkv * (2 * 4 + 1) + 8 + d * 4) + meta     # live/slot, evict, position, cos/sin
    else:
        kv_bytes = int(lv.sum()) * d * 2 * elem
        io_bytes = nl * b * (2 * hq * d * 2 + 4 * hkv) + meta
    bytes_per_launch = (kv_bytes + io_bytes) / nl
    mfma = mfma_attention_path(q, arenas[0][0], hq // hkv)
    splits, split_rows = attention_split_plan(q.device, b * hkv, hint, mfma)
    if plan is not None:  # the step's work plan (layer 0)
        p_rows, p_heavy, p_splits = plan.partition(b * hkv)
        per_pair = torch.where(lv[0] <= p_rows, torch.ones_like(lv[0]),
                               (lv[0] + p_heavy - 1) // p_heavy).clamp(1, p_splits)
        splits = {"planned": True, "rows_per_split": p_rows, "heavy_rows": p_heavy, "bound": p_splits,
                  "workgroups": int(per_pair.sum()), "max_per_pair": int(per_pair.max())}
    elif mfma:  # per-pair split counts, as the kernel derives them (layer 0)
        splits, split_rows = attention_split_plan(q.device, b * hkv, hint, mfma,
                                                  waves=attention_waves(d, fused, b * hkv), head_dim=d)
        heavy = mfma_heavy_rows(-(-split_rows // 64) * 64, d, b * hkv)
        per_pair = torch.where(lv[0] <= split_rows, torch.ones_like(lv[0]),
                               (lv[0] + heavy - 1) // heavy).clamp(1, splits)
        splits = {"rows_per_split": split_rows, "bound": splits, "workgroups": int(per_pair.sum()),
                  "max_per_pair": int(per_pair.max())}
    achieved = bytes_per_launch / per_launch_s / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": _pmc_traffic("decode_attention_pmc_traffic.json", config),
            "kernel": ("decode_attn_mfma_kernel<fused, planned>" if plan is not None else
                       "decode_attn_mfma_kernel<fused>" if fused else
                       "decode_attn_mfma_kernel" if mfma else "decode_attn_wave_kernel"),
            "layout": "paged (16-row pages)" if bt is not None else "span",
            "avg_launch_us": round(per_launch_s * 1e6, 3),
            "bytes_per_launch": int(bytes_per_launch), "partition": splits,
            "live_tokens_per_head": {"mean": round(float(lv.float().mean()), 1), "max": int(lv.max()),
                                     "p99": int(lv.float().quantile(0.99))}}


def attention_scaling(llm, seqs, batches=(8, 32, 128), layers: int = 8, replays: int = 20):
    """The same fused decode attention kernel at larger batches: per-(seq, head)
    live counts resampled from the bench's own decode state (layer-major), one
    arena per layer (distinct memory, more than the MALL at the larger sizes),
    HIP events over graph replays of `layers` launches.  Shows how the kernel's
    HBM rate grows once a launch carries more than the c=8 step's few MB."""
    import torch
    from fastdms_amd.layers.compact_attention import fused_dms_rope_store_compact_decode_attention

    runner = llm.model_runner
    mgr = runner.compact_kv_manager
    cfg = llm.config.hf_config
    md = runner.dms_metadata
    states = [mgr.seq_states[s.seq_id] for s in seqs]
    start = mgr._contiguous_active_slot_start(states)
    pool = mgr.layer_major_live_counts[:, start:start + len(seqs)].reshape(-1).to(torch.int64).cpu()
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    cos_sin = runner.model.model.layers[0].self_attn.rotary_emb.cos_sin_cache
    dt = mgr.compact_k_per_layer[0].dtype
    gen = torch.Generator(device="cpu").manual_seed(3)
    rows = []
    for b in batches:
        live = pool[torch.randint(0, pool.numel(), (layers, b, hkv), generator=gen)].to(torch.int32)
        # the engine's paged layout: every span ceil(live / 16) pages, page ids
        # a random permutation of each layer's pool
        npg = (live.to(torch.int64) + 15) // 16
        maxp = int(npg.max())
        bt = torch.full((layers, b, hkv, maxp), -1, dtype=torch.int32)
        for l in range(layers):
            ids = torch.randperm(int(npg[l].sum()), generator=gen).to(torch.int32)
            at = 0
            for i in range(b):
                for h in range(hkv):
                    n = int(npg[l, i, h])
                    bt[l, i, h, :n] = ids[at:at + n]
                    at += n
        rows_per_layer = int(npg.sum(dim=(1, 2)).max()) * 16
        arenas = [(torch.randint(0, 120, (rows_per_layer, d), dtype=torch.uint8, device="cuda").view(dt),
                   torch.randint(0, 120, (rows_per_layer, d), dtype=torch.uint8, device="cuda").view(dt))
                  for _ in range(layers)]
        live_d, bt_d = live.cuda(), bt.cuda()
        last = (live_d - 1).long()
        slot = (torch.gather(bt_d, 3, (last // 16).unsqueeze(-1)).squeeze(-1) * 16 + last % 16).to(torch.int32)
        qkv = (torch.randn((b, (hq + 2 * hkv) * d), generator=gen) * 4).to(device="cuda", dtype=torch.bfloat16)
        q = qkv[:, :hq * d].view(b, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(b, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
        positions = torch.full((b,), 8300, device="cuda", dtype=torch.int64)
        evict = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
        out = torch.empty_like(q)
        hint = (int(live.max()) // 256 + 1) * 256

        def launch(l):
            fused_dms_rope_store_compact_decode_attention(
                q, k, v, cos_sin, arenas[l][0], arenas[l][1], slot[l], evict, positions, None, live_d[l],
                num_kv_heads=hkv, alpha_scale=md.alpha_scale, alpha_offset=md.alpha_offset, max_live_count=hint,
                out=out, block_tables=bt_d[l])

        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        with torch.inference_mode(), torch.cuda.stream(s):
            for l in range(layers):
                launch(l)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                for l in range(layers):
                    launch(l)
            g.replay()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(s)
            for _ in range(replays):
                g.replay()
            t1.record(s)
            torch.cuda.synchronize()
        per_launch_s = t0.elapsed_time(t1) / 1e3 / (replays * layers)
        elem = arenas[0][0].element_size()
        kv_bytes = int((live.to(torch.int64) - 1).clamp(min=0).sum()) * d * 2 * elem / layers
        io_bytes = (b * ((hq + 2 * hkv) * d * 2 + 2 * hkv * d * elem + hq * d * 2 + hkv * 9 + 8 + d * 4)
                    + 4 * int(npg.sum()) / layers)
        nbytes = kv_bytes + io_bytes
        achieved = nbytes / per_launch_s / 1e9
        rows.append({"batch": b, "pairs": b * hkv, "bytes_per_launch": int(nbytes),
                     "avg_launch_us": round(per_launch_s * 1e6, 2), "achieved": round(achieved, 1),
                     "frac": round(achieved / HBM_PEAK_GBPS, 4)})
        del arenas
    return {"kernel": "decode_attn_mfma_kernel<fused>", "layout": "paged (16-row pages, permuted ids)",
            "unit": "GB/s", "peak": HBM_PEAK_GBPS, "live_counts": "resampled from this run's decode state",
            "points": rows}


def _pmc_traffic(name: str, config: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by the factor the same counter
    reads for the plain copy kernel), or None when it is absent or was taken
    on another bench config."""
    path = ROOT / "profiles" / name
    try:
        d = json.loads(path.read_text())
        if "configs" in d:  # one summary per bench config
            return d["configs"][config]["traffic_bytes_per_launch"] if config in d["configs"] else None
        return d["traffic_bytes_per_launch"] if d.get("config") == config else None
    except (OSError, KeyError, ValueError, TypeError):
        return None


def _graph_time(run, replays: int) -> float:
    """Seconds per replay of a HIP graph of run()'s launches (HIP events on
    the capture stream)."""
    import torch
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.stream(s):
        run()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            run()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(replays):
            g.replay()
        e1.record(s)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / replays


def compaction_roofline(lens, replays: int = 20, layers: int = 16, config: str = "l1b-c8"):
    """Prefill compaction (A4 + A5) as the engine runs it for one layer of a
    prefill batch on the paged layout (PagedCompactKVManager.streaming_pack_layer):
    one count/scan launch that also pops each span's 16-row pages and writes
    its block-table row, and one rank-scatter launch (bf16 K/V -> FP8 pages +
    positions / evict metadata), for the bench's prompt lengths, 8 KV heads,
    D = 64, keep = last 256 tokens + 1/8 of the older ones.  One HIP graph
    packs `layers` layers with their own K/V, pools and metadata (more than the
    256 MB MALL); HIP events bracket `replays` replays (each layer's pool holds
    fresh pages for every replay).  Algorithmic bytes per layer, the
    headline `bytes` / `achieved` / `frac`: what the kernels must move --
    T*H evict bytes + live*2*D*2 kept bf16 K/V rows read + live*(2*D + 5) FP8
    rows and metadata written + the counts / offsets and two int32 per page
    (table entry, page id).  `survey_formula` gives the figure that counts
    every prompt row's K/V as read (T*H*(2*D*2 + 1) + live*(2*D + 5) +
    metadata), which the kernels never do (they read kept rows only)."""
    import numpy as np
    import torch
    from fastdms_amd import _native as nat

    h, d, window = 8, 64, 256
    nseq = len(lens)
    t_tot = int(sum(lens))
    cap = int(max(lens))
    chunks = -(-cap // 256)
    max_pages = -(-cap // 16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32).cuda()
    gen = torch.Generator(device="cuda").manual_seed(2)  # drawn on the device: no host copies
    keep_old = 0.125
    runs = replays + 3  # eager warm-up, capture (not run), first replay, timed replays
    pool = runs * sum(-(-(window + int(n * keep_old * 1.3)) // 16) for n in lens) * h
    per_layer = []
    for _ in range(layers):
        k = torch.randn((t_tot, h, d), generator=gen, device="cuda").to(torch.bfloat16)
        v = torch.randn((t_tot, h, d), generator=gen, device="cuda").to(torch.bfloat16)
        evict = (torch.rand((t_tot, h), generator=gen, device="cuda") >= keep_old).to(torch.uint8)
        ck = torch.zeros((pool * 16, d), dtype=torch.uint8, device="cuda").view(torch.float8_e4m3fn)
        cv = torch.zeros_like(ck)
        stack = torch.arange(pool, dtype=torch.int32, device="cuda")
        top = torch.full((1,), pool, dtype=torch.int32, device="cuda")
        budget = torch.full((1,), pool, dtype=torch.int32, device="cuda")  # the whole pool: nothing is reserved
        bt = torch.full((nseq, h, max_pages), -1, dtype=torch.int32, device="cuda")
        held = torch.zeros((nseq, h), dtype=torch.int32, device="cuda")
        pos = torch.full((nseq, h, cap), -1, dtype=torch.int32, device="cuda")
        em = torch.zeros((nseq, h, cap), dtype=torch.uint8, device="cuda")
        live = torch.empty((nseq, h), dtype=torch.int32, device="cuda")
        offs = torch.empty((nseq, h, chunks), dtype=torch.int32, device="cuda")
        per_layer.append((k, v, evict, ck, cv, stack, top, bt, held, pos, em, live, offs, budget))
    rows = torch.arange(nseq, dtype=torch.int32, device="cuda")
    overflow = torch.zeros(1, dtype=torch.int32, device="cuda")

    def run():
        for k, v, ev, ck, cv, stack, top, bt, held, pos, em, live, offs, budget in per_layer:
            nat.call("fdms_paged_pack_prepare", ev.data_ptr(), ev.stride(0), ev.stride(1), cu.data_ptr(), nseq,
                     window, h, chunks, live.data_ptr(), live.stride(0), live.stride(1), offs.data_ptr(),
                     offs.stride(0), offs.stride(1), offs.stride(2), pos.data_ptr(), em.data_ptr(), rows.data_ptr(),
                     pos.stride(0), pos.stride(1), em.stride(0), em.stride(1), 0, stack.data_ptr(), top.data_ptr(),
                     budget.data_ptr(), bt.data_ptr(), bt.stride(0), bt.stride(1), held.data_ptr(), held.stride(0),
                     held.stride(1), max_pages, overflow.data_ptr(), nat.stream())
            nat.call("fdms_paged_pack_scatter", k.data_ptr(), v.data_ptr(), nat.DT_BF16, k.stride(0), k.stride(1),
                     v.stride(0), v.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), cu.data_ptr(), nseq,
                     offs.data_ptr(), offs.stride(0), offs.stride(1), offs.stride(2), ck.data_ptr(), cv.data_ptr(),
                     nat.DT_FP8, ck.stride(0), pos.data_ptr(), em.data_ptr(), rows.data_ptr(), pos.stride(0),
                     pos.stride(1), pos.stride(2), em.stride(0), em.stride(1), em.stride(2), bt.data_ptr(),
                     bt.stride(0), bt.stride(1), window, h, d, chunks, 8, None, None, nat.stream())

    layer_s = _graph_time(run, replays) / layers
    if int(overflow.item()):
        raise RuntimeError("compaction roofline: a page pool ran short")
    live = sum(int(x[11].sum()) for x in per_layer) / layers
    pages = sum(int(((x[11] + 15) // 16).sum()) for x in per_layer) / layers
    meta = nseq * h * (1 + chunks) * 4 + pages * 4 * 2  # live + offsets; table entries and page ids
    algo = t_tot * h * (2 * d * 2 + 1) + live * (2 * d + 4 + 1) + meta
    kept = t_tot * h + live * 2 * d * 2 + live * (2 * d + 5) + meta
    achieved = kept / layer_s / 1e9
    del per_layer
    return {"bound": "hbm", "layout": "paged (16-row pages)",
            "kernels": "pack_prepare_kernel<paged> + pack_scatter_kernel<paged> (one prefill layer, all sequences)",
            "basis": "bytes the kernels must move per layer (evict bytes, kept bf16 K/V rows read, FP8 rows and "
                     "metadata written)",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "bytes": int(kept),
            "traffic": _pmc_traffic("compaction_pmc_traffic.json", config),
            "us_per_layer": round(layer_s * 1e6, 2), "tokens": t_tot,
            "live_rows": round(live, 1), "pages": round(pages, 1),
            "survey_formula": {"what": "every prompt row's bf16 K/V counted as read: T*H*(2*D*2+1) + "
                                       "live*(2*D+5) + metadata", "bytes": int(algo),
                               "achieved": round(algo / layer_s / 1e9, 1),
                               "frac": round(algo / layer_s / 1e9 / HBM_PEAK_GBPS, 4)}}


def expiry_roofline(replays: int = 10, layers: int = 16, seqs: int = 8, heads: int = 8, d: int = 64,
                    config: str = "l1b-c8", trials: int = 5):
    """Decode expiry A12 (the exact re-compaction the first decode step and
    every window-th step run; fdms_paged_expiry, all layers in one launch) on
    paged spans shaped like the bench's decode state: live ~ U[700, 1300] per
    (layer, seq, head), the older ranks kept prefill survivors (evict 0), the
    last 256 the in-window tokens (7/8 flagged), the step's position 64 past
    the window, so the 64 oldest window tokens expire (about 56 of them are
    flagged) and the rows after them move.  Each replay expires its own copy
    of the state (`replays` copies in one graph).  Algorithmic bytes (the
    metadata read once, each moved row read and written once): live_before * 5 metadata read + moved rows * 2 * D * 2 (K and V,
    read + write) + live_after * 5 written, summed over the spans."""
    import numpy as np
    import torch
    from fastdms_amd import _native as nat

    window, cap = 256, 1400
    rng = np.random.default_rng(4)
    live = rng.integers(700, 1301, (layers, seqs, heads)).astype(np.int32)
    cur = 8400
    pos = np.full((layers, seqs, heads, cap), -1, np.int32)
    ev = np.zeros((layers, seqs, heads, cap), np.uint8)
    moved = kept = 0
    for idx in np.ndindex(layers, seqs, heads):
        n = int(live[idx])
        old = np.sort(rng.choice(cur - window - 64, n - window, replace=False))
        pos[idx][:n] = np.concatenate([old, np.arange(cur - window - 64, cur - 64)])
        ev[idx][n - window:n] = rng.random(window) < 7 / 8
        keep = ~((ev[idx][:n] == 1) & (pos[idx][:n] < cur - window))
        first = int(np.argmin(keep)) if not keep.all() else n
        moved += int(keep[first:].sum())
        kept += int(keep.sum())
    npg = (live.astype(np.int64) + 15) // 16
    max_pages = int(npg.max())
    pages_per_layer = int(npg.sum(axis=(1, 2)).max())
    copies = []
    for _ in range(replays + 1):
        bt = np.full((layers, seqs, heads, max_pages), -1, np.int32)
        for l in range(layers):
            ids = rng.permutation(pages_per_layer).astype(np.int32)
            at = 0
            for b in range(seqs):
                for h in range(heads):
                    n = int(npg[l, b, h])
                    bt[l, b, h, :n] = ids[at:at + n]
                    at += n
        # one allocation per copy, sliced per layer and K / V, as the engine
        # holds its arenas
        arena = torch.randint(0, 120, (layers, 2, pages_per_layer * 16, d), dtype=torch.uint8, device="cuda")
        arenas = [(arena[l, 0], arena[l, 1]) for l in range(layers)]
        copies.append(dict(
            pos=torch.from_numpy(pos).cuda(), ev=torch.from_numpy(ev).cuda(), live=torch.from_numpy(live).cuda(),
            bt=torch.from_numpy(bt).cuda(), held=torch.from_numpy(npg.astype(np.int32)).cuda(),
            stack=torch.zeros((layers, pages_per_layer), dtype=torch.int32, device="cuda"),
            top=torch.zeros(layers, dtype=torch.int32, device="cuda"), arena=arena, arenas=arenas,
            pk=torch.tensor([a[0].data_ptr() for a in arenas], dtype=torch.int64, device="cuda"),
            pv=torch.tensor([a[1].data_ptr() for a in arenas], dtype=torch.int64, device="cuda")))
    curs = torch.full((seqs,), cur, dtype=torch.int64, device="cuda")
    it = iter(copies)

    def run():
        c = next(it)
        p, e, lv, bt, hd = c["pos"], c["ev"], c["live"], c["bt"], c["held"]
        nat.call("fdms_paged_expiry", 0, p.data_ptr(), p.stride(0), p.stride(1), p.stride(2), e.data_ptr(),
                 e.stride(0), e.stride(1), e.stride(2), lv.data_ptr(), lv.stride(0), lv.stride(1), lv.stride(2),
                 bt.data_ptr(), bt.stride(0), bt.stride(1), bt.stride(2), hd.data_ptr(), hd.stride(0),
                 hd.stride(1), hd.stride(2), c["stack"].data_ptr(), c["stack"].stride(0), c["top"].data_ptr(),
                 c["pk"].data_ptr(), c["pv"].data_ptr(), d, d, curs.data_ptr(), layers, seqs, heads, window,
                 nat.stream())

    run()  # warm-up on the first copy; each copy is expired once per replay
    # the timed launches, one per copy, captured in one graph: HIP events
    # around its replay time the kernels, not the host's launch calls.  The
    # graph is replayed `trials` times on the same initial states (restored
    # from clones between replays, the MALL flushed after each restore) and
    # the median replay is reported: the first replay after the set-up took
    # 40-74 us per launch depending on what the process ran before it, the
    # later ones 38-39 us.
    state_keys = ("pos", "ev", "live", "bt", "held", "stack", "top", "arena")
    pristine = [{k: c[k].clone() for k in state_keys} for c in copies[1:]]
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    times = []
    with torch.inference_mode(), torch.cuda.stream(st):  # as the engine's own captures
        with torch.cuda.graph(g, stream=st):
            for _ in range(replays):
                run()
        for t in range(trials):
            if t:
                for c, p in zip(copies[1:], pristine):
                    for k in state_keys:
                        c[k].copy_(p[k])
            _flush_mall()
            st.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            g.replay()
            e1.record(st)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) / 1e3 / replays)
    torch.cuda.synchronize()
    launch_s = float(np.median(times))
    lv_after = copies[-1]["live"].to(torch.int64).sum().item()
    if lv_after != kept:
        raise RuntimeError(f"expiry roofline: {lv_after} rows kept, expected {kept}")
    nbytes = int(live.sum()) * 5 + moved * 2 * d * 2 + kept * 5
    achieved = nbytes / launch_s / 1e9
    del copies, pristine
    return {"bound": "hbm", "layout": "paged (16-row pages)",
            "kernel": "dms_expiry_kernel<exact> (fdms_paged_expiry, all layers one launch)",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": _pmc_traffic("expiry_pmc_traffic.json", config),
            "avg_launch_us": round(launch_s * 1e6, 2),
            "bytes": nbytes, "spans": layers * seqs * heads, "live_before": int(live.sum()),
            "live_after": int(kept), "moved_rows": moved,
            "trials_us": [round(x * 1e6, 2) for x in times],
            "timing": (f"HIP events around a graph replay of {replays} launches, each on its own copy; median of "
                       f"{trials} replays of the same initial states")}


def _flush_mall(nbytes: int = 1 << 30) -> None:
    """Write 1 GiB (four times MI355X's 256 MB memory-side cache) so that the
    next timed kernels read their inputs from HBM."""
    import torch
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    torch.cuda.synchronize()
    del buf


def hbm_copy_gbps(nbytes: int = 1 << 30) -> float:
    """Achieved read+write bandwidth of the plain 16-byte copy kernel."""
    import torch
    from fastdms_amd import _native as nat
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    blocks = 256 * 16
    for _ in range(3):
        nat.call("fdms_copy_bytes", src.data_ptr(), dst.data_ptr(), nbytes, blocks, nat.stream())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    reps = 20
    for _ in range(reps):
        nat.call("fdms_copy_bytes", src.data_ptr(), dst.data_ptr(), nbytes, blocks, nat.stream())
    e1.record()
    torch.cuda.synchronize()
    return 2 * nbytes * reps / (e0.elapsed_time(e1) / 1e3) / 1e9


def counter_calibration(reps: int = 3) -> None:
    """Dispatches of known traffic for reading HBM counters (run under
    rocprofv3 --pmc): per repetition a gather and a scatter of random 64-byte
    and 128-byte rows of a 64 MiB table (16 MiB moved each) and a contiguous
    16 MiB copy, in that order."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(0)
    n = 1 << 20
    src64 = torch.randint(0, 255, (n, 64), dtype=torch.uint8, device="cuda", generator=g)
    src128 = torch.randint(0, 255, (n // 2, 128), dtype=torch.uint8, device="cuda", generator=g)
    idx64 = torch.randperm(n, device="cuda", generator=g)[: n // 4]
    idx128 = torch.randperm(n // 2, device="cuda", generator=g)[: n // 8]
    vals64 = torch.randint(0, 255, (n // 4, 64), dtype=torch.uint8, device="cuda", generator=g)
    vals128 = torch.randint(0, 255, (n // 8, 128), dtype=torch.uint8, device="cuda", generator=g)
    dst64, dst128 = torch.zeros_like(src64), torch.zeros_like(src128)
    flat = torch.empty(n // 4 * 64, dtype=torch.uint8, device="cuda")
    for _ in range(reps):
        src64[idx64]
        src128[idx128]
        dst64[idx64] = vals64
        dst128[idx128] = vals128
        flat.copy_(vals64.view(-1))
        torch.cuda.synchronize()


def cpu_baseline(llm, seqs, budget_s: float):
    """The fp32 torch-CPU oracle decoding the same batch from a copy of the
    GPU's compact state (same weights, same live spans), for ~budget_s seconds."""
    import numpy as np
    import torch
    from oracle import compact_kv as ock
    from oracle import numerics
    from oracle.model import OracleModel, weights_from_model

    torch.set_num_threads(os.cpu_count() or 1)
    runner = llm.model_runner
    mgr = runner.compact_kv_manager
    cfg = llm.config.hf_config
    md = runner.dms_metadata
    om = ock.OracleCompactKVManager(mgr.num_layers, mgr.num_kv_heads, mgr.capacity_tokens, mgr.max_model_len,
                                    head_dim=mgr.head_dim, dtype_code=numerics.DT_FP8)
    arenas_k = [t.view(torch.uint8).cpu().numpy() for t in mgr.compact_k_per_layer]
    arenas_v = [t.view(torch.uint8).cpu().numpy() for t in mgr.compact_v_per_layer]
    if mgr.paged:  # the oracle keeps flat spans: gather each span from its pages in rank order
        slots = [mgr.seq_states[s.seq_id].active_slot for s in seqs]
        caps = [mgr.seq_states[s.seq_id].max_capacity_per_lh for s in seqs]
        live_all = mgr.layer_major_live_counts.cpu().numpy()
        arenas_k, arenas_v, bases = ock.spans_from_pages(arenas_k, arenas_v, mgr.block_tables.cpu().numpy(),
                                                         live_all, slots, caps)
        om.free_ranges_per_layer = [[] for _ in range(mgr.num_layers)]
    else:
        om.free_ranges_per_layer = [list(r) for r in mgr.free_ranges_per_layer]
    om.compact_k_per_layer, om.compact_v_per_layer = arenas_k, arenas_v
    for i, s in enumerate(seqs):
        st = mgr.seq_states[s.seq_id]
        if mgr.paged:
            base, rcap = bases[i], np.full_like(bases[i], caps[i])
        else:
            base, rcap = st.base_offsets.cpu().numpy().copy(), st.range_capacity.cpu().numpy().copy()
        om.seq_states[s.seq_id] = ock.SeqState(
            s.seq_id, base, rcap, st.live_counts.cpu().numpy().copy(), st.token_positions.cpu().numpy().copy(),
            st.evict_mask.cpu().numpy().copy(), st.max_capacity_per_lh, st.decode_headroom,
            st.dms_initial_expiry_done, st.last_dms_expiry_position)
    scaled = mgr.kv_scales is not None
    orc = OracleModel(weights_from_model(runner.model), cfg, window_size=md.window_size, alpha_scale=md.alpha_scale,
                      alpha_offset=md.alpha_offset, capacity_tokens=mgr.capacity_tokens,
                      max_model_len=mgr.max_model_len, manager=om,
                      fp8_scales="calibrate" if scaled else "unit")
    if scaled:  # the GPU's per-(layer, kv head) FP8 scales, already calibrated by the prefill
        orc.kv_scales = mgr.kv_scales.cpu().numpy().copy()
        orc._calibrated = [True] * mgr.num_layers
    ids = [s.seq_id for s in seqs]
    last = [s.last_token for s in seqs]
    pos = [len(s) - 1 for s in seqs]
    steps = 0
    t0 = time.perf_counter()
    while True:
        toks = orc.decode(ids, last, pos)
        steps += 1
        last = toks
        pos = [p + 1 for p in pos]
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    # prefill: the oracle packs the first prefill_tokens of one prompt (fresh
    # compact state, same weights); tok/s = prompt tokens / wall time, as the
    # reference harness defines prefill throughput
    prefill_tokens = min(1024, len(seqs[0].prompt_token_ids))
    porc = OracleModel(orc.w, cfg, window_size=md.window_size, alpha_scale=md.alpha_scale,
                       alpha_offset=md.alpha_offset, capacity_tokens=1 << 16, max_model_len=mgr.max_model_len,
                       fp8_scales="calibrate" if scaled else "unit")
    t1 = time.perf_counter()
    porc.prefill([(0, list(seqs[0].prompt_token_ids[:prefill_tokens]), 1)])
    pdt = time.perf_counter() - t1
    return {"value": round(len(seqs) * steps / dt, 3), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu_model": _cpu_model(),
            "sample": f"{steps} decode steps of the same {len(seqs)}-sequence batch from the GPU's compact state "
                      f"after the timed steps (fp32 torch-CPU oracle, {os.cpu_count()} host cpus)",
            "prefill": {"value": round(prefill_tokens / pdt, 2), "unit": "tok/s",
                        "sample": f"one {prefill_tokens}-token prompt (the first tokens of the batch's first "
                                  f"prompt) prefilled and packed by the same oracle, all layers"}}


def _cpu_model() -> str:
    """The host CPU's model name (what lscpu reports as 'Model name')."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_decode_workload(args, config: str, *, extras: bool):
    """One BASELINE decode configuration: build, warm up, prefill the batch
    (prefill_tok_s), time args.steps decode steps of the engine (value), the
    device-side greedy loop over the rest of the generation, and the decode
    attention roofline on the live state.  With ``extras`` also the CPU
    baseline, the attention batch scaling and the compaction / expiry
    rooflines.  Returns (result dict, decode seconds)."""
    import numpy as np
    import torch
    from fastdms_amd import LLM, SamplingParams

    model, batch, lo, hi, workload = CONFIGS[config]
    model = args.model or model
    batch = args.batch or batch
    lo = args.min_prompt or lo
    hi = args.max_prompt or hi
    rng = np.random.default_rng(args.seed)
    lens = rng.integers(lo, hi + 1, batch).tolist()
    progress(f"{config}: building {model}, prompts {lens}")
    llm = LLM(model, max_model_len=hi + args.gen, max_num_seqs=batch, max_num_batched_tokens=sum(lens),
              dms_window_size=256, dms_alpha_scale=10.0, dms_alpha_offset=5.0, kv_cache_dtype="float8_e4m3fn",
              seed=args.seed, enforce_eager=args.eager, compact_kv_fp8_scales=args.kv_scales)
    vocab = llm.config.hf_config.vocab_size
    # warm-up generation of the same prompt lengths (first-call library set-up,
    # graph capture), then freed; the reference times post-warm-up as well
    progress(f"{config}: warm-up generation")
    wrng = np.random.default_rng(args.seed + 1)
    warm_sp = SamplingParams(temperature=0.0, max_tokens=2, ignore_eos=True)
    for n in lens:
        llm.add_request(wrng.integers(0, vocab, n).tolist(), warm_sp)
    while not llm.is_finished():
        llm.step()
    sp = SamplingParams(temperature=0.0, max_tokens=args.gen, ignore_eos=True)
    seqs = [llm.add_request(rng.integers(0, vocab, n).tolist(), sp) for n in lens]
    torch.cuda.synchronize()
    progress(f"{config}: prefill")
    t0 = time.perf_counter()
    llm.step()  # prefill of all prompts
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for _ in range(args.warmup):
        llm.step()
    torch.cuda.synchronize()
    progress(f"{config}: timing {args.steps} decode steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        llm.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    value = batch * args.steps / dt
    progress(f"{config}: decode {value:.1f} tok/s")
    # the engine launches a certain next decode step before reading back the
    # current one (FASTDMS_AMD_DECODE_LOOKAHEAD): finish it before driving the
    # runner directly
    llm.drain()
    fast = None
    left = min(s.max_tokens - s.num_completion_tokens for s in seqs)
    if left >= 8 and not args.no_fast_loop:  # the device-side greedy loop over the rest of the generation
        progress(f"{config}: greedy fast loop, {left} steps")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        llm.model_runner.run_compact_greedy_decode_loop(seqs, left)
        fast_dt = time.perf_counter() - t0
        fast = {"tok_s": round(batch * left / fast_dt, 2), "ms_per_step": round(fast_dt / left * 1e3, 4),
                "steps": left}
        progress(f"{config}: fast loop {fast['tok_s']:.1f} tok/s")
    out = {"value": round(value, 2), "ms_per_step": round(dt / args.steps * 1e3, 4),
           "config": {"workload": workload, "model": model, "global_batch": batch, "seq_len": int(max(lens)),
                      "prompt_lens": lens, "parallelism": "single GPU", "graphs": not args.eager,
                      "kv_scales": ("per (layer, kv head), calibrated" if args.kv_scales == "calibrate"
                                    else "unit"),
                      "linear_weights": "fp8_e4m3 (FASTDMS_FP8_WEIGHTS=1)" if os.environ.get(
                          "FASTDMS_FP8_WEIGHTS", "0").strip().lower() in ("1", "true", "yes", "on") else "bf16"},
           "prefill_tok_s": round(sum(lens) / prefill_s, 1), "decode_fast_loop": fast}
    if extras and not args.no_cpu_baseline:  # before the roofline replays re-append rows
        progress(f"{config}: cpu baseline")
        out["cpu_baseline"] = cpu_baseline(llm, seqs, args.cpu_seconds)
    progress(f"{config}: attention roofline")
    out["roofline"] = attention_roofline(llm, seqs, args.attn_replays, config)
    if extras:
        progress("attention scaling")
        out["roofline_scaling"] = attention_scaling(llm, seqs) if not args.no_scaling else None
        progress("compaction roofline")
        out["compaction_roofline"] = compaction_roofline(lens, config=config)
        progress("expiry roofline")
        out["expiry_roofline"] = expiry_roofline(config=config)
    llm.exit()
    del llm, seqs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out, dt


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    # the engine steps one token at a time here (value); the device-side
    # greedy loop is timed separately on the same batch (decode_fast_loop)
    os.environ.setdefault("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "0")
    if args.config == "multitenant":
        return run_multitenant(args)
    if args.warmup + args.steps > args.gen - 1:
        sys.exit(f"warmup + steps must be <= gen - 1 = {args.gen - 1}")
    res, _ = run_decode_workload(args, args.config, extras=True)
    # the metric names both shapes: the default run also times configs[3]
    # (Qwen3-8B shape, c=8, 8192-token prompts) with the same harness
    q8b = None
    if args.config == "l1b-c8" and not args.no_8b and not (args.model or args.batch or args.min_prompt
                                                           or args.max_prompt):
        q8b, _ = run_decode_workload(args, "q8b-c8", extras=False)
    # the plain copy kernel's read + write rate on this box, and each
    # roofline's achieved rate against it (beside frac, which is against the
    # published 8 TB/s)
    copy_gbps = round(hbm_copy_gbps(), 1)
    for r in (res.get("roofline"), (q8b or {}).get("roofline"), res.get("compaction_roofline"),
              res.get("expiry_roofline")):
        if r and r.get("achieved"):
            r["frac_of_copy"] = round(r["achieved"] / copy_gbps, 4)
    for pt in (res.get("roofline_scaling") or {}).get("points", []):
        pt["frac_of_copy"] = round(pt["achieved"] / copy_gbps, 4)
    out = {
        "metric": "decode tok/s @ctx8192 c=8 (1B/8B shapes); compact-attn HBM GB/s % of peak",
        "value": res["value"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 activations/weights, fp8_e4m3 compact KV", "data": "synthetic",
        "config": res["config"],
        "prefill_tok_s": res["prefill_tok_s"],
        "decode_fast_loop": res["decode_fast_loop"],
        "roofline": res["roofline"],
        "roofline_scaling": res.get("roofline_scaling"),
        "compaction_roofline": res.get("compaction_roofline"),
        "expiry_roofline": res.get("expiry_roofline"),
        "hbm_copy_gbps": copy_gbps,
        "cpu_baseline": res.get("cpu_baseline"),
        "q8b_c8": q8b,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
