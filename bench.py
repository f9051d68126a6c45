#!/usr/bin/env python3
"""Compact-DMS decode throughput on one MI355X.

Workload: Llama-3.2-1B-shaped model with random bf16
weights, DMS window 256 / threshold 0.5 (~1/8 of tokens outside the window
survive), FP8 compact KV; 8 requests with prompt lengths uniform in
[4096, 8192] and uniform-random token ids, 128 greedy tokens each.  The 8
prompts are prefilled together (untimed), then one "step" is one decode step of
the 8-sequence batch: expiry policy, DMS decision + RoPE + FP8 append, compact
attention and the full model forward, greedy argmax and decision recording.

Prints one JSON line:
  value            decode tok/s over the K timed steps (inputs resident in HBM)
  roofline         the compact decode attention kernel: algorithmic bytes per
                   launch / average launch time, measured with HIP events around
                   graph replays of that kernel on the live decode state
  cpu_baseline     the fp32 torch-CPU oracle (oracle/model.py) decoding the same
                   batch from the same compact state on the host cores
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


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--min-prompt", type=int, default=4096)
    p.add_argument("--max-prompt", type=int, default=8192)
    p.add_argument("--gen", type=int, default=128)
    p.add_argument("--model", default="llama-3.2-1b")
    p.add_argument("--attn-replays", type=int, default=50)
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--eager", action="store_true", help="decode without HIP graphs")
    return p.parse_args()


def attention_roofline(llm, seqs, replays: int):
    """Average duration and algorithmic HBM bytes of the compact decode attention
    kernel on the live decode state: one graph holds the kernel of every layer
    with the exact decode-step arguments; HIP events bracket `replays` replays."""
    import torch
    from fastdms_amd.layers.compact_attention import (attention_split_plan, compact_decode_attention,
                                                      mfma_attention_path)

    runner = llm.model_runner
    mgr = runner.compact_kv_manager
    cfg = llm.config.hf_config
    states = [mgr.seq_states[s.seq_id] for s in seqs]
    start = mgr._contiguous_active_slot_start(states)
    b = len(seqs)
    base = mgr.layer_major_base_offsets[:, start:start + b]
    live = mgr.layer_major_live_counts[:, start:start + b]
    hint = runner.attention_hint(seqs)  # the bound (and so the split count) the decode step uses
    q = torch.randn((b, cfg.num_attention_heads, cfg.head_dim), device="cuda").to(torch.bfloat16)
    layers = list(range(cfg.num_hidden_layers))
    arenas = [(mgr.compact_k_per_layer[l], mgr.compact_v_per_layer[l]) for l in layers]
    g = torch.cuda.CUDAGraph()
    with torch.inference_mode():  # the engine's tensors are inference tensors
        for l in layers:  # warm-up outside capture
            compact_decode_attention(q, arenas[l][0], arenas[l][1], base[l], live[l], max_live_count=hint)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for l in layers:
                compact_decode_attention(q, arenas[l][0], arenas[l][1], base[l], live[l], max_live_count=hint)
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(replays):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    per_launch_s = t0.elapsed_time(t1) / 1e3 / (replays * len(layers))
    lv = live.to(torch.int64).cpu()
    kv_bytes = int(lv.sum()) * cfg.head_dim * 2 * arenas[0][0].element_size()   # K and V rows read
    qo_bytes = 2 * b * cfg.num_attention_heads * cfg.head_dim * 2                # q read + out write (bf16)
    meta_bytes = 2 * 4 * b * cfg.num_key_value_heads * len(layers)               # base + live (int32)
    bytes_per_launch = (kv_bytes + qo_bytes * len(layers) + meta_bytes) / len(layers)
    mfma = mfma_attention_path(q, arenas[0][0], cfg.num_attention_heads // cfg.num_key_value_heads)
    splits, split_rows = attention_split_plan(q.device, b * cfg.num_key_value_heads, hint, mfma)
    if split_rows:  # per-pair split counts, as the kernel derives them
        splits = int(((lv + split_rows - 1) // split_rows).clamp(1, splits).max())
    achieved = bytes_per_launch / per_launch_s / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "decode_attn_mfma_kernel" if mfma else "decode_attn_wave_kernel",
            "avg_launch_us": round(per_launch_s * 1e6, 3),
            "bytes_per_launch": int(bytes_per_launch), "splits": splits,
            "live_tokens_mean_per_head": round(float(lv.float().mean()), 1)}


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
    om.free_ranges_per_layer = [list(r) for r in mgr.free_ranges_per_layer]
    om.compact_k_per_layer = [t.view(torch.uint8).cpu().numpy() for t in mgr.compact_k_per_layer]
    om.compact_v_per_layer = [t.view(torch.uint8).cpu().numpy() for t in mgr.compact_v_per_layer]
    for s in seqs:
        st = mgr.seq_states[s.seq_id]
        om.seq_states[s.seq_id] = ock.SeqState(
            s.seq_id, st.base_offsets.cpu().numpy().copy(), st.range_capacity.cpu().numpy().copy(),
            st.live_counts.cpu().numpy().copy(), st.token_positions.cpu().numpy().copy(),
            st.evict_mask.cpu().numpy().copy(), st.max_capacity_per_lh, st.decode_headroom,
            st.dms_initial_expiry_done, st.last_dms_expiry_position)
    orc = OracleModel(weights_from_model(runner.model), cfg, window_size=md.window_size, alpha_scale=md.alpha_scale,
                      alpha_offset=md.alpha_offset, capacity_tokens=mgr.capacity_tokens,
                      max_model_len=mgr.max_model_len, manager=om)
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
    return {"value": round(len(seqs) * steps / dt, 3), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{steps} decode steps of the same {len(seqs)}-sequence batch from the GPU's compact state "
                      f"after the timed steps (fp32 torch-CPU oracle, {os.cpu_count()} host cpus)"}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from fastdms_amd import LLM, SamplingParams

    if args.warmup + args.steps > args.gen - 1:
        sys.exit(f"warmup + steps must be <= gen - 1 = {args.gen - 1}")
    rng = np.random.default_rng(args.seed)
    lens = rng.integers(args.min_prompt, args.max_prompt + 1, args.batch).tolist()
    llm = LLM(args.model, max_model_len=args.max_prompt + args.gen, max_num_seqs=args.batch,
              max_num_batched_tokens=sum(lens), dms_window_size=256, dms_alpha_scale=10.0, dms_alpha_offset=5.0,
              kv_cache_dtype="float8_e4m3fn", seed=args.seed, enforce_eager=args.eager)
    vocab = llm.config.hf_config.vocab_size
    sp = SamplingParams(temperature=0.0, max_tokens=args.gen, ignore_eos=True)
    seqs = [llm.add_request(rng.integers(0, vocab, n).tolist(), sp) for n in lens]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    llm.step()  # prefill of all 8 prompts
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for _ in range(args.warmup):
        llm.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        llm.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    value = args.batch * args.steps / dt
    roof = attention_roofline(llm, seqs, args.attn_replays)
    copy_bw = hbm_copy_gbps()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(llm, seqs, args.cpu_seconds)
    out = {
        "metric": "decode tok/s @ctx8192 c=8 (1B/8B shapes); compact-attn HBM GB/s % of peak",
        "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 activations/weights, fp8_e4m3 compact KV", "data": "synthetic",
        "config": {"workload": "BASELINE configs[2]: Llama-3.2-1B shape, c=8 ragged prompts U[4096,8192], "
                               "128 greedy tokens, DMS window 256 thr 0.5",
                   "model": args.model, "global_batch": args.batch, "seq_len": int(max(lens)),
                   "prompt_lens": lens, "parallelism": "single GPU", "graphs": not args.eager},
        "prefill_tok_s": round(sum(lens) / prefill_s, 1),
        "roofline": roof,
        "hbm_copy_gbps": round(copy_bw, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    llm.exit()


if __name__ == "__main__":
    main()
