"""Engine parity at the benchmark model shapes: the Llama-3.2-1B shape (all
16 layers), the Qwen3-8B shape (hidden 4096, QK-norm, head_dim 128, 4 of its
36 layers) and the W4A16 weights of the multitenant configuration, each with
the benchmark's DMS rule (window 256, alpha 10 / 5, about 1/8 of
out-of-window tokens kept) and FP8 compact KV, against the CPU model oracle
(oracle/model.py).

Two checks per configuration:

* logits: every step's logits (prefill, then 31 decode steps, the oracle
  decoding from the GPU's compact state) within a relative-RMS tolerance of
  the oracle's (the random model; see LOGIT_CASES for the tolerances);
* tokens: the north star's criterion, the first 32 greedy tokens of every
  sequence identical to the oracle's, free running, on the production path
  (HIP graphs, LM head fused with the greedy argmax, the device-side greedy
  loop for a lone sequence).  No mismatch is allowed (the reference's guard
  allows one, check_dms_compact_guard.py:53).  Random weights give nearly
  flat logits (the top two of 128 256 are typically 1-2 bf16 ulps apart), on
  which two correct implementations that round differently cannot agree, so
  this check runs the same shapes with the previous-token plant
  (ModelConfig.successor_margin, models/synthetic.py): a layer-0 head that
  attends to the previous token through RoPE and a successor table in the LM
  head, so the greedy token at position p is succ[token at p - 1] by a margin
  of about ten logits, and it is retrieved by the decode attention from the
  FP8 K/V the previous step appended -- a mistake in the attention, RoPE,
  appends or page addressing changes the tokens (CPU mutation test:
  tests/test_greedy_check_mutations.py).  The smallest oracle top-2 gap is
  reported.

Prompt lengths are shorter than the benchmark's 4-8K so that the fp32 CPU
oracle finishes in seconds; every prompt crosses the DMS window, so the
compact pack, decode expiry and append all take part.
"""
from __future__ import annotations

import os
from dataclasses import replace

import numpy as np
import pytest
import torch

from engine_oracle import oracle_for
from oracle_sync import sync_oracle_state

from helpers import require_gpu

pytestmark = pytest.mark.gpu

DMS = dict(dms_window_size=256, dms_alpha_scale=10.0, dms_alpha_offset=5.0)
GEN = 32


def _model_config(name: str, layers: int | None):
    from fastdms_amd.models.synthetic import PRESETS
    cfg = PRESETS[name]
    return replace(cfg, num_hidden_layers=layers) if layers else replace(cfg)


def _oracle_for(runner, config, *, quant: bool):
    return oracle_for(runner, config, quant=quant, dms=DMS)


SUCCESSOR_MARGIN = 1.0

QUANT_ENV = {"FASTDMS_FP8_WEIGHTS": "1", "FASTDMS_FP8_WEIGHT_SCOPE": "all", "FASTDMS_FP8_LM_HEAD": "0",
             "FASTDMS_INT4_ROW1_WEIGHTS": "1", "FASTDMS_INT4_ROW1_SCOPE": "all",
             "FASTDMS_INT4_ROW1_GROUP_SIZE": "128", "FASTDMS_INT4_ROW1_QUANT_MODE": "symmetric",
             "FASTDMS_INT4_ROW1_MAX_ROWS": "8"}
# FP8 weights on every linear (the reference's FASTDMS_FP8_WEIGHTS=1 with its
# attention-full default): decode rows on the small-M FP8 kernel with dynamic
# activation quantisation, prefill rows on the FP8 GEMM
FP8_ENV = {"FASTDMS_FP8_WEIGHTS": "1", "FASTDMS_FP8_WEIGHT_SCOPE": "all", "FASTDMS_FP8_LM_HEAD": "0"}
QUANT_ENVS = {"w4a16": QUANT_ENV, "fp8": FP8_ENV}


def _set_quant_env(monkeypatch, quant):
    for k, v in QUANT_ENVS.get(quant, {}).items():
        monkeypatch.setenv(k, v)


def _run(model_cfg, lens, *, seed=0, quant=False, layout="paged", with_oracle=True):
    from fastdms_amd import LLM, SamplingParams
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, model_cfg.vocab_size, n).tolist() for n in lens]
    llm = LLM(model_cfg, max_model_len=max(lens) + GEN + 8, max_num_seqs=len(lens),
              max_num_batched_tokens=sum(lens), seed=seed, compact_kv_layout=layout, **DMS)
    sp = SamplingParams(temperature=0.0, max_tokens=GEN, ignore_eos=True)
    got = [o["token_ids"] for o in llm.generate(prompts, sp)]
    orc = _oracle_for(llm.model_runner, llm.config, quant=bool(quant)) if with_oracle else None
    llm.exit()
    del llm
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    print(f"engine done: {len(lens)} prompts {lens}", flush=True)
    if orc is None:
        return got, None, None

    ids = list(range(len(lens)))
    toks = orc.prefill([(i, p, GEN) for i, p in zip(ids, prompts)])
    print("oracle prefill done", flush=True)
    want = [[t] for t in toks]
    gaps = [[_top2_gap(orc.last_logits[i])] for i in ids]
    for step in range(GEN - 1):
        if step % 8 == 7:
            print(f"oracle decode step {step + 1}", flush=True)
        pos = [len(p) + step for p in prompts]
        toks = orc.decode(ids, toks, pos)
        for i, t in enumerate(toks):
            want[i].append(t)
            gaps[i].append(_top2_gap(orc.last_logits[i]))
    return got, want, gaps


def _top2_gap(logits: torch.Tensor) -> float:
    top = torch.topk(logits.float(), 2).values
    return float(top[0] - top[1])


def _check(got, want, gaps, what):
    report = []
    for i, (g, w) in enumerate(zip(got, want)):
        first = next((j for j, (a, b) in enumerate(zip(g, w)) if a != b), None)
        if first is not None:
            report.append(f"seq {i}: first mismatch at token {first} (oracle top-2 gap {gaps[i][first]:.4g}); "
                          f"min gap before it {min(gaps[i][:first + 1]):.4g}")
    min_gap = min(min(g) for g in gaps)
    print(f"{what}: {len(got)} sequences x {GEN} tokens, {len(report)} with a mismatch; "
          f"smallest oracle top-2 logit gap {min_gap:.4g}", flush=True)
    assert all(len(g) == GEN for g in got)
    assert not report, "\n".join(report)


def _sync_oracle_state(orc, mgr, seq_ids):
    """Give the oracle the GPU's compact state (arenas, spans, live counts,
    positions, decisions), so its next decode step starts from the same KV."""
    sync_oracle_state(orc, mgr, seq_ids)


def _follow(model_cfg, lens, *, seed=0, quant=False, steps=GEN - 1):
    """Teacher-forced logits: the engine decodes step by step (logits
    materialised); before each step the oracle takes the GPU's compact state
    and the engine's last tokens.  Returns per-step (rel-RMS, max-abs-rel)."""
    from fastdms_amd import LLM, SamplingParams
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, model_cfg.vocab_size, n).tolist() for n in lens]
    llm = LLM(model_cfg, max_model_len=max(lens) + GEN + 8, max_num_seqs=len(lens),
              max_num_batched_tokens=sum(lens), seed=seed, fused_greedy_head=False, **DMS)
    runner = llm.model_runner
    orc = _oracle_for(runner, llm.config, quant=bool(quant))
    sp = SamplingParams(temperature=0.0, max_tokens=steps + 1, ignore_eos=True)
    seqs = [llm.add_request(p, sp) for p in prompts]
    llm.step()  # prefill
    orc.prefill([(s.seq_id, s.prompt_token_ids, steps + 1) for s in seqs])
    errors = []

    def logit_error():
        got = runner.model.lm_head.last_logits.float().cpu()
        want = orc.last_logits
        assert torch.isfinite(got).all(), "non-finite logits"
        rms = float((got - want).pow(2).mean().sqrt()) / max(1e-6, float(want.pow(2).mean().sqrt()))
        mx = float((got - want).abs().max()) / max(1e-6, float(want.abs().max()))
        errors.append((rms, mx))

    logit_error()
    for _ in range(steps):
        torch.cuda.synchronize()
        _sync_oracle_state(orc, runner.compact_kv_manager, [s.seq_id for s in seqs])
        orc.decode([s.seq_id for s in seqs], [s.last_token for s in seqs], [len(s) - 1 for s in seqs])
        llm.step()
        logit_error()
    llm.exit()
    del llm
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    print(f"logits {lens}: rel-RMS max {max(e[0] for e in errors):.2e}, max-abs-rel max "
          f"{max(e[1] for e in errors):.2e} over {len(errors)} steps; per step rel-RMS "
          f"{[round(e[0], 4) for e in errors]}", flush=True)
    return errors


def _check_logits(errors, tol, prefill_tol=None):
    """errors[0] is the prefill step, the rest decode steps."""
    pt = tol if prefill_tol is None else prefill_tol
    assert errors[0][0] <= pt and errors[0][1] <= 2 * pt, errors[0]
    assert max(e[0] for e in errors[1:]) <= tol
    assert max(e[1] for e in errors[1:]) <= 2 * tol


L1B = ("llama-3.2-1b", None)
Q8B4 = ("qwen3-8b", 4)
CASES = {
    "l1b_c1": (L1B, [2048], False),
    "l1b_c8": (L1B, np.random.default_rng(2).integers(300, 900, 8).tolist(), False),
    "q8b4_c8": (Q8B4, np.random.default_rng(3).integers(300, 600, 8).tolist(), False),
    "l1b_w4a16_c4": (L1B, np.random.default_rng(4).integers(300, 700, 4).tolist(), "w4a16"),
    "l1b4_fp8_c4": (("llama-3.2-1b", 4), np.random.default_rng(5).integers(300, 600, 4).tolist(), "fp8"),
}


# Tolerances of the logit comparison.  A random-weight network of this depth
# amplifies rounding: on the CPU oracle alone, moving 0.1 % of layer 0's
# o_proj outputs by one bf16 ulp moves the Llama-3.2-1B-shape logits by 1.9 %
# relative RMS after 16 layers (0.8 % from layer 8, 0.15 % from layer 15) and
# flips about a dozen DMS decisions.  Two correct implementations that round
# in a different order therefore differ by a few percent at full depth, and
# the full-depth cases get 5 %; the same widths with 2 layers, where that
# amplification is small, are held to 1 %.  The W4A16 configuration runs its
# prefill rows through FP8 linears (the reference's _scaled_mm path for rows
# above the INT4 row limit) with per-row dynamic activation quantisation: an
# activation that upstream rounding moved across an e4m3 rounding boundary
# changes by a whole FP8 step (6-12 %), so its prefill logits get 10 % (2
# layers) / 30 % (16 layers); its decode steps (INT4 rows) keep 1 % / 5 %.
# With FP8 weights everywhere the decode rows quantise their activations too
# and get the prefill's tolerance.
LOGIT_CASES = {
    "l1b_c1": (CASES["l1b_c1"], 5e-2, None),
    "l1b_c8": (CASES["l1b_c8"], 5e-2, None),
    "q8b4_c8": (CASES["q8b4_c8"], 5e-2, None),
    "l1b_w4a16_c4": (CASES["l1b_w4a16_c4"], 5e-2, 0.3),
    "l1b2_c8": ((("llama-3.2-1b", 2),) + CASES["l1b_c8"][1:], 1e-2, None),
    "q8b2_c8": ((("qwen3-8b", 2),) + CASES["q8b4_c8"][1:], 1e-2, None),
    "l1b2_w4a16_c4": ((("llama-3.2-1b", 2),) + CASES["l1b_w4a16_c4"][1:], 1e-2, 0.1),
    "l1b2_fp8_c8": ((("llama-3.2-1b", 2),) + CASES["l1b_c8"][1:2] + ("fp8",), 0.1, 0.1),
}


@pytest.mark.parametrize("case", sorted(LOGIT_CASES))
def test_logits_follow_the_oracle_at_baseline_shapes(monkeypatch, case):
    """configs[1] (l1b_c1), [2] (l1b_c8, ragged), [3] (q8b4_c8) and [4]'s
    W4A16 weights (l1b_w4a16_c4), and 2-layer models of the same widths:
    per-step logits against the oracle."""
    require_gpu()
    ((name, layers), lens, quant), tol, prefill_tol = LOGIT_CASES[case]
    monkeypatch.setenv("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "0")
    _set_quant_env(monkeypatch, quant)
    _check_logits(_follow(_model_config(name, layers), lens, seed=7, quant=quant), tol, prefill_tol)


@pytest.mark.parametrize("case", sorted(CASES))
def test_first_32_greedy_tokens_match_the_oracle_at_baseline_shapes(monkeypatch, case):
    """The same configurations on the production decode path, free running,
    with the planted successor margin: the first 32 greedy tokens of every
    sequence are the oracle's."""
    require_gpu()
    (name, layers), lens, quant = CASES[case]
    _set_quant_env(monkeypatch, quant)
    cfg = replace(_model_config(name, layers), successor_margin=SUCCESSOR_MARGIN)
    got, want, gaps = _run(cfg, lens, seed=1, quant=quant)
    _check(got, want, gaps, case)
    assert min(min(g) for g in gaps) >= 0.5, "the planted margin did not hold"


@pytest.mark.parametrize("case", ["l1b_c8", "q8b4_c8"])
def test_span_layout_gives_the_paged_layouts_tokens(case):
    """The reference's flat-span layout and the paged layout hold the same
    ranks, so the engine's first 32 greedy tokens agree token for token (and
    with the oracle's)."""
    require_gpu()
    (name, layers), lens, quant = CASES[case]
    cfg = replace(_model_config(name, layers), successor_margin=SUCCESSOR_MARGIN)
    span, want, gaps = _run(cfg, lens, seed=1, quant=quant, layout="span")
    _check(span, want, gaps, case + " span")
    paged, _, _ = _run(cfg, lens, seed=1, quant=quant, layout="paged", with_oracle=False)
    assert paged == span
