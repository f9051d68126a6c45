"""The engine-level checks can fail.

The GPU engine tests judge the engine by (1) its free-running greedy tokens
against the model oracle's, with the previous-token plant (models/synthetic.py:
the greedy token at position p is succ[token at p - 1], retrieved by a layer-0
attention head from the compact FP8 K/V), and (2) its compact state (live
counts per layer, sequence and kv head) against the oracle's.  Here the same
two checks run on the CPU, the engine's HIP entry points emulated
(tests/native_emulator.py), once as they are and once per planted mistake in
the emulated kernels.  The unmodified engine must pass both; every mistake
must fail at least one, and each mistake on the decode attention path must
fail the greedy check itself:

* attention output zeroed, K and V swapped, q rotated one position off, the
  decode append dropped: greedy tokens (the state then diverges too, but
  only because the engine goes on from different tokens);
* the DMS window one token short (window 1 -> 0): greedy tokens -- with a
  one-token window the previous token is an out-of-window token, kept only
  if its decision says so -- and the state;
* one eviction decision dropped (a token to evict kept): the state only -- a
  token outside the window never carries the planted head's margin.
"""
from __future__ import annotations

import inspect
from dataclasses import replace

import numpy as np
import pytest
import torch

from native_emulator import Emulator, cpu_engine

WINDOW = 1
DMS = dict(dms_window_size=WINDOW, dms_alpha_scale=10.0, dms_alpha_offset=5.0)
GEN = 8
LENS = [40, 57, 33]


def _args(emu, name, a, k):
    """The bound arguments of emulator entry point `name` (by parameter name)."""
    return inspect.signature(getattr(Emulator, name).__get__(emu)).bind(*a, **k).arguments


def _wrap(emu, name, fn):
    orig = getattr(emu, name)
    setattr(emu, name, lambda *a, **k: fn(orig, *a, **k))


def _zero_attention(emu):
    def fn(orig, *a, **k):
        rc = orig(*a, **k)
        p = _args(emu, "compact_decode_attention", a, k)
        emu.view(p["out"], torch.bfloat16, (p["B"], p["H"] * p["G"], p["D"]), (p["os_b"], p["os_h"], 1),
                 "out").zero_()
        return rc
    _wrap(emu, "compact_decode_attention", fn)


def _swap_kv(emu):
    def fn(orig, *a, **k):
        p = _args(emu, "compact_decode_attention", a, k)
        p["ck"], p["cv"] = p["cv"], p["ck"]
        return orig(**p)
    _wrap(emu, "compact_decode_attention", fn)


def _shift_q_rope(emu):
    def fn(orig, *a, **k):
        p = _args(emu, "compact_decode_attention", a, k)
        if not p["rope_pos"]:
            return orig(*a, **k)
        pos = emu.view(p["rope_pos"], torch.int64, (p["B"],), (1,), "rope_positions")
        pos += 1
        try:
            return orig(*a, **k)
        finally:
            pos -= 1
    _wrap(emu, "compact_decode_attention", fn)


def _drop_append(emu):
    """The decode append leaves the rows at its slots as they were."""
    def fn(orig, *a, **k):
        p = _args(emu, "dms_rope_store_compact_decode", a, k)
        sl = emu.view(p["slot"], torch.int32, (p["B"], p["H"]), (p["sm_b"], p["sm_h"]), "slot")
        saved = []
        for ptr in (p["ck"], p["cv"]):
            flat, off = emu.flat_at(ptr, torch.uint8, "arena")
            for r in sl.flatten().tolist():
                if r >= 0:
                    idx = off + r * p["c_s"] + torch.arange(p["D"])
                    saved.append((flat, idx, flat[idx].clone()))
        rc = orig(*a, **k)
        for flat, idx, old in saved:
            flat[idx] = old
        return rc
    _wrap(emu, "dms_rope_store_compact_decode", fn)


def _short_window(emu):
    """Every kernel that applies the DMS window uses one token less (the paged
    entry points delegate to these three)."""
    for name in ("streaming_pack_prepare", "streaming_pack_rank_scatter", "dms_expiry"):
        def fn(orig, *a, _name=name, **k):
            p = _args(emu, _name, a, k)
            p["window"] = p["window"] - 1
            return orig(**p)
        _wrap(emu, name, fn)


def _drop_one_eviction(emu):
    """The first prefill decision of layer 0 that evicts an out-of-window
    token of kv head 0 in the first prompt is flipped to keep."""
    state = {"done": False}

    def fn(orig, *a, **k):
        rc = orig(*a, **k)
        if not state["done"]:
            state["done"] = True
            p = _args(emu, "extract_dms_decisions", a, k)
            ev = emu.view(p["evict"], torch.uint8, (p["T"], p["H"]), (p["es_t"], p["es_h"]), "evict")
            first = next(t for t in torch.nonzero(ev[:, 0]).flatten().tolist() if t < LENS[0] - 1 - WINDOW)
            ev[first, 0] = 0
        return rc
    _wrap(emu, "extract_dms_decisions", fn)


MUTATIONS = {
    "attention output zeroed": (_zero_attention, {"greedy"}),
    "K and V swapped": (_swap_kv, {"greedy"}),
    "q RoPE one position off": (_shift_q_rope, {"greedy"}),
    "decode append dropped": (_drop_append, {"greedy"}),
    "DMS window one token short": (_short_window, {"greedy", "state"}),
    "one eviction dropped": (_drop_one_eviction, {"state"}),
}


def _run(mutation=None):
    """Greedy generation through the emulated engine and the oracle, step by
    step; returns the set of checks that failed."""
    from engine_oracle import oracle_for
    from fastdms_amd import LLM, SamplingParams
    from fastdms_amd.models.synthetic import PRESETS
    failed = set()
    with cpu_engine() as emu:
        if mutation is not None:
            mutation(emu)
        cfg = replace(PRESETS["tiny-llama"], successor_margin=1.0)
        llm = LLM(cfg, max_model_len=256, max_num_seqs=4, max_num_batched_tokens=4096, enforce_eager=True,
                  fused_greedy_head=True, seed=3, **DMS)
        runner = llm.model_runner
        orc = oracle_for(runner, llm.config, quant=False, dms=DMS)
        rng = np.random.default_rng(11)
        prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in LENS]
        sp = SamplingParams(temperature=0.0, max_tokens=GEN, ignore_eos=True)
        seqs = [llm.add_request(p, sp) for p in prompts]
        ids = [s.seq_id for s in seqs]
        llm.step()
        want = [[int(t)] for t in orc.prefill([(s.seq_id, s.prompt_token_ids, GEN) for s in seqs])]

        def compare():
            if [s.completion_token_ids for s in seqs] != want:
                failed.add("greedy")
            mgr = runner.compact_kv_manager
            for s in seqs:
                if s.seq_id in mgr.seq_states:
                    got = mgr.seq_states[s.seq_id].live_counts[0].tolist()
                    if got != orc.mgr.seq_states[s.seq_id].live_counts[0].tolist():
                        failed.add("state")

        compare()
        for _ in range(GEN - 1):
            toks = orc.decode(ids, [w[-1] for w in want],
                              [len(p) + len(w) - 1 for p, w in zip(prompts, want)])
            for w, t in zip(want, toks):
                w.append(int(t))
            llm.step()
            compare()
        llm.exit()
    return failed


def test_unmodified_engine_passes_both_checks(monkeypatch):
    monkeypatch.setenv("FASTDMS_AMD_DECODE_LOOKAHEAD", "0")
    assert _run() == set()


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_fails_a_check(monkeypatch, name):
    monkeypatch.setenv("FASTDMS_AMD_DECODE_LOOKAHEAD", "0")
    mutation, must_fail = MUTATIONS[name]
    failed = _run(mutation)
    assert must_fail <= failed, f"{name}: failed checks {sorted(failed)}, expected {sorted(must_fail)}"
