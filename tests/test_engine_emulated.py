"""The engine's host glue, end to end on the CPU.

The model runner, compact-KV manager, scheduler and layers run unchanged; each
HIP entry point is replaced by tests/native_emulator.py, which bounds-checks
every access the kernel would make against the buffer it was handed and fills
fresh allocations with NaN bytes so that reading memory nobody wrote poisons
the logits.  The engine is then teacher-forced against the CPU model oracle
(oracle/model.py): prefill and every decode step must give the oracle's logits
within bf16 noise.  This pins the glue — strides, slot mapping, metadata rows,
expiry policy, append/record order — independently of the kernels, which the
GPU tests pin one by one.
"""
import numpy as np
import pytest
import torch

from native_emulator import cpu_engine
from paged_invariants import check_page_invariants
from oracle import linear as olin

DMS = dict(dms_window_size=32, dms_alpha_scale=10.0, dms_alpha_offset=5.0)


def _check_logits(got: torch.Tensor, want: torch.Tensor, what: str):
    got = got.float()
    assert torch.isfinite(got).all(), f"{what}: non-finite logits"
    scale = max(1.0, float(want.abs().max()))
    err = float((got - want).abs().max())
    assert err <= 2e-2 * scale, f"{what}: max |logit diff| {err:.4g} (scale {scale:.3g})"


@pytest.mark.parametrize("layout", ["paged", "span"])
@pytest.mark.parametrize("model,lens,gen", [("tiny-llama", [300, 517, 800, 64], 40),
                                            ("tiny-qwen3", [129, 700], 12),
                                            ("tiny-llama", [40], 6)])
def test_engine_glue_matches_oracle(model, lens, gen, layout):
    _run(model, lens, gen, fused_head=False, layout=layout)


@pytest.mark.parametrize("model,lens,gen", [("tiny-llama", [300, 517, 64], 10), ("tiny-qwen3", [129, 700], 8)])
def test_norm_stats_decode_matches_oracle(monkeypatch, model, lens, gen):
    """The decode step with the RMSNorms split between the linears around them
    (o_proj / down_proj finish the residual add and the row sums of squares,
    qkv / gate_up apply the norm: fdms_linear_small_m epilogue 4 / prologue 2;
    the default at hidden sizes from 4096) against the oracle's logits, and
    that path is the one that ran."""
    monkeypatch.setenv("FASTDMS_AMD_NORM_STATS", "1")
    calls = _run(model, lens, gen, fused_head=False)
    assert "fdms_linear_small_m:norm_stats" in calls and "fdms_linear_small_m:residual_stats" in calls


@pytest.mark.parametrize("model,lens,gen", [("tiny-llama", [300, 517, 64], 12), ("tiny-qwen3", [129, 700], 8)])
def test_engine_fused_greedy_head_matches_oracle_tokens(monkeypatch, model, lens, gen):
    """Decode with the LM-head GEMV fused with the argmax: no logits, tokens
    equal to the oracle model's greedy tokens step for step.  (The compact
    state is compared after every step, so no step may run ahead.)"""
    monkeypatch.setenv("FASTDMS_AMD_DECODE_LOOKAHEAD", "0")
    _run(model, lens, gen, fused_head=True)


@pytest.mark.parametrize("layout", ["paged", "span"])
def test_decode_lookahead_gives_the_oracle_tokens(layout):
    """With the decode lookahead (the next step of a certain batch launched
    before the current step's ids are read back; paged layout only) every
    step still returns the oracle's greedy tokens -- those of the steps
    launched ahead included, so their appends and expiry decisions are the
    oracle's -- and the last step launches nothing ahead."""
    calls = _run("tiny-llama", [300, 517, 64], 10, fused_head=True, layout=layout, lookahead=True)
    assert calls.count("lookahead") == (8 if layout == "paged" else 0)


def _lookahead_probe(runner, calls):
    """Record each decode step that launched the next one ahead."""
    orig = runner._lookahead_ok

    def probe(seqs):
        ok = orig(seqs)
        if ok:
            calls.append("lookahead")
        return ok
    runner._lookahead_ok = probe


FP8_ENV = {"FASTDMS_FP8_WEIGHTS": "1", "FASTDMS_FP8_WEIGHT_SCOPE": "all", "FASTDMS_FP8_LM_HEAD": "0"}


def test_fp8_decode_glue_matches_the_quantised_oracle(monkeypatch):
    """FP8 weights on every linear (the reference's FASTDMS_FP8_WEIGHTS=1 with
    its attention-full default): prefill rows on the FP8 GEMM, decode rows on
    the small-M kernel, which takes each activation's row amax from its
    producer (the RMSNorms, which also quantise qkv's and gate_up's input;
    gate_up for down_proj) and leaves o_proj's and down_proj's split merge and
    FP8 scaling to the next RMSNorm.  Logits follow
    the oracle holding the same FP8 weights and routes, and the emulator checks
    that every amax handed to a linear is its activation's own."""
    for k, v in FP8_ENV.items():
        monkeypatch.setenv(k, v)
    calls = _run("tiny-llama", [300, 517, 64], 8, fused_head=False, quant=True)
    for tag in ("x_amax", "x_amax:fp8_x", "fp8_partials"):
        assert "fdms_linear_small_m:" + tag in calls, tag


INT4_ENV = dict(FP8_ENV, FASTDMS_INT4_ROW1_WEIGHTS="1", FASTDMS_INT4_ROW1_SCOPE="all",
                FASTDMS_INT4_ROW1_GROUP_SIZE="128", FASTDMS_INT4_ROW1_QUANT_MODE="symmetric",
                FASTDMS_INT4_ROW1_MAX_ROWS="16")


def test_int4_decode_glue_matches_the_quantised_oracle(monkeypatch):
    """W4A16 decode linears (the reference's FASTDMS_INT4_ROW1_* switches, as
    configs[4] runs them; FP8 rows for the prefill): o_proj's and down_proj's
    split partials go to the next RMSNorm, as on the bf16 path.  Logits follow
    the oracle holding the same dequantised INT4 weights and routes."""
    for k, v in INT4_ENV.items():
        monkeypatch.setenv(k, v)
    calls = _run("tiny-llama", [300, 517, 64], 8, fused_head=False, quant=True)
    assert "fdms_linear_int4_small_m:partials" in calls


def _run(model, lens, gen, fused_head, layout="paged", quant=False, lookahead=False):
    """lookahead: the decode lookahead runs (the compact state is then one
    step ahead between steps and is compared once the sequences finish)."""
    from engine_oracle import oracle_for
    probe: list[str] = []
    with cpu_engine() as emu:
        from fastdms_amd import LLM, SamplingParams
        llm = LLM(model, max_model_len=2048, max_num_seqs=8, max_num_batched_tokens=16384, enforce_eager=True,
                  fused_greedy_head=fused_head, compact_kv_layout=layout, **DMS)
        runner = llm.model_runner
        if lookahead:
            _lookahead_probe(runner, probe)
        orc = oracle_for(runner, llm.config, quant=quant, dms=DMS)
        rng = np.random.default_rng(3)
        sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
        seqs = [llm.add_request(rng.integers(0, 512, n).tolist(), sp) for n in lens]
        llm.step()
        orc.prefill([(s.seq_id, s.prompt_token_ids, gen) for s in seqs])
        if fused_head:
            want = olin.argmax_lowest(orc.last_logits.float().numpy()).tolist()
            assert [s.completion_token_ids[0] for s in seqs] == want, "prefill tokens"
        else:
            _check_logits(runner.model.lm_head.last_logits, orc.last_logits, "prefill")
        for step in range(gen - 1):
            pos = [len(s) - 1 for s in seqs]
            last = [s.last_token for s in seqs]
            o_tok = orc.decode([s.seq_id for s in seqs], last, pos)
            llm.step()
            if fused_head:
                assert [s.completion_token_ids[-1] for s in seqs] == list(o_tok), f"tokens at decode step {step}"
            else:
                _check_logits(runner.model.lm_head.last_logits, orc.last_logits, f"decode step {step}")
            # the compact state the manager keeps must follow the oracle's: layer 0
            # exactly; deeper layers' decisions see GEMM-order noise, and a
            # decision sitting on the threshold may flip
            mgr = runner.compact_kv_manager
            if lookahead:  # the state runs a step ahead of the oracle's
                assert runner.lookahead_pending() == (step < gen - 2 and layout == "paged"), step
                continue
            for s in seqs:
                if s.seq_id not in mgr.seq_states:  # finished and freed on the last step
                    continue
                got = np.array(mgr.seq_states[s.seq_id].live_counts.tolist())
                want = np.array(orc.mgr.seq_states[s.seq_id].live_counts.tolist())
                assert (got[0] == want[0]).all(), f"layer-0 live counts at step {step}: {got[0]} vs {want[0]}"
                assert np.abs(got - want).max() <= 2, f"live counts at step {step}: {got} vs {want}"
            if layout == "paged":
                check_page_invariants(mgr)
        assert ("fdms_paged_expiry" if layout == "paged" else "fdms_dms_expiry") in emu.calls
        llm.exit()
        return list(emu.calls) + probe


@pytest.mark.parametrize("lens,gen", [([300], 14), ([300, 64, 517], 10)])
def test_greedy_fast_loop_matches_the_oracle_tokens(lens, gen):
    """The device-side greedy loop (model_runner.py:971-1053) takes the whole
    decode tail after prefill: its tokens are the oracle's greedy tokens, the
    sequences end FINISHED with consistent counters, and their compact state
    follows the oracle's."""
    from oracle.model import OracleModel, weights_from_model
    with cpu_engine():
        from fastdms_amd import LLM, SamplingParams
        from fastdms_amd.engine.sequence import SequenceStatus
        llm = LLM("tiny-llama", max_model_len=2048, max_num_seqs=8, max_num_batched_tokens=16384,
                  enforce_eager=True, fused_greedy_head=True, **DMS)
        runner = llm.model_runner
        orc = OracleModel(weights_from_model(runner.model), llm.config.hf_config, window_size=32, alpha_scale=10.0,
                          alpha_offset=5.0, capacity_tokens=runner.compact_kv_manager.capacity_tokens,
                          max_model_len=llm.config.max_model_len)
        rng = np.random.default_rng(5)
        sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
        seqs = [llm.add_request(rng.integers(0, 512, n).tolist(), sp) for n in lens]
        llm.step()
        ids = [s.seq_id for s in seqs]
        want = [[int(t)] for t in orc.prefill([(s.seq_id, s.prompt_token_ids, gen) for s in seqs])]
        assert [s.completion_token_ids for s in seqs] == want, "prefill tokens"
        got = runner.run_compact_greedy_decode_loop(seqs, gen - 1)
        if len(seqs) == 1:
            got = [got]
        for _ in range(gen - 1):
            toks = orc.decode(ids, [w[-1] for w in want], [len(s.prompt_token_ids) + len(w) - 1
                                                             for s, w in zip(seqs, want)])
            for w, t in zip(want, toks):
                w.append(int(t))
        assert [w[1:] for w in want] == got
        mgr = runner.compact_kv_manager
        for s, w in zip(seqs, want):
            assert s.completion_token_ids == w and s.last_token == w[-1]
            assert s.status == SequenceStatus.FINISHED and s.num_cached_tokens == s.num_tokens
            live = np.array(mgr.seq_states[s.seq_id].live_counts.tolist())
            o_live = np.array(orc.mgr.seq_states[s.seq_id].live_counts.tolist())
            assert (live[0] == o_live[0]).all() and np.abs(live - o_live).max() <= 2
        with pytest.raises(RuntimeError, match="max_tokens"):
            runner.run_compact_greedy_decode_loop(seqs, 1)
        llm.exit()


def test_engine_takes_the_greedy_fast_loop_only_for_a_lone_greedy_sequence(monkeypatch):
    """llm_engine.py:55-74: after a prefill, a lone greedy ignore_eos sequence
    (the only one running) hands its decode tail to the device-side loop, which
    finishes it and frees its compact state.  The loop itself is stubbed here
    (graph replay is GPU-only); its tokens are pinned by the test above."""
    with cpu_engine():
        from fastdms_amd import LLM, SamplingParams
        from fastdms_amd.engine.sequence import SequenceStatus
        llm = LLM("tiny-llama", max_model_len=1024, max_num_seqs=4, max_num_batched_tokens=4096,
                  enforce_eager=True, fused_greedy_head=True, **DMS)
        calls = []

        def loop(seqs, n):
            calls.append((list(seqs), n))
            for s in seqs:
                for _ in range(n):
                    s.append_token(7)
                    s.num_cached_tokens += 1
                s.status = SequenceStatus.FINISHED
            return [7] * n

        monkeypatch.setattr(llm.model_runner, "run_compact_greedy_decode_loop", loop)
        llm.config.enforce_eager = False  # the reference takes the loop only with decode graphs
        greedy = SamplingParams(temperature=0.0, max_tokens=9, ignore_eos=True)
        a = llm.add_request(list(range(40)), greedy)
        outputs, _ = llm.step()
        assert calls == [([a], 8)] and a.is_finished and outputs == [(a.seq_id, a.completion_token_ids)]
        assert a.seq_id not in llm.model_runner.compact_kv_manager.seq_states and llm.is_finished()
        assert llm.last_step_stats["fast_loop"]["tokens"] == 8
        # not taken: two sequences prefilled together, a sampled sequence, or the switch off
        short = SamplingParams(temperature=0.0, max_tokens=3, ignore_eos=True)
        for prompts, sp, env in (([list(range(30)), list(range(50))], short, "1"),
                                 ([list(range(30))], SamplingParams(temperature=0.7, max_tokens=3, ignore_eos=True),
                                  "1"),
                                 ([list(range(30))], short, "0")):
            monkeypatch.setenv("FASTDMS_COMPACT_GREEDY_FAST_LOOP", env)
            calls.clear()
            for p in prompts:
                llm.add_request(p, sp)
            llm.step()  # the prefill, with the gate evaluated under decode graphs
            assert calls == [] and llm.last_step_stats["fast_loop"] is None
            llm.config.enforce_eager = True  # decode steps run eagerly on the CPU
            while not llm.is_finished():
                llm.step()
            llm.config.enforce_eager = False
        llm.exit()


def _generate(lens, gen, budget, seed=9, max_model_len=2048):
    """Greedy generation of random prompts with a per-step token budget."""
    from fastdms_amd import LLM, SamplingParams
    llm = LLM("tiny-llama", max_model_len=max_model_len, max_num_seqs=4, max_num_batched_tokens=budget,
              enforce_eager=True, fused_greedy_head=True, **DMS)
    rng = np.random.default_rng(seed)
    sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
    seqs = [llm.add_request(rng.integers(0, 512, n).tolist(), sp) for n in lens]
    prefill_counts = []
    while not llm.is_finished():
        _, num = llm.step()
        if num > 0:
            prefill_counts.append(num)
    # llm_engine.py:51-52: a prefill step reports the tokens it computed, so
    # the chunks of the prompts add up to their lengths, each within the budget
    assert sum(prefill_counts) == sum(lens) and max(prefill_counts) <= budget
    return llm, [list(s.completion_token_ids) for s in seqs]


@pytest.mark.parametrize("budget", [128, 200])
def test_chunked_prefill_equals_the_unchunked_prefill(budget):
    """Prompts longer than the step's token budget are prefilled in chunks
    over a dense-retained prefix (each chunk attends to the staged earlier
    chunks plus itself; the completing chunk packs the whole prompt).  The
    reference's semantics are dense causal attention over the whole prompt
    with evictions at pack time (attention.py:85-92), so the generation must
    equal the unchunked one token for token, and the first tokens the CPU
    model oracle's."""
    from oracle.model import OracleModel, weights_from_model
    lens, gen = [300, 517, 64], 6
    with cpu_engine() as emu:
        llm_c, chunked = _generate(lens, gen, budget)
        assert emu.calls.count("fdms_prefill_attention_varlen") > 0
        assert not llm_c.model_runner.prompt_stages, "stages of completed prompts are dropped"
        runner = llm_c.model_runner
        orc = OracleModel(weights_from_model(runner.model), llm_c.config.hf_config, window_size=32,
                          alpha_scale=10.0, alpha_offset=5.0, capacity_tokens=1 << 16,
                          max_model_len=llm_c.config.max_model_len)
        rng = np.random.default_rng(9)
        prompts = [rng.integers(0, 512, n).tolist() for n in lens]
        first = orc.prefill([(i, p, gen) for i, p in enumerate(prompts)])
        assert [t[0] for t in chunked] == [int(x) for x in first]
        llm_c.exit()
        llm_u, whole = _generate(lens, gen, 4096)
        llm_u.exit()
    assert chunked == whole


def test_chunked_prefill_state_equals_the_unchunked_state():
    """After a chunked prefill the compact state (live counts, token
    positions, FP8 rows of every span) is the unchunked prefill's, byte for
    byte."""
    from fastdms_amd import LLM, SamplingParams
    states = []
    with cpu_engine():
        for budget in (96, 4096):
            llm = LLM("tiny-llama", max_model_len=1024, max_num_seqs=2, max_num_batched_tokens=budget,
                      enforce_eager=True, fused_greedy_head=True, **DMS)
            sp = SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True)
            seq = llm.add_request(np.random.default_rng(2).integers(0, 512, 333).tolist(), sp)
            while seq.num_completion_tokens == 0:
                llm.step()
            mgr = llm.model_runner.compact_kv_manager
            st = mgr.seq_states[seq.seq_id]
            live = st.live_counts.clone()
            rows = []
            for layer in range(mgr.num_layers):
                for h in range(mgr.num_kv_heads):
                    b, n = int(st.base_offsets[layer, h]), int(live[layer, h])
                    rows.append((mgr.compact_k_per_layer[layer][b:b + n].view(torch.uint8).clone(),
                                 mgr.compact_v_per_layer[layer][b:b + n].view(torch.uint8).clone(),
                                 st.token_positions[layer, h, :n].clone()))
            states.append((live, rows, seq.completion_token_ids[0]))
            llm.exit()
    (lc, rc, tc), (lu, ru, tu) = states
    assert torch.equal(lc, lu) and tc == tu
    for (kc, vc, pc), (ku, vu, pu) in zip(rc, ru):
        assert torch.equal(kc, ku) and torch.equal(vc, vu) and torch.equal(pc, pu)


@pytest.mark.parametrize("lookahead", [False, True])
def test_decode_step_reports_a_page_pool_overflow(monkeypatch, lookahead):
    """The page pool's overflow flag reaches the host with the step's token ids
    (one read-back): a flag the device set (here by hand, as a failed page pop
    would) makes the decode step raise, with and without the lookahead.  Set
    between steps, the flag travels with the next step launched; with the
    lookahead that step is already in flight with its read-back queued, so
    the raise comes one step later."""
    if not lookahead:
        monkeypatch.setenv("FASTDMS_AMD_DECODE_LOOKAHEAD", "0")
    with cpu_engine():
        from fastdms_amd import LLM, SamplingParams
        llm = LLM("tiny-llama", max_model_len=2048, max_num_seqs=8, max_num_batched_tokens=16384,
                  enforce_eager=True, fused_greedy_head=True, compact_kv_layout="paged", **DMS)
        mgr = llm.model_runner.compact_kv_manager
        rng = np.random.default_rng(5)
        sp = SamplingParams(temperature=0.0, max_tokens=6, ignore_eos=True)
        for n in (80, 120):
            llm.add_request(rng.integers(0, 512, n).tolist(), sp)
        llm.step()  # prefill
        llm.step()  # a clean decode step
        mgr.overflow.fill_(1)
        if lookahead:
            llm.step()  # the step in flight: its read-back was queued before the flag was set
        with pytest.raises(RuntimeError, match="pool empty"):
            llm.step()
