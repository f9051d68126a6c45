"""Compact-capacity admission, decode growth and preemption / re-admission.

A build extension: the reference sizes every span for all of max_tokens, admits
prefills by token budget only (scheduler.py:40-54), raises when the compact
allocator runs out (compact_kv.py:715-718) and never preempts compact
sequences (scheduler.py:74-81).  Here a prefill whose spans do not fit is
deferred (or preempts younger running sequences), spans may be overcommitted
(compact_decode_reserve_tokens) and grow during decode, and a sequence that
cannot grow is preempted: freed, then re-admitted by re-prefilling its tokens
but the last, which the next decode step appends.

Run on the CPU through tests/native_emulator.py with the fused greedy head.
Each sequence's tokens are checked against the CPU model oracle replaying that
sequence alone through the same history (prefill, decode steps, free at each
preemption, re-prefill of all tokens but the last, decode): the same tokens,
step for step.  The incremental expiry branch is forced (interval 1), so the
live sets do not depend on the batch size.
"""
import numpy as np
import pytest

from native_emulator import cpu_engine
from paged_invariants import check_page_invariants

DMS = dict(dms_window_size=32, dms_alpha_scale=10.0, dms_alpha_offset=5.0)
GEN = 30


def _replay_alone(runner, llm, seq, preempted_at):
    """Greedy tokens of the oracle for ``seq`` alone, following its history."""
    from oracle.model import OracleModel, weights_from_model
    orc = OracleModel(weights_from_model(runner.model), llm.config.hf_config, window_size=32, alpha_scale=10.0,
                      alpha_offset=5.0, capacity_tokens=1 << 16, max_model_len=llm.config.max_model_len)
    prompt = list(seq.prompt_token_ids)
    want = list(seq.completion_token_ids)
    sid = 0
    cur = prompt + [orc.prefill([(sid, prompt, GEN)])[0]]
    for g in list(preempted_at) + [GEN]:
        while len(cur) - len(prompt) < g:
            tok = orc.decode([sid], [cur[-1]], [len(cur) - 1], expiry_mode="1")[0]
            cur.append(tok)
        if g == GEN:
            break
        orc.mgr.free(sid)  # preempted: freed, then re-prefilled but for the last token
        sid += 1
        orc.prefill([(sid, cur[:-1], GEN)])
    got = cur[len(prompt):]
    return got, want


@pytest.mark.parametrize("admission,reserve,cap,layout", [
    ("defer", None, 260, "paged"), ("defer", None, 260, "span"),
    # the paged pool admits the second prompt only once both fit (23 pages of
    # 16 rows); their decode growth then forces a preemption
    ("preempt", 4, 368, "paged"), ("preempt", 4, 300, "span")])
def test_admission_and_preemption_follow_the_oracle(monkeypatch, admission, reserve, cap, layout):
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "1")
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_INTERVAL", "1")
    with cpu_engine():
        from fastdms_amd import LLM, SamplingParams
        llm = LLM("tiny-llama", max_model_len=1024, max_num_seqs=4, max_num_batched_tokens=4096,
                  enforce_eager=True, fused_greedy_head=True, compact_kv_capacity_tokens=cap,
                  compact_admission=admission, compact_decode_reserve_tokens=reserve, compact_kv_layout=layout,
                  **DMS)
        runner = llm.model_runner
        rng = np.random.default_rng(11)
        sp = SamplingParams(temperature=0.0, max_tokens=GEN, ignore_eos=True)
        seqs = [llm.add_request(rng.integers(0, 512, n).tolist(), sp) for n in (300, 200)]
        for _ in range(5):
            llm.step()
        seqs.append(llm.add_request(rng.integers(0, 512, 160).tolist(), sp))
        steps = 0
        while not llm.is_finished():
            llm.step()
            steps += 1
            assert steps < 400, "the engine stopped making progress"
        sched = llm.scheduler
        mgr = runner.compact_kv_manager
        assert all(len(s.completion_token_ids) == GEN for s in seqs)
        if admission == "defer":
            assert sched.num_deferrals >= 1 and sched.num_preemptions == 0
        else:  # spans grow by moving to a larger range; pages grow in place
            assert sched.num_preemptions >= 1 and (layout == "paged" or mgr.num_span_moves >= 1)
        assert not mgr.seq_states
        if layout == "span":
            assert mgr.free_tokens == cap * mgr.num_layers  # every span came back
        else:
            check_page_invariants(mgr)  # every page came back: the whole pool is on the free stacks
            assert mgr.page_top.tolist() == [mgr.num_pages] * mgr.num_layers
        for s in seqs:
            at = [g for sid, g in sched.preemption_log if sid == s.seq_id]
            got, want = _replay_alone(runner, llm, s, at)
            assert got == want, f"seq {s.seq_id} (preempted at {at}): oracle {got} vs engine {want}"


def test_a_request_that_can_never_fit_raises():
    with cpu_engine():
        from fastdms_amd import LLM, SamplingParams
        from fastdms_amd.engine.compact_kv import CompactCapacityExhausted
        llm = LLM("tiny-llama", max_model_len=1024, max_num_seqs=2, max_num_batched_tokens=4096,
                  enforce_eager=True, compact_kv_capacity_tokens=40, compact_admission="preempt", **DMS)
        llm.add_request(list(range(300)), SamplingParams(temperature=0.0, max_tokens=8, ignore_eos=True))
        with pytest.raises(CompactCapacityExhausted, match=r"\(300 tokens\) does not fit .*\(40 tokens per layer\)"):
            llm.step()


def test_streaming_pack_rejects_a_live_count_above_the_span_capacity():
    """compact_kv.py:1018-1023: with the per-sequence target capped below a
    prompt's live count, the pack raises before it allocates or scatters
    (a span of max_capacity_per_lh rows cannot hold the survivors)."""
    with cpu_engine():
        from fastdms_amd import LLM, SamplingParams
        llm = LLM("tiny-llama", max_model_len=1024, max_num_seqs=2, max_num_batched_tokens=4096,
                  enforce_eager=True, compact_kv_target_live_tokens_per_seq=64, compact_kv_layout="span", **DMS)
        rng = np.random.default_rng(5)
        sp = SamplingParams(temperature=0.0, max_tokens=8, ignore_eos=True)
        for n in (500, 400):
            llm.add_request(rng.integers(0, 512, n).tolist(), sp)
        mgr = llm.model_runner.compact_kv_manager
        free_before = [list(r) for r in mgr.free_ranges_per_layer]
        with pytest.raises(RuntimeError, match="exceeds metadata capacity"):
            llm.step()
        assert [list(r) for r in mgr.free_ranges_per_layer] == free_before
