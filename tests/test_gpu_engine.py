"""End-to-end compact-DMS generation on the GPU: graph-replayed decode equals
eager decode token for token, and the engine follows the CPU model oracle
(teacher-forced: a step may pick a different token only where the oracle's
own top-2 logits are within bf16 noise, since GEMM accumulation order
differs between the GPU library and the CPU)."""
import numpy as np
import pytest
import torch

from oracle_sync import sync_oracle_state
from paged_invariants import check_page_invariants

from helpers import require_gpu

pytestmark = pytest.mark.gpu

DMS = dict(dms_window_size=32, dms_alpha_scale=10.0, dms_alpha_offset=5.0)


def _prompts(rng, lens, vocab):
    return [rng.integers(0, vocab, n).tolist() for n in lens]


def _llm(model, max_num_seqs=8, eager=False, seed=0, fused_head=True):
    from fastdms_amd import LLM
    return LLM(model, max_model_len=2048, max_num_seqs=max_num_seqs, max_num_batched_tokens=16384,
               enforce_eager=eager, seed=seed, fused_greedy_head=fused_head, **DMS)


@pytest.mark.parametrize("model,lens", [("tiny-llama", [300, 517, 800, 64]), ("tiny-qwen3", [129, 700])])
def test_graph_decode_equals_eager(model, lens):
    require_gpu()
    from fastdms_amd import SamplingParams
    rng = np.random.default_rng(0)
    prompts = _prompts(rng, lens, 512)
    sp = SamplingParams(temperature=0.0, max_tokens=80, ignore_eos=True)
    outs = []
    for eager in (True, False):
        llm = _llm(model, eager=eager)
        outs.append([o["token_ids"] for o in llm.generate(prompts, sp)])
        llm.exit()
        del llm
        torch.cuda.synchronize()
    assert outs[0] == outs[1]
    assert all(len(t) == 80 for t in outs[0])


def _fp32_linear(x, w, b=None):
    """The oracle's linear: fp32 accumulation, one bf16 rounding (test-only patch)."""
    y = x.float() @ w.float().t()
    if b is not None:
        y = y + b.float()
    return y.to(x.dtype)


def _sync_oracle_state(orc, mgr, seqs):
    """Give the oracle the GPU's compact state (arenas, spans, live counts,
    positions, decisions), so its next decode step starts from the same KV."""
    sync_oracle_state(orc, mgr, [s.seq_id for s in seqs])


def _follow_oracle(model, lens, *, oracle_gemm: bool, gen: int = 40, sync_state: bool = False):
    """Teacher-forced comparison; returns per-step (relative RMS, max-abs-rel)
    logit errors and the (exact, near-tie) token counts.  With sync_state the
    oracle decodes every step from the GPU's compact state, which removes the
    effect of DMS decisions that flip on threshold ties."""
    from oracle.model import OracleModel, weights_from_model
    from fastdms_amd import SamplingParams
    saved = torch.nn.functional.linear
    if oracle_gemm:
        torch.nn.functional.linear = _fp32_linear
    try:
        rng = np.random.default_rng(1)
        prompts = _prompts(rng, lens, 512)
        llm = _llm(model, fused_head=False)  # logits are compared, so materialise them
        runner = llm.model_runner
        orc = OracleModel(weights_from_model(runner.model), llm.config.hf_config, window_size=32, alpha_scale=10.0,
                          alpha_offset=5.0, capacity_tokens=runner.compact_kv_manager.capacity_tokens,
                          max_model_len=llm.config.max_model_len)
        sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
        seqs = [llm.add_request(p, sp) for p in prompts]
        llm.step()  # prefill
        gpu_first = [s.completion_token_ids[0] for s in seqs]
        orc_first = orc.prefill([(s.seq_id, s.prompt_token_ids, gen) for s in seqs])
        counts = [0, 0]
        errors = []

        def check(g, o, row):
            if g == o:
                counts[0] += 1
                return
            lg = orc.last_logits[row]
            gap = float(abs(lg[o] - lg[g]))
            assert gap <= 2e-2 * max(1.0, float(lg.abs().max())), (g, o, gap)
            counts[1] += 1

        def logit_error():
            got = runner.model.lm_head.last_logits.float().cpu()
            want = orc.last_logits
            assert torch.isfinite(got).all(), "non-finite logits"
            rms = float((got - want).pow(2).mean().sqrt()) / max(1e-6, float(want.pow(2).mean().sqrt()))
            mx = float((got - want).abs().max()) / max(1e-6, float(want.abs().max()))
            errors.append((rms, mx))

        for i, (g, o) in enumerate(zip(gpu_first, orc_first)):
            check(g, o, i)
        logit_error()
        for _ in range(gen - 1):
            pos = [len(s) - 1 for s in seqs]
            last = [s.last_token for s in seqs]
            if sync_state:
                torch.cuda.synchronize()
                _sync_oracle_state(orc, runner.compact_kv_manager, seqs)
            o_tok = orc.decode([s.seq_id for s in seqs], last, pos)
            llm.step()
            for i, (g, o) in enumerate(zip([s.completion_token_ids[-1] for s in seqs], o_tok)):
                check(g, o, i)
            logit_error()
        llm.exit()
    finally:
        torch.nn.functional.linear = saved
    print(f"{model} {lens} oracle_gemm={oracle_gemm} sync_state={sync_state}: tokens exact/near-tie {counts}; logit rel-RMS per step "
          f"{[round(e[0], 4) for e in errors]}; max-abs-rel {max(e[1] for e in errors):.4f}", flush=True)
    return errors, counts


CASES = [("tiny-llama", [300, 517, 800, 64]), ("tiny-llama", [1000]), ("tiny-llama", [200, 400]),
         ("tiny-qwen3", [129, 700])]


@pytest.mark.parametrize("model,lens", CASES)
def test_engine_step_matches_cpu_oracle(model, lens):
    """Each decode step from the same compact state, with the oracle's GEMM
    numerics: what is left is the kernels' own rounding (fp32 reduction order,
    bf16 P in the prefill MFMA, one bf16 rounding of each output)."""
    require_gpu()
    errors, (exact, near) = _follow_oracle(model, lens, oracle_gemm=True, sync_state=True)
    assert max(e[0] for e in errors) <= 1e-2
    assert max(e[1] for e in errors) <= 2e-2
    assert exact >= 0.95 * (exact + near)


@pytest.mark.parametrize("model,lens", CASES)
def test_engine_follows_cpu_oracle_native_gemm(model, lens):
    """Free-running with production bf16 GEMMs (hipBLASLt): reduction order
    differs from the CPU, which can flip a DMS decision sitting on the
    threshold and so which tokens a head keeps; logits stay within a few
    percent and greedy tokens agree except on near-ties."""
    require_gpu()
    errors, (exact, near) = _follow_oracle(model, lens, oracle_gemm=False)
    assert max(e[0] for e in errors) <= 5e-2
    assert exact >= 0.9 * (exact + near)


@pytest.mark.parametrize("model,lens", [("tiny-llama", [300, 517, 800, 64]), ("tiny-qwen3", [129, 700])])
def test_fused_greedy_head_equals_logits_argmax(model, lens):
    """The LM-head GEMV fused with the argmax picks the same tokens as logits +
    argmax, in graph-replayed decode."""
    require_gpu()
    from fastdms_amd import SamplingParams
    rng = np.random.default_rng(4)
    prompts = _prompts(rng, lens, 512)
    sp = SamplingParams(temperature=0.0, max_tokens=40, ignore_eos=True)
    outs = []
    for fused in (False, True):
        llm = _llm(model, fused_head=fused)
        outs.append([o["token_ids"] for o in llm.generate(prompts, sp)])
        llm.exit()
        del llm
        torch.cuda.synchronize()
    assert outs[0] == outs[1]


@pytest.mark.parametrize("lens", [[1500], [300, 517, 800, 64]])
def test_greedy_fast_loop_equals_per_step_decode(monkeypatch, lens):
    """The device-side greedy loop (model_runner.py:971-1053) gives the tokens
    of per-step graph decode.  A lone sequence takes it from the engine step
    after its prefill (llm_engine.py:55-74); a batch calls it on the runner."""
    require_gpu()
    from fastdms_amd import SamplingParams
    rng = np.random.default_rng(8)
    prompts = _prompts(rng, lens, 512)
    gen = 48
    sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
    monkeypatch.setenv("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "0")
    llm = _llm("tiny-llama")
    want = [o["token_ids"] for o in llm.generate(prompts, sp)]
    llm.exit()
    del llm
    torch.cuda.synchronize()
    monkeypatch.setenv("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "1")
    llm = _llm("tiny-llama")
    if len(lens) == 1:
        got = [o["token_ids"] for o in llm.generate(prompts, sp)]
        assert llm.last_step_stats["fast_loop"] == {"tokens": gen - 1,
                                                    "seconds": llm.last_step_stats["fast_loop"]["seconds"]}
    else:
        seqs = [llm.add_request(p, sp) for p in prompts]
        llm.step()
        assert llm.last_step_stats["fast_loop"] is None
        first = [s.completion_token_ids[0] for s in seqs]
        tail = llm.model_runner.run_compact_greedy_decode_loop(seqs, gen - 1)
        got = [[f] + t for f, t in zip(first, tail)]
        assert all(s.is_finished for s in seqs)
    assert got == want
    llm.exit()
    del llm
    torch.cuda.synchronize()


def test_chunked_prefill_matches_the_unchunked_prefill():
    """A prompt longer than the step's token budget, prefilled in chunks over
    its dense-retained prefix: the prefill logits equal the unchunked
    prefill's to bf16 noise, layer 0's compact live counts match exactly (its
    decisions see only the embedding) and deeper layers within a decision or
    two; generation then runs to completion from the chunked state."""
    require_gpu()
    from fastdms_amd import LLM, SamplingParams
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, 512, 1500).tolist()
    sp = SamplingParams(temperature=0.0, max_tokens=24, ignore_eos=True)
    res = []
    for budget in (256, 4096):
        llm = LLM("tiny-llama", max_model_len=2048, max_num_seqs=2, max_num_batched_tokens=budget,
                  fused_greedy_head=False, **DMS)
        seq = llm.add_request(prompt, sp)
        steps = 0
        while seq.num_completion_tokens == 0:
            llm.step()
            steps += 1
        logits = llm.model_runner.model.lm_head.last_logits.float().cpu()
        live = llm.model_runner.compact_kv_manager.seq_states[seq.seq_id].live_counts.cpu().clone()
        while not llm.is_finished():
            llm.step()
        res.append((steps, logits, live, len(seq.completion_token_ids)))
        assert not llm.model_runner.prompt_stages
        llm.exit()
        del llm
        torch.cuda.synchronize()
    (sc, lc, vc, nc), (su, lu, vu, nu) = res
    assert sc == 6 and su == 1, "1500 tokens in 256-token chunks"
    scale = max(1.0, float(lu.abs().max()))
    assert float((lc - lu).abs().max()) <= 2e-2 * scale
    assert torch.equal(vc[0], vu[0]) and int((vc - vu).abs().max()) <= 2
    assert nc == nu == 24


_QUANT_ENVS = {
    "fp8_all": {"FASTDMS_FP8_WEIGHTS": "1", "FASTDMS_FP8_WEIGHT_SCOPE": "all", "FASTDMS_FP8_LM_HEAD": "1"},
    "fp8_mlp_int4": {"FASTDMS_FP8_WEIGHTS": "1", "FASTDMS_FP8_WEIGHT_SCOPE": "mlp_lm_head",
                     "FASTDMS_INT4_ROW1_WEIGHTS": "1", "FASTDMS_INT4_ROW1_SCOPE": "mlp+lm_head",
                     "FASTDMS_INT4_ROW1_MAX_ROWS": "8",
                     "FASTDMS_INT4_ROW1_GROUP_SIZE": "128", "FASTDMS_INT4_ROW1_QUANT_MODE": "asymmetric"},
}


@pytest.mark.parametrize("env", sorted(_QUANT_ENVS))
def test_quantized_weights_graph_equals_eager(monkeypatch, env):
    """FP8 / INT4 weights selected by the reference's environment switches
    (model_runner.py:72-113): graph-replayed decode equals eager decode, and
    the fused greedy head equals logits + argmax (at more than one row both
    score the bf16 logits)."""
    require_gpu()
    from fastdms_amd import SamplingParams
    for k, v in _QUANT_ENVS[env].items():
        monkeypatch.setenv(k, v)
    rng = np.random.default_rng(6)
    prompts = _prompts(rng, [300, 517, 64], 512)
    sp = SamplingParams(temperature=0.0, max_tokens=40, ignore_eos=True)
    outs = []
    for eager, fused in ((True, True), (False, True), (False, False)):
        llm = _llm("tiny-llama", eager=eager, fused_head=fused)
        runner = llm.model_runner
        assert runner.fp8_weight_modules > 0 and runner.fp8_lm_head
        layer = runner.model.model.layers[0]
        if env == "fp8_mlp_int4":
            assert layer.mlp.down_proj._int4_enabled and not layer.self_attn.o_proj._int4_enabled
            assert layer.mlp.down_proj.route(3)[0] == "int4"
        else:
            assert layer.self_attn.qkv_proj._fp8_weight_enabled and not layer.mlp.down_proj._int4_enabled
        outs.append([o["token_ids"] for o in llm.generate(prompts, sp)])
        llm.exit()
        del llm
        torch.cuda.synchronize()
    assert outs[0] == outs[1] == outs[2]


@pytest.mark.parametrize("cap", [260, 300])
def test_preempted_sequences_follow_the_oracle_on_the_gpu(monkeypatch, cap):
    """(f)1 on the GPU: capped span KV with preemption (graphs on), on the
    tiny-llama shape with a planted successor margin (greedy decisions a few
    logits apart, so GPU and CPU rounding cannot flip them).  Every sequence's
    tokens -- those after a re-admission included -- equal the CPU model
    oracle replaying that sequence alone through the same history: prefill,
    decode, free at each preemption, re-prefill of its tokens but the last,
    decode (tests/test_engine_preemption.py's replay)."""
    require_gpu()
    from dataclasses import replace
    from fastdms_amd import LLM, SamplingParams
    from fastdms_amd.models.synthetic import PRESETS
    from test_engine_preemption import GEN, _replay_alone
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "1")
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_INTERVAL", "1")
    monkeypatch.setenv("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "0")
    cfg = replace(PRESETS["tiny-llama"], successor_margin=1.0)
    llm = LLM(cfg, max_model_len=1024, max_num_seqs=4, max_num_batched_tokens=4096, fused_greedy_head=True,
              compact_kv_capacity_tokens=cap, compact_admission="preempt", compact_decode_reserve_tokens=4,
              compact_kv_layout="span", **DMS)
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
    assert sched.num_preemptions >= 1, "no preemption: the test did not exercise re-admission"
    torch.cuda.synchronize()
    for s in seqs:
        at = [g for sid, g in sched.preemption_log if sid == s.seq_id]
        got, want = _replay_alone(llm.model_runner, llm, s, at)
        assert got == want, f"seq {s.seq_id} (preempted at {at}): oracle {got} vs engine {want}"
    print(f"cap {cap}: {sched.num_preemptions} preemptions {sched.preemption_log}", flush=True)
    llm.exit()
    del llm
    torch.cuda.synchronize()


@pytest.mark.parametrize("admission,reserve,cap,layout", [
    ("defer", None, 260, "span"), ("preempt", 4, 300, "span"),
    # 18 pages of 16 rows: the second prompt waits for the first.  (Preemption
    # on the paged layout needs a pool sized to these prompts' DMS decisions;
    # the CPU engine test pins it with the emulator's exact numerics.)
    ("defer", None, 288, "paged")])
def test_admission_and_preemption_on_the_gpu(monkeypatch, admission, reserve, cap, layout):
    """Capped compact KV on the GPU (graphs on): deferred prefills, spans that
    grow during decode and preempted sequences re-admitted by re-prefill.  Every
    request completes, every span returns to the allocator, a rerun is token-
    for-token identical (deterministic across preemptions), and the tokens each
    sequence produced before its first preemption equal an uncapped run's."""
    require_gpu()
    from fastdms_amd import LLM, SamplingParams
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "1")
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_INTERVAL", "1")
    # a sequence admitted alone would otherwise finish inside its prefill step
    # (the greedy fast loop), and no decode would meet a deferred admission
    monkeypatch.setenv("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "0")
    gen = 30

    def run(capped):
        llm = LLM("tiny-llama", max_model_len=1024, max_num_seqs=4, max_num_batched_tokens=4096,
                  fused_greedy_head=True, compact_kv_capacity_tokens=cap if capped else 0,
                  compact_admission=admission, compact_decode_reserve_tokens=reserve if capped else None,
                  compact_kv_layout=layout, **DMS)
        rng = np.random.default_rng(11)
        sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
        seqs = [llm.add_request(rng.integers(0, 512, n).tolist(), sp) for n in (300, 200)]
        for _ in range(5):
            llm.step()
        seqs.append(llm.add_request(rng.integers(0, 512, 160).tolist(), sp))
        steps = 0
        while not llm.is_finished():
            llm.step()
            steps += 1
            assert steps < 400, "the engine stopped making progress"
        mgr = llm.model_runner.compact_kv_manager
        assert not mgr.seq_states and mgr.free_tokens == mgr.capacity_tokens * mgr.num_layers
        if layout == "paged":
            check_page_invariants(mgr)
            assert mgr.page_top.tolist() == [mgr.num_pages] * mgr.num_layers
        first = {}
        for sid, g in llm.scheduler.preemption_log:
            first.setdefault(sid, g)
        out = ([list(s.completion_token_ids) for s in seqs], [first.get(s.seq_id, gen) for s in seqs],
               llm.scheduler.num_deferrals, mgr.num_span_moves)
        llm.exit()
        torch.cuda.synchronize()
        return out

    toks, first, deferrals, moves = run(True)
    assert all(len(t) == gen for t in toks)
    if admission == "defer":
        assert deferrals >= 1 and all(g == gen for g in first)
    else:
        assert any(g < gen for g in first) and (layout == "paged" or moves >= 1)
    assert run(True)[0] == toks
    free_toks = run(False)[0]
    for t, f, g in zip(toks, free_toks, first):
        assert t[:g] == f[:g]
