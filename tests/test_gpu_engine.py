"""End-to-end compact-DMS generation on the GPU: graph-replayed decode equals
eager decode token for token, and the engine follows the CPU model oracle
(teacher-forced: a step may pick a different token only where the oracle's
own top-2 logits are within bf16 noise, since GEMM accumulation order
differs between the GPU library and the CPU)."""
import numpy as np
import pytest
import torch

from helpers import require_gpu

pytestmark = pytest.mark.gpu

DMS = dict(dms_window_size=32, dms_alpha_scale=10.0, dms_alpha_offset=5.0)


def _prompts(rng, lens, vocab):
    return [rng.integers(0, vocab, n).tolist() for n in lens]


def _llm(model, max_num_seqs=8, eager=False, seed=0):
    from fastdms_amd import LLM
    return LLM(model, max_model_len=2048, max_num_seqs=max_num_seqs, max_num_batched_tokens=16384,
               enforce_eager=eager, seed=seed, **DMS)


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


@pytest.mark.parametrize("model,lens", [("tiny-llama", [300, 517, 800, 64]), ("tiny-llama", [1000]),
                                        ("tiny-llama", [200, 400]), ("tiny-qwen3", [129, 700])])
def test_engine_follows_cpu_oracle(model, lens):
    require_gpu()
    from oracle.model import OracleModel, weights_from_model
    from fastdms_amd import SamplingParams
    rng = np.random.default_rng(1)
    prompts = _prompts(rng, lens, 512)
    gen = 40
    llm = _llm(model)
    runner = llm.model_runner
    orc = OracleModel(weights_from_model(runner.model), llm.config.hf_config, window_size=32, alpha_scale=10.0,
                      alpha_offset=5.0, capacity_tokens=runner.compact_kv_manager.capacity_tokens,
                      max_model_len=llm.config.max_model_len)
    sp = SamplingParams(temperature=0.0, max_tokens=gen, ignore_eos=True)
    seqs = [llm.add_request(p, sp) for p in prompts]
    llm.step()  # prefill
    gpu_first = [s.completion_token_ids[0] for s in seqs]
    orc_first = orc.prefill([(s.seq_id, s.prompt_token_ids, gen) for s in seqs])
    exact = mismatch = 0

    def check(g, o, row):
        nonlocal exact, mismatch
        if g == o:
            exact += 1
            return
        lg = orc.last_logits[row]
        gap = float(abs(lg[o] - lg[g]))
        assert gap <= 2e-2 * max(1.0, float(lg.abs().max())), (g, o, gap)
        mismatch += 1

    for i, (g, o) in enumerate(zip(gpu_first, orc_first)):
        check(g, o, i)
    for _ in range(gen - 1):
        pos = [len(s) - 1 for s in seqs]
        last = [s.last_token for s in seqs]
        o_tok = orc.decode([s.seq_id for s in seqs], last, pos)
        llm.step()
        g_tok = [s.completion_token_ids[-1] for s in seqs]
        for i, (g, o) in enumerate(zip(g_tok, o_tok)):
            check(g, o, i)
    assert exact >= 0.9 * (exact + mismatch), (exact, mismatch)
    llm.exit()
