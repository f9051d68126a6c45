"""Engine loop (mirror of fastdms/engine/llm_engine.py:16-116, single GPU)."""
from __future__ import annotations

import time
from dataclasses import fields

from ..config import Config
from ..sampling_params import SamplingParams
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import Sequence


class LLMEngine:

    def __init__(self, model, **kwargs):
        names = {f.name for f in fields(Config)}
        config = Config(model, **{k: v for k, v in kwargs.items() if k in names})
        self.config = config
        self.model_runner = ModelRunner(config)
        self.scheduler = Scheduler(config)
        self.last_step_stats: dict = {}

    def add_request(self, prompt: list[int], sampling_params: SamplingParams) -> Sequence:
        if isinstance(prompt, str):
            raise ValueError("this build takes token ids (there is no tokenizer for synthetic models)")
        seq = Sequence(prompt, sampling_params)
        self.scheduler.add(seq)
        return seq

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        t0 = time.perf_counter()
        token_ids = self.model_runner.run(seqs, is_prefill)
        dt = time.perf_counter() - t0
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        freed = self.scheduler.consume_freed_seq_ids()
        if freed:
            self.model_runner.free_compact(freed)
        outputs = [(seq.seq_id, seq.completion_token_ids) for seq in seqs if seq.is_finished]
        num_tokens = sum(seq.num_scheduled_tokens or len(seq) for seq in seqs) if is_prefill else len(seqs)
        if is_prefill:
            num_tokens = sum(len(s.prompt_token_ids) for s in seqs)
        self.last_step_stats = {"is_prefill": is_prefill, "seconds": dt, "tokens": num_tokens}
        return outputs, (num_tokens if is_prefill else -len(seqs))

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def generate(self, prompts: list[list[int]], sampling_params, use_tqdm: bool = False) -> list[dict]:
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        for prompt, sp in zip(prompts, sampling_params):
            self.add_request(prompt, sp)
        outputs = {}
        while not self.is_finished():
            out, _ = self.step()
            for seq_id, token_ids in out:
                outputs[seq_id] = token_ids
        return [{"text": None, "token_ids": outputs[k]} for k in sorted(outputs)]

    def exit(self):
        self.model_runner.exit()
