"""Engine loop (mirror of fastdms/engine/llm_engine.py:16-116, single GPU)."""
from __future__ import annotations

import time
from dataclasses import fields

from ..config import Config
from ..sampling_params import SamplingParams
from .compact_kv import CompactCapacityExhausted
from .model_runner import ModelRunner, compact_greedy_fast_loop_enabled
from .scheduler import Scheduler
from .sequence import Sequence, SequenceStatus


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

    def _free_preempted(self) -> None:
        freed = self.scheduler.consume_freed_seq_ids()
        if freed:
            self.model_runner.free_compact(freed)

    def _run_prefill_admitting(self, seqs):
        """Run a prefill batch; when its compact spans do not fit, preempt
        running sequences (compact_admission="preempt") or defer the batch.
        Returns (the sequences prefilled, their sampled tokens), or (None, None)
        when the batch was deferred."""
        while True:
            try:
                return seqs, self.model_runner.run(seqs, True)
            except CompactCapacityExhausted:
                self.model_runner.free_compact([s.seq_id for s in seqs])  # spans of the failed attempt
                victim = None
                if self.config.compact_admission == "preempt":
                    victim = self.scheduler.preemption_victim(seqs)
                if victim is not None:
                    self.scheduler.preempt(victim)
                    self._free_preempted()
                    continue
                if len(seqs) > 1:  # retry the head of the batch alone, the rest waits
                    self.scheduler.defer_prefill(seqs[1:])
                    self.scheduler.admission_blocked = False
                    seqs = seqs[:1]
                    continue
                if not any(s is not seqs[0] for s in self.scheduler.running):
                    # nothing runs that could free space: the request never fits
                    raise CompactCapacityExhausted(
                        f"request {seqs[0].seq_id} ({len(seqs[0])} tokens) does not fit the compact KV capacity "
                        f"({self.config.compact_kv_capacity_tokens} tokens per layer) on its own")
                self.scheduler.defer_prefill(seqs)
                return None, None

    def _make_decode_room(self, seqs):
        """Before a decode step: grow the full spans of overcommitted sequences
        (oldest first), preempting the youngest running sequence -- possibly
        the one that needs room -- when no range is free.  Returns the batch
        without the preempted sequences."""
        mgr = self.model_runner.compact_kv_manager
        for seq in sorted(seqs, key=lambda s: s.seq_id):
            while seq in self.scheduler.running and mgr.decode_room_needed(seq):
                try:
                    mgr.grow_for_decode(seq)
                except CompactCapacityExhausted:
                    victim = self.scheduler.preemption_victim([seq], include_self=True)
                    self.scheduler.preempt(victim)
                    self._free_preempted()
        return [s for s in seqs if s in self.scheduler.running]

    def _make_page_room(self, seqs):
        """Paged layout, before a decode step: while the next append of every
        running sequence may not fit the page pool (one sync of the page
        counts decides), preempt the youngest running sequence.  With the full
        decode reservation admission already guarantees the room.  Returns
        the batch without the preempted sequences."""
        mgr = self.model_runner.compact_kv_manager
        while seqs and not mgr.decode_pages_fit():
            victim = self.scheduler.preemption_victim([min(seqs, key=lambda s: s.seq_id)], include_self=True)
            if victim is None:
                raise CompactCapacityExhausted("paged compact KV: no page for the next decode step")
            self.scheduler.preempt(victim)
            self._free_preempted()
            seqs = [s for s in seqs if s in self.scheduler.running]
        return seqs

    def drain(self) -> None:
        """Finish the decode step launched ahead, if any (one more step of the
        running batch, launching nothing further), so that host and device
        state agree before the runner is driven directly."""
        if self.model_runner.lookahead_pending():
            self.step(lookahead=False)

    def step(self, lookahead: bool = True):
        runner = self.model_runner
        if runner.lookahead_pending():
            # the decode step launched ahead by the previous step is in flight:
            # this step is that decode (a new request's prefill comes next)
            seqs, is_prefill = self.scheduler.schedule_running(), False
        else:
            seqs, is_prefill = self.scheduler.schedule()
        t0 = time.perf_counter()
        if is_prefill:
            done, token_ids = self._run_prefill_admitting(seqs)
            if done is None:  # deferred: run a decode step of the running batch instead
                seqs, is_prefill = self.scheduler.schedule()
                if is_prefill:
                    raise RuntimeError("prefill admission is paused but the scheduler chose a prefill")
            else:
                seqs = done
        if not is_prefill:
            if runner.lookahead_pending():
                pass  # its room was checked when it was launched
            elif runner.compact_kv_manager.paged:
                seqs = self._make_page_room(seqs)
            elif self.config.compact_decode_reserve_tokens is not None:
                seqs = self._make_decode_room(seqs)
            # the next step decodes this same batch when nothing waits to be
            # admitted (and, checked by the runner, none of it finishes now)
            token_ids = runner.run(seqs, False, lookahead=lookahead and not self.scheduler.waiting) if seqs else []
        dt = time.perf_counter() - t0
        # llm_engine.py:51-52: a prefill step counts the tokens it computed (a
        # chunk of a long prompt, a re-prefill's tokens), read before
        # postprocess clears them; a decode step counts its sequences
        num_tokens = sum(s.num_scheduled_tokens for s in seqs) if is_prefill else len(seqs)
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        fast = self._greedy_fast_loop(seqs) if is_prefill else None
        freed = self.scheduler.consume_freed_seq_ids()
        if freed:
            self.model_runner.free_compact(freed)
        outputs = [(seq.seq_id, seq.completion_token_ids) for seq in seqs if seq.is_finished]
        self.last_step_stats = {"is_prefill": is_prefill, "seconds": dt, "tokens": num_tokens, "fast_loop": fast}
        return outputs, (num_tokens if is_prefill else -len(seqs))

    def _greedy_fast_loop(self, seqs):
        """llm_engine.py:55-74: a lone greedy ignore_eos sequence that has just
        been prefilled decodes its whole tail in one device-side loop.  Besides
        the reference's conditions it must be the only running sequence (the
        loop packs the active slots) and hold its full span reservation.
        Returns {"tokens", "seconds"} of the loop, or None when not taken."""
        cfg = self.config
        if not (compact_greedy_fast_loop_enabled() and len(seqs) == 1 and list(self.scheduler.running) == seqs
                and cfg.fused_greedy_head and cfg.compact_decode_cudagraph and not cfg.enforce_eager
                and cfg.compact_decode_reserve_tokens is None):
            return None
        seq = seqs[0]
        if not (seq.temperature <= 1e-10 and seq.ignore_eos and seq.status == SequenceStatus.RUNNING
                and seq.num_cached_tokens == seq.num_tokens):
            return None
        remaining = seq.max_tokens - seq.num_completion_tokens
        if remaining <= 0:
            return None
        t0 = time.perf_counter()
        self.model_runner.run_compact_greedy_decode_loop([seq], remaining)
        dt = time.perf_counter() - t0
        if seq.is_finished:
            self.scheduler.freed_seq_ids.append(seq.seq_id)
            self.scheduler.running.remove(seq)
            self.scheduler.admission_blocked = False
        return {"tokens": remaining, "seconds": dt}

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
