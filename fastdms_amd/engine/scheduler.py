"""FCFS scheduler (mirror of fastdms/engine/scheduler.py:8-133, compact-DMS mode).

Prefill admission is token-budget only, as in the reference's streaming-pack
mode (scheduler.py:40-54); compact decode never preempts (74-81).
"""
from __future__ import annotations

from collections import deque

from ..config import Config
from .sequence import Sequence, SequenceStatus


class Scheduler:

    def __init__(self, config: Config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self.freed_seq_ids: list[int] = []

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        scheduled: list[Sequence] = []
        batched = 0
        while self.waiting and len(scheduled) < self.max_num_seqs:
            seq = self.waiting[0]
            num_tokens = max(seq.num_tokens - seq.num_cached_tokens, 1)
            remaining = self.max_num_batched_tokens - batched
            if remaining == 0 or (remaining < num_tokens and scheduled):
                break
            seq.num_scheduled_tokens = min(num_tokens, remaining)
            if seq.num_scheduled_tokens == num_tokens:
                seq.status = SequenceStatus.RUNNING
                self.waiting.popleft()
                self.running.append(seq)
            scheduled.append(seq)
            batched += seq.num_scheduled_tokens
        if scheduled:
            return scheduled, True
        while self.running and len(scheduled) < self.max_num_seqs:
            seq = self.running.popleft()
            seq.num_scheduled_tokens = 1
            scheduled.append(seq)
        assert scheduled
        self.running.extendleft(reversed(scheduled))
        return scheduled, False

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        for seq, token_id in zip(seqs, token_ids):
            if is_prefill:
                seq.num_cached_tokens = min(seq.num_cached_tokens + seq.num_scheduled_tokens, seq.num_tokens)
                if seq.num_cached_tokens < seq.num_tokens or seq.num_completion_tokens > 0:
                    seq.num_scheduled_tokens = 0
                    continue
            seq.append_token(token_id)
            seq.num_cached_tokens += 1
            seq.num_scheduled_tokens = 0
            if (not seq.ignore_eos and token_id == self.eos) or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                self.freed_seq_ids.append(seq.seq_id)
                self.running.remove(seq)

    def consume_freed_seq_ids(self) -> list[int]:
        ids, self.freed_seq_ids = self.freed_seq_ids, []
        return ids
