"""FCFS scheduler (mirror of fastdms/engine/scheduler.py:8-133, compact-DMS mode).

Prefill admission is token-budget first, as in the reference's streaming-pack
mode (scheduler.py:40-54).  Compact capacity is checked by attempt: when a
prefill's spans do not fit, the engine either defers it (``defer_prefill``:
back to the queue head, admission paused until a running sequence finishes)
or preempts running sequences (``preempt``, scheduler.py:95-99: freed, and
re-admitted later by re-prefilling their tokens).
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
        self.admission_blocked = False
        self.num_preemptions = 0
        self.num_deferrals = 0
        self.preemption_log: list[tuple[int, int]] = []  # (seq_id, completion tokens at preemption)

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        scheduled: list[Sequence] = []
        batched = 0
        if self.admission_blocked and not self.running:
            self.admission_blocked = False
        while self.waiting and len(scheduled) < self.max_num_seqs and not self.admission_blocked:
            seq = self.waiting[0]
            # a re-prefill leaves the last token to the next decode step
            target = seq.num_tokens - 1 if seq.reprefill else seq.num_tokens
            num_tokens = max(target - seq.num_cached_tokens, 1)
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
        return self.schedule_running(), False

    def schedule_running(self) -> list[Sequence]:
        """The decode batch: the first max_num_seqs running sequences."""
        scheduled: list[Sequence] = []
        while self.running and len(scheduled) < self.max_num_seqs:
            seq = self.running.popleft()
            seq.num_scheduled_tokens = 1
            scheduled.append(seq)
        assert scheduled
        self.running.extendleft(reversed(scheduled))
        return scheduled

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        for seq, token_id in zip(seqs, token_ids):
            if is_prefill:
                seq.num_cached_tokens = min(seq.num_cached_tokens + seq.num_scheduled_tokens, seq.num_tokens)
                if seq.num_cached_tokens < seq.num_tokens or seq.num_completion_tokens > 0:
                    # chunked prefill, or re-prefill after preemption (its sampled
                    # token is dropped: the next decode step recomputes it); a
                    # re-prefill stays one until its last chunk
                    seq.num_scheduled_tokens = 0
                    if seq.num_cached_tokens >= seq.num_tokens - 1:
                        seq.reprefill = False
                    continue
            seq.append_token(token_id)
            seq.num_cached_tokens += 1
            seq.num_scheduled_tokens = 0
            if (not seq.ignore_eos and token_id == self.eos) or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                self.freed_seq_ids.append(seq.seq_id)
                self.running.remove(seq)
                self.admission_blocked = False

    def preempt(self, seq: Sequence) -> None:
        """scheduler.py:95-99: back to the head of the queue with its compact
        state freed (the engine frees the ids in freed_seq_ids); its tokens so
        far are prefilled again on re-admission."""
        if seq in self.running:
            self.running.remove(seq)
        seq.status = SequenceStatus.WAITING
        seq.num_cached_tokens = 0
        seq.num_scheduled_tokens = 0
        seq.reprefill = seq.num_completion_tokens > 0
        self.freed_seq_ids.append(seq.seq_id)
        self.waiting.appendleft(seq)
        self.num_preemptions += 1
        self.preemption_log.append((seq.seq_id, seq.num_completion_tokens))

    def preemption_victim(self, requester: list[Sequence], *, include_self: bool = False) -> Sequence | None:
        """The youngest running sequence (largest seq_id: arrival order) that
        is younger than every sequence of ``requester``; with include_self, a
        requester itself when nothing younger runs.  Age priority keeps the
        oldest running sequence always making progress (no preemption cycles)."""
        oldest = min(s.seq_id for s in requester)
        skip = {s.seq_id for s in requester}
        cands = [s for s in self.running if s.seq_id not in skip and s.seq_id > oldest]
        if cands:
            return max(cands, key=lambda s: s.seq_id)
        if include_self:
            mine = [s for s in self.running if s.seq_id in skip]
            return max(mine, key=lambda s: s.seq_id) if mine else None
        return None

    def defer_prefill(self, seqs: list[Sequence]) -> None:
        """Undo the admission of a prefill batch whose spans did not fit: the
        sequences return to the head of the queue in order, and admission waits
        until a running sequence finishes."""
        for seq in reversed(seqs):
            if seq in self.running:
                self.running.remove(seq)
            seq.status = SequenceStatus.WAITING
            seq.num_scheduled_tokens = 0
            self.waiting.appendleft(seq)
        self.admission_blocked = True
        self.num_deferrals += 1

    def consume_freed_seq_ids(self) -> list[int]:
        ids, self.freed_seq_ids = self.freed_seq_ids, []
        return ids
