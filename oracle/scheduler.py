"""Restatement of ContinuousBatchingScheduler (TEST INFRASTRUCTURE ONLY).

Follows Sources/PagedAttentionMetal/Scheduler.swift:42-177:
  addRequest            :59-70   (rejects with -1 once the table holds maxSequences;
                                  completed sequences are never removed)
  step                  :78-114  (waiting by arrival first, then running & !done, then paused)
  markPrefilled / markDecoded / preemptSequence / completeSequence
  handleMemoryPressure  :135-152 (pauses the newest running sequence while the
                                  available-blocks closure stays below the requirement)
"""
from __future__ import annotations

WAITING, RUNNING, PAUSED, COMPLETED = 0, 1, 2, 3


class RefSequence:
    def __init__(self, sid, prompt, max_new, arrival):
        self.id = sid
        self.prompt = prompt
        self.max_new = max_new
        self.arrival = arrival
        self.status = WAITING
        self.generated = 0

    @property
    def current_length(self):
        return self.prompt + self.generated

    @property
    def done(self):
        return self.generated >= self.max_new


class RefScheduler:
    def __init__(self, max_batch: int, max_sequences: int = 128):
        self.max_batch = max_batch
        self.max_sequences = max_sequences
        self.seqs: dict[int, RefSequence] = {}
        self.next_id = 0
        self.arrival = 0

    def add_request(self, prompt: int, max_new: int) -> int:
        if len(self.seqs) >= self.max_sequences:
            return -1
        sid = self.next_id
        self.next_id += 1
        self.seqs[sid] = RefSequence(sid, prompt, max_new, self.arrival)
        self.arrival += 1
        return sid

    def complete(self, sid):
        if sid in self.seqs:
            self.seqs[sid].status = COMPLETED

    def step(self):
        by_arr = lambda s: s.arrival
        waiting = sorted((s for s in self.seqs.values() if s.status == WAITING), key=by_arr)
        running = sorted((s for s in self.seqs.values() if s.status == RUNNING and not s.done), key=by_arr)
        paused = sorted((s for s in self.seqs.values() if s.status == PAUSED), key=by_arr)
        batch = []
        for s in waiting[: min(len(waiting), self.max_batch)]:
            s.status = RUNNING
            batch.append(s)
        rem = self.max_batch - len(batch)
        if rem > 0:
            batch.extend(running[:rem])
        rem = self.max_batch - len(batch)
        if rem > 0:
            for s in paused[:rem]:
                s.status = RUNNING
                batch.append(s)
        return [s.id for s in batch]

    def mark_prefilled(self, sid):
        if sid in self.seqs:
            self.seqs[sid].status = RUNNING

    def mark_decoded(self, sid):
        if sid in self.seqs:
            self.seqs[sid].generated += 1

    def preempt(self, sid):
        if sid in self.seqs:
            self.seqs[sid].status = PAUSED

    def handle_memory_pressure(self, required: int, available) -> list:
        out = []
        while available() < required:
            cands = sorted((s for s in self.seqs.values() if s.status == RUNNING),
                           key=lambda s: -s.arrival)
            if not cands:
                break
            cands[0].status = PAUSED
            out.append(cands[0].id)
        return out

    def count(self, status):
        return sum(1 for s in self.seqs.values() if s.status == status)
