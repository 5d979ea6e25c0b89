"""A minimal greedy generation loop with relay's batch composition.

Each step builds one ForwardBatch the way relay's Engine::step_locked does
(engine.cpp:173-254): first the requests that are generating, one token each, oldest
first; then prompt chunks (requests part-way through their prompt first, then new ones)
under the max_batch_tokens budget. Greedy sampling is relay's argmax, lowest id on ties
(sampler.cpp:17-22). Prefix caching, preemption, temperature sampling and the
thread-safe API are relay's scheduler concerns and are not restated here: this loop
exists to drive a backend (ours or the CPU oracle) through the same schedule relay uses.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .backend import ForwardBatch, SeqChunk


def argmax(row: np.ndarray) -> int:
    """Index of the largest value; ties go to the lowest index (np.argmax does the same)."""
    return int(np.argmax(row))


@dataclass
class _Seq:
    rid: int
    tokens: list
    max_new: int
    computed: int = 0
    generated: int = 0
    blocks: list = field(default_factory=list)
    done: bool = False


class GreedyEngine:
    def __init__(self, backend, num_blocks: int, block_size: int, max_batch_tokens: int = 512, max_seqs: int = 64,
                 on_logits=None):
        self.be = backend
        self.bs = block_size
        self.budget = max_batch_tokens
        self.max_seqs = max_seqs
        self.free = list(range(num_blocks - 1, -1, -1))  # a stack: block 0 is handed out first
        self.waiting: list[_Seq] = []
        self.running: list[_Seq] = []
        self.on_logits = on_logits
        self.steps = 0

    def add(self, rid: int, prompt: list, max_new_tokens: int) -> None:
        if not prompt:
            raise ValueError("empty prompt")
        self.waiting.append(_Seq(rid, list(prompt), max_new_tokens))

    def _ensure(self, s: _Seq, tokens: int) -> bool:
        need = (tokens + self.bs - 1) // self.bs - len(s.blocks)
        if need <= 0:
            return True
        if need > len(self.free):
            return False
        for _ in range(need):
            s.blocks.append(self.free.pop())
        return True

    def step(self) -> list:
        batch, members = ForwardBatch(), []
        budget = self.budget
        for s in self.running:  # admission order = oldest first
            if len(s.tokens) - s.computed == 1 and budget > 0:
                if not self._ensure(s, len(s.tokens)):
                    raise RuntimeError("KV cache full (this loop does not preempt)")
                batch.seqs.append(SeqChunk([s.tokens[-1]], s.computed, list(s.blocks), True))
                members.append(s)
                budget -= 1

        def add_chunk(s: _Seq) -> bool:
            nonlocal budget
            n = min(len(s.tokens) - s.computed, budget)
            if n <= 0 or not self._ensure(s, s.computed + n):
                return False
            batch.seqs.append(SeqChunk(s.tokens[s.computed:s.computed + n], s.computed, list(s.blocks),
                                       s.computed + n == len(s.tokens)))
            members.append(s)
            budget -= n
            return True

        for s in self.running:
            if budget == 0:
                break
            if len(s.tokens) - s.computed > 1:
                add_chunk(s)
        while budget > 0 and self.waiting and len(self.running) < self.max_seqs:
            s = self.waiting[0]
            if not add_chunk(s):
                break
            self.running.append(self.waiting.pop(0))
        if not batch.seqs:
            return []
        logits = self.be.forward(batch)
        self.steps += 1
        events, r = [], 0
        for s, ch in zip(members, batch.seqs):
            s.computed += len(ch.tokens)
            if not ch.want_logits:
                continue
            row = logits[r]
            r += 1
            if self.on_logits:
                self.on_logits(s.rid, s.generated, row)
            tok = argmax(row)
            s.generated += 1
            s.tokens.append(tok)
            events.append((s.rid, tok))
            if s.generated >= s.max_new:
                s.done = True
        for s in [s for s in self.running if s.done]:
            self.free.extend(reversed(s.blocks))
            s.blocks = []
            self.running.remove(s)
        return events

    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def run_all(self) -> dict:
        out: dict = {}
        while self.has_work():
            for rid, tok in self.step():
                out.setdefault(rid, []).append(tok)
        return out
