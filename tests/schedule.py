"""relay's backend comparison schedule (tests/test_attention.cpp:39-138), restated: two
backends driven through the same forward passes. Several prompts are prefilled in
chunks, several per forward pass under a 2048-token budget; then decode steps in which
every sequence adds one token and every odd step also carries a throwaway prompt, so
decode and prefill share a batch. Backend A's greedy tokens feed both.
"""
from __future__ import annotations

import numpy as np

from helpers import rel_diff_l2
from relay_amd.backend import ForwardBatch, SeqChunk


class Mt19937:
    """std::mt19937 (the reference schedule draws its tokens with seed 7)."""

    def __init__(self, seed: int):
        self.mt = [0] * 624
        self.mt[0] = seed & 0xFFFFFFFF
        for i in range(1, 624):
            self.mt[i] = (1812433253 * (self.mt[i - 1] ^ (self.mt[i - 1] >> 30)) + i) & 0xFFFFFFFF
        self.i = 624

    def __call__(self) -> int:
        if self.i >= 624:
            for k in range(624):
                y = (self.mt[k] & 0x80000000) | (self.mt[(k + 1) % 624] & 0x7FFFFFFF)
                self.mt[k] = self.mt[(k + 397) % 624] ^ (y >> 1) ^ (0x9908B0DF if y & 1 else 0)
            self.i = 0
        y = self.mt[self.i]
        self.i += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        return y & 0xFFFFFFFF


def blocks_needed(prompt_lens, decode_steps, bs=16):
    return sum((n + decode_steps + 1 + bs - 1) // bs for n in prompt_lens) + 4


def compare(a, b, vocab, prompt_lens, chunk, decode_steps, bs=16):
    """Returns (worst L2 relative logit difference, argmax agreements, total rows)."""
    rng = Mt19937(7)
    seqs, next_block = [], 0
    for n in prompt_lens:
        toks = [rng() % vocab for _ in range(n)]
        table = list(range(next_block, next_block + (n + decode_steps + 1 + bs - 1) // bs))
        next_block += len(table)
        seqs.append({"tokens": toks, "table": table, "prompt": n, "done": 0})
    worst, agree, total = 0.0, 0, 0

    def run(batch, owners, first_token_only):
        nonlocal worst, agree, total
        la, lb = a.forward(batch), b.forward(batch)
        assert la.shape == lb.shape
        worst = max(worst, rel_diff_l2(lb, la))
        for r, o in enumerate(owners):
            ia, ib = int(np.argmax(la[r])), int(np.argmax(lb[r]))
            agree += ia == ib
            total += 1
            if o < 0:
                continue
            s = seqs[o]
            if not first_token_only or s["done"] == s["prompt"]:
                s["tokens"].append(ia)

    more = True
    while more:
        batch, owners, budget = ForwardBatch(), [], 2048
        for i, s in enumerate(seqs):
            left = s["prompt"] - s["done"]
            if left <= 0 or budget <= 0:
                continue
            n = min(left, chunk, budget)
            batch.seqs.append(SeqChunk(s["tokens"][s["done"]:s["done"] + n], s["done"], list(s["table"]), True))
            owners.append(i)
            s["done"] += n
            budget -= n
        more = any(s["done"] < s["prompt"] for s in seqs)
        run(batch, owners, True)
    for d in range(decode_steps):
        batch, owners = ForwardBatch(), []
        for i, s in enumerate(seqs):
            batch.seqs.append(SeqChunk([s["tokens"][s["done"]]], s["done"], list(s["table"]), True))
            owners.append(i)
            s["done"] += 1
        if d % 2 == 1:
            extra = [rng() % vocab for _ in range(40 + d)]
            batch.seqs.append(SeqChunk(extra, 0, list(range(next_block, next_block + 4)), True))
            owners.append(-1)
        run(batch, owners, False)
    return worst, agree, total
