"""Shared test helpers: seeded paged-cache cases and relay's comparison metrics."""
from __future__ import annotations

import numpy as np


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


def bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(h, np.uint16).view(np.float16).astype(np.float32)


class PagedCase:
    """A step's worth of paged-attention inputs: per sequence a chunk of `n_new` tokens
    ending at context `ctx` (decode when n_new == 1), block tables drawn from a seeded
    permutation of the pool, fp16 Q/K/V ~ N(0, scale)."""

    def __init__(self, ctxs, n_new, heads, kv_heads, D, block_size, seed=0, extra_blocks=3, value_scale=1.0):
        rng = np.random.default_rng(seed)
        self.heads, self.kv_heads, self.D, self.bs = heads, kv_heads, D, block_size
        need = [(c + block_size - 1) // block_size for c in ctxs]
        self.num_blocks = sum(need) + extra_blocks
        perm = rng.permutation(self.num_blocks)
        self.tables, self.table_off, self.pos, self.seq = [], [], [], []
        off = 0
        for s, (c, nb) in enumerate(zip(ctxs, need)):
            self.table_off.append(len(self.tables))
            self.tables.extend(int(b) for b in perm[off:off + nb])
            off += nb
            k = n_new[s] if isinstance(n_new, (list, tuple)) else n_new
            for p in range(c - k, c):
                self.pos.append(p)
                self.seq.append(s)
        self.T = len(self.pos)
        elems = self.num_blocks * kv_heads * block_size * D
        self.kpool = f16_bits(rng.standard_normal(elems, dtype=np.float32) * value_scale)
        self.vpool = f16_bits(rng.standard_normal(elems, dtype=np.float32) * value_scale)
        self.q = f16_bits(rng.standard_normal((self.T, heads * D), dtype=np.float32) * value_scale)
        self.meta = {"pos": np.array(self.pos, np.int32), "seq": np.array(self.seq, np.int32),
                     "table_off": np.array(self.table_off, np.int32), "tables": np.array(self.tables, np.int32)}

    def dec_meta(self, tokens=None) -> np.ndarray:
        """rh_paged_decode_attention's descriptors: (row, context, table offset, 0) per token."""
        toks = range(self.T) if tokens is None else tokens
        return np.array([[t, self.pos[t] + 1, self.table_off[self.seq[t]], 0] for t in toks], np.int32)

    def to_device(self, torch, dev):
        t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dev) if dt is None else \
            torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(dev)
        return {"q": t(self.q, np.int16), "k": t(self.kpool, np.int16), "v": t(self.vpool, np.int16),
                "pos": t(self.meta["pos"], None), "seq": t(self.meta["seq"], None),
                "table_off": t(self.meta["table_off"], None), "tables": t(self.meta["tables"], None)}


def rel_err_rowmax(a: np.ndarray, b: np.ndarray) -> float:
    """relay's test_reference metric: max |a - b| / max |b| per row, the worst row
    (test_reference.cpp:50-57)."""
    a = np.atleast_2d(a).astype(np.float64)
    b = np.atleast_2d(b).astype(np.float64)
    worst = 0.0
    for x, y in zip(a, b):
        worst = max(worst, float(np.abs(x - y).max() / max(1e-6, np.abs(y).max())))
    return worst


def rel_diff_l2(a: np.ndarray, b: np.ndarray) -> float:
    """relay's test_attention metric: L2 of the difference over L2 of b
    (test_attention.cpp:25-32)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(((a - b) ** 2).sum() / (1e-12 + (b ** 2).sum())))
