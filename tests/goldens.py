"""Whole-model golden runs: synthetic weights, prompt and greedy continuation.

Each golden is a model shape, a prompt of uniform-random token ids and a number of
greedy steps. tests/golden/make_goldens.py runs it on the reference's own CPU backend
(oracle/_ref, built from /root/reference) and commits tests/golden/<name>.npz:
  prompt      int32 [n]          the prompt ids
  tokens      int32 [steps]      the greedy continuation
  row_sha256  bytes [steps, 32]  SHA-256 of each logits row (fp32 bytes); row 0 is the
                                 prompt's last row, row i the logits that chose tokens[i]
  margins     f32 [steps]        top-1 minus top-2 logit of each row
The CPU oracle must reproduce every row bit for bit (test_oracle.py); the GPU backend must
give the same tokens with every row within 2e-3 of the oracle's (test_e2e.py).

Weights: relay_amd.model.HostWeights.synthetic (counter-based N(0, 0.02), norms 1), seed 0;
fp32 for config 1, rounded to fp16 values (RNE) for the shapes of configs 3 and 5, whose
models are specified with fp16 weights. Scaled variants keep the full layer shapes (hidden,
heads, head_dim, intermediate, vocab) and cut the layer count and context, as the configs
allow for CPU runs.
"""
from __future__ import annotations

import dataclasses
import hashlib

import numpy as np

from relay_amd.model import HostWeights, llama3_8b, smollm2_135m, tinyllama_1b

# name -> (config, prompt length, greedy steps)
GOLDENS = {
    # BASELINE config 1 as specified: SmolLM2-135M shape, 512-token prompt, 128 steps.
    "smollm2_135m": (smollm2_135m(), 512, 128),
    # Config 3's shape (D 64, 32/4 heads), 2 layers, 256-token prompt.
    "tinyllama_2layer": (dataclasses.replace(tinyllama_1b(), layers=2), 256, 16),
    # Config 5's shape (D 128, 32/8 heads, llama3 RoPE scaling), 2 layers, 128-token prompt.
    "llama3_8b_2layer": (dataclasses.replace(llama3_8b(), layers=2), 128, 8),
    # Config 3(a)'s workload: one 2048-token prompt in one chunk, 2 layers.
    "tinyllama_2layer_p2048": (dataclasses.replace(tinyllama_1b(), layers=2), 2048, 4),
}
FP16_WEIGHTS = {"tinyllama_2layer", "llama3_8b_2layer", "tinyllama_2layer_p2048", "tinyllama_2layer_decode32",
                "llama3_8b_2layer_mixed"}

BLOCK_SIZE = 16
MAX_BATCH_TOKENS = 2048  # the whole prompt is one chunk


# Step goldens: batches at the configs' real batch shapes, on a KV cache whose earlier
# positions are filled with seeded fp16-valued N(0, 1) draws (the same values in every
# backend), so a step at context 2048 needs no 2048-token prefill on the CPU.
#   decode: contexts of the decode sequences (their token sits at position context - 1)
#   chunk:  tokens of one prefill chunk at position 0 in the same ForwardBatch (0: none)
#   steps:  forward steps; step 2 continues every sequence with its greedy token of step 1
STEP_GOLDENS = {
    # Config 3(b): one TinyLlama decode step of 32 sequences at context 2048, then one more.
    "tinyllama_2layer_decode32": dict(config=dataclasses.replace(tinyllama_1b(), layers=2), decode=[2048] * 32,
                                      chunk=0, steps=2),
    # Config 5's mixed step at Llama-3 layer shapes: 48 decode sequences (context 1024, so
    # the planner splits them) plus one 512-token chunk in one ForwardBatch, then one more.
    "llama3_8b_2layer_mixed": dict(config=dataclasses.replace(llama3_8b(), layers=2), decode=[1024] * 48,
                                   chunk=512, steps=2),
}


def config_of(name: str):
    if name in STEP_GOLDENS:
        return STEP_GOLDENS[name]["config"]
    return GOLDENS[name][0]


def prompt_of(name: str) -> list:
    c, n, _ = GOLDENS[name]
    return np.random.default_rng(0).integers(0, c.vocab, size=n).astype(np.int32).tolist()


def _to_f16_values(a):
    if a is None:
        return None
    import oracle as O

    # RNE, in place: the oracle's conversion (equal to numpy's cast, test_oracle.py), which
    # allocates nothing and runs on every core
    O.round_f16_inplace(a)
    return a


_WEIGHTS_CACHE = {}


def weights_for(name: str) -> HostWeights:
    """The golden's weights (the two last used are kept: goldens of one shape share them, and
    the test order alternates between the TinyLlama and Llama-3 shapes; at most ~7 GB)."""
    key = (repr(config_of(name)), name in FP16_WEIGHTS)
    if key in _WEIGHTS_CACHE:
        _WEIGHTS_CACHE[key] = _WEIGHTS_CACHE.pop(key)  # most recently used last
    else:
        while len(_WEIGHTS_CACHE) >= 2:
            del _WEIGHTS_CACHE[next(iter(_WEIGHTS_CACHE))]
        _WEIGHTS_CACHE[key] = _build_weights(name)
    return _WEIGHTS_CACHE[key]


def _build_weights(name: str) -> HostWeights:
    w = HostWeights.synthetic(config_of(name), seed=0)
    if name in FP16_WEIGHTS:
        for t in (w.embed, w.lm_head, w.final_norm):
            _to_f16_values(t)
        for L in w.layers:
            for f in ("attn_norm", "wqkv", "bqkv", "wo", "mlp_norm", "w_gate_up", "w_down"):
                _to_f16_values(getattr(L, f))
    return w


def num_blocks(name: str) -> int:
    _, n, steps = GOLDENS[name]
    return (n + steps + BLOCK_SIZE - 1) // BLOCK_SIZE + 1


def row_sha(rows: np.ndarray) -> np.ndarray:
    rows = np.ascontiguousarray(rows, np.float32)
    return np.array([np.frombuffer(hashlib.sha256(r.tobytes()).digest(), np.uint8) for r in rows])


def margins(rows: np.ndarray) -> np.ndarray:
    top2 = np.sort(rows, axis=1)[:, -2:]
    return (top2[:, 1] - top2[:, 0]).astype(np.float32)


def run_backend(name: str, backend) -> dict:
    """Greedy generation through relay's batch composition (relay_amd.engine.GreedyEngine,
    a mirror of engine.cpp:173-254) on any backend with relay's forward()."""
    from relay_amd.engine import GreedyEngine

    _, n, steps = GOLDENS[name]
    rows = []
    eng = GreedyEngine(backend, num_blocks(name), BLOCK_SIZE, MAX_BATCH_TOKENS, 8,
                       on_logits=lambda rid, i, row: rows.append(np.array(row, np.float32)))
    eng.add(1, prompt_of(name), steps)
    tokens = eng.run_all()[1]
    return {"tokens": np.array(tokens, np.int32), "rows": np.stack(rows)}


def run_oracle(name: str, w: HostWeights) -> dict:
    import oracle as O

    return run_backend(name, O.CpuBackend(w, num_blocks(name), BLOCK_SIZE))


# ---- step goldens ----------------------------------------------------------------------

def step_layout(name: str):
    """Block tables: every sequence's blocks, drawn from a seeded permutation of the pool."""
    g = STEP_GOLDENS[name]
    per = [(ctx + g["steps"] + BLOCK_SIZE - 1) // BLOCK_SIZE for ctx in g["decode"]]
    if g["chunk"]:
        per.append((g["chunk"] + g["steps"] + BLOCK_SIZE - 1) // BLOCK_SIZE)
    total = sum(per) + 3
    perm = np.random.default_rng(11).permutation(total).tolist()
    tables, o = [], 0
    for n in per:
        tables.append(perm[o:o + n])
        o += n
    return tables, total


def step_kv(name: str, layer: int):
    """The prefilled K and V of `layer`: for each decode sequence, its blocks' contents as
    fp32 arrays [blocks, kv_heads * block_size * head_dim] holding fp16 values."""
    c = config_of(name)
    g = STEP_GOLDENS[name]
    tables, _ = step_layout(name)
    rng = np.random.default_rng(1000 + layer)
    be = c.kv_heads * BLOCK_SIZE * c.head_dim
    out = []
    for i in range(len(g["decode"])):
        nb = len(tables[i])
        k = rng.standard_normal((nb, be), dtype=np.float32).astype(np.float16).astype(np.float32)
        v = rng.standard_normal((nb, be), dtype=np.float32).astype(np.float16).astype(np.float32)
        out.append((k, v))
    return out


def fill_step_kv(name: str, backend, fp16: bool) -> None:
    """Writes the prefilled cache into a backend: write_kv_block with fp32 arrays (the CPU
    backends) or with fp16 bytes (the HIP backend)."""
    c = config_of(name)
    tables, _ = step_layout(name)
    for layer in range(c.layers):
        for i, (k, v) in enumerate(step_kv(name, layer)):
            for j, blk in enumerate(tables[i]):
                if fp16:
                    backend.write_kv_block(layer, blk, k[j].astype(np.float16), v[j].astype(np.float16))
                else:
                    backend.write_kv_block(layer, blk, k[j], v[j])


def step_tokens(name: str):
    """Step 1's tokens: one seeded id per decode sequence, then the chunk's ids."""
    c = config_of(name)
    g = STEP_GOLDENS[name]
    rng = np.random.default_rng(7)
    dec = rng.integers(0, c.vocab, size=len(g["decode"])).tolist()
    chunk = rng.integers(0, c.vocab, size=g["chunk"]).tolist()
    return dec, chunk


def run_steps(name: str, backend, forced=None) -> dict:
    """The golden's steps on a backend whose cache step_kv filled: step 1 is the decode
    sequences (and the chunk) in one ForwardBatch; each later step feeds every sequence its
    greedy token, or forced[step] (the golden's tokens, so that every backend sees the same
    inputs). Returns the tokens chosen (argmax per row) and the logits rows."""
    from relay_amd.backend import ForwardBatch, SeqChunk

    g = STEP_GOLDENS[name]
    tables, _ = step_layout(name)
    dec, chunk = step_tokens(name)
    pos = [ctx - 1 for ctx in g["decode"]]
    feed = [[t] for t in dec]
    if g["chunk"]:
        pos.append(0)
        feed.append(chunk)
    all_rows, all_tokens = [], []
    for _ in range(g["steps"]):
        batch = ForwardBatch([SeqChunk(list(f), p, tables[i], True) for i, (f, p) in enumerate(zip(feed, pos))])
        rows = np.asarray(backend.forward(batch), np.float32)
        assert rows.shape[0] == len(feed)
        toks = [int(np.argmax(r)) for r in rows]
        all_rows.append(rows)
        all_tokens.append(toks)
        pos = [p + len(f) for p, f in zip(pos, feed)]
        feed = [[int(t)] for t in (toks if forced is None else forced[len(all_tokens) - 1])]
    return {"tokens": np.array(all_tokens, np.int32), "rows": np.concatenate(all_rows)}


def run_step_oracle(name: str, w: HostWeights) -> dict:
    import oracle as O

    _, total = step_layout(name)
    cpu = O.CpuBackend(w, total, BLOCK_SIZE)
    fill_step_kv(name, cpu, fp16=False)
    return run_steps(name, cpu)
