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
}
FP16_WEIGHTS = {"tinyllama_2layer", "llama3_8b_2layer"}

BLOCK_SIZE = 16
MAX_BATCH_TOKENS = 2048  # the whole prompt is one chunk


def config_of(name: str):
    return GOLDENS[name][0]


def prompt_of(name: str) -> list:
    c, n, _ = GOLDENS[name]
    return np.random.default_rng(0).integers(0, c.vocab, size=n).astype(np.int32).tolist()


def _to_f16_values(a):
    if a is None:
        return None
    np.copyto(a, a.astype(np.float16).astype(np.float32))  # RNE, in place
    return a


def weights_for(name: str) -> HostWeights:
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
