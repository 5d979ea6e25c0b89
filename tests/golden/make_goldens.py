"""Writes tests/golden/<name>.npz for the whole-model goldens of tests/goldens.py by
running the reference's own CPU backend and Engine (oracle/_ref/librelay_ref.so, built by
`make -C oracle ref` from /root/reference) on the synthetic weights.

    python tests/golden/make_goldens.py [name ...]

The weights go to a temporary Hugging Face directory (config.json + model.safetensors,
fp32) that the reference's loader reads; nothing of the reference is copied. Each golden
is also checked against this repository's CPU oracle before it is written.
"""
from __future__ import annotations

import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # tests/
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # repo root
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))

import goldens as G  # noqa: E402
import oracle as O  # noqa: E402
from relay_amd.model import write_safetensors  # noqa: E402


def make_steps(name: str) -> None:
    """A step golden: the reference CPU backend with the seeded cache, the batches of
    goldens.run_steps; the committed file holds each row's SHA-256, the chosen tokens and
    the top-2 margins."""
    c = G.config_of(name)
    t = time.time()
    w = G.weights_for(name)
    _, total = G.step_layout(name)
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(c.to_hf_json(), f)
        write_safetensors(os.path.join(d, "model.safetensors"), w.to_hf_tensors())
        ref = O.RefBackend(d, total, G.BLOCK_SIZE)
        G.fill_step_kv(name, ref, fp16=False)
        want = G.run_steps(name, ref)
        del ref
    print(f"{name}: reference run {time.time() - t:.1f} s", flush=True)
    mine = G.run_step_oracle(name, w)
    same = np.array_equal(mine["tokens"], want["tokens"]) and np.array_equal(mine["rows"].view(np.uint32),
                                                                             want["rows"].view(np.uint32))
    print(f"{name}: oracle bit-identical to the reference: {same}", flush=True)
    if not same:
        raise SystemExit(f"{name}: the oracle differs from the reference build; not writing the golden")
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), tokens=want["tokens"], row_sha256=G.row_sha(want["rows"]),
                        margins=G.margins(want["rows"]))


def make(name: str) -> None:
    if name in G.STEP_GOLDENS:
        return make_steps(name)
    c, n, steps = G.GOLDENS[name]
    t = time.time()
    w = G.weights_for(name)
    prompt = G.prompt_of(name)
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(c.to_hf_json(), f)
        write_safetensors(os.path.join(d, "model.safetensors"), w.to_hf_tensors())
        ref = O.RefBackend(d, G.num_blocks(name), G.BLOCK_SIZE)
        tokens, rows = ref.generate(prompt, steps, G.MAX_BATCH_TOKENS)
        del ref
    print(f"{name}: reference run {time.time() - t:.1f} s", flush=True)
    mine = G.run_oracle(name, w)
    same = mine["tokens"].tolist() == tokens and np.array_equal(mine["rows"].view(np.uint32), rows.view(np.uint32))
    print(f"{name}: oracle bit-identical to the reference: {same}", flush=True)
    if not same:
        raise SystemExit(f"{name}: the oracle differs from the reference build; not writing the golden")
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), prompt=np.array(prompt, np.int32),
                        tokens=np.array(tokens, np.int32), row_sha256=G.row_sha(rows), margins=G.margins(rows))


if __name__ == "__main__":
    if not O.ref_available():
        raise SystemExit("oracle/_ref is not built (needs /root/reference): make -C oracle ref")
    for name in sys.argv[1:] or list(G.GOLDENS) + list(G.STEP_GOLDENS):
        make(name)
