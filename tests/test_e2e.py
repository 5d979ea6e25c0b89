"""End-to-end parity of the HIP backend with the CPU oracle on the whole-model goldens
(tests/goldens.py): BASELINE config 1 (SmolLM2-135M shape, 512-token prompt, 128 greedy
steps) and 2-layer variants of configs 3 and 5.

The oracle (the fp32 CPU restatement, bit-identical to the reference build's CPU backend
on these goldens, test_oracle.py) runs on the same synthetic weights. The bar
(north star): the same greedy tokens as the committed golden, and every logits row within
2e-3 of the oracle's, measured as max|gpu - cpu| / max|cpu| per row (test_reference.cpp:50-57).
"""
import numpy as np
import pytest

import goldens as G
from helpers import rel_err_rowmax

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.mark.parametrize("name", ["smollm2_135m", "tinyllama_2layer", "llama3_8b_2layer"])
def test_greedy_run_matches_the_oracle(dev, name):
    import os

    from relay_amd.backend import HipBackend, HipOptions

    golden = np.load(os.path.join(os.path.dirname(__file__), "golden", f"{name}.npz"), allow_pickle=False)
    w = G.weights_for(name)
    print(f"e2e {name}: oracle run", flush=True)
    want = G.run_oracle(name, w)
    assert want["tokens"].tolist() == golden["tokens"].tolist()
    print(f"e2e {name}: HIP run", flush=True)
    be = HipBackend(w, G.num_blocks(name), G.BLOCK_SIZE, max_batch_tokens=G.MAX_BATCH_TOKENS,
                    options=HipOptions(False, False))
    got = G.run_backend(name, be)
    be.close()
    errs = [rel_err_rowmax(a, b) for a, b in zip(got["rows"], want["rows"])]
    print(f"e2e {name}: rows {len(errs)}, worst rel err {max(errs):.2e} (row {int(np.argmax(errs))}), "
          f"smallest top-2 margin {float(golden['margins'].min()):.3e}", flush=True)
    assert got["tokens"].tolist() == golden["tokens"].tolist()
    assert max(errs) <= TOL
