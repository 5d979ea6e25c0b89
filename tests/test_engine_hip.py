"""relay's own Engine driving the HIP backend: oracle/_ref/relay_engine_hip links the
reference's engine.cpp and CPU backend (built from its sources by oracle/Makefile) with this
build's HipBackend compiled against relay's own headers, and runs the same requests through
relay's scheduler -- continuous batching, chunked prefill (engine.cpp:173-254), prefix
caching, preemption under a full cache -- once on the CPU backend and once on the HIP backend.
Greedy tokens must be identical and every logits row close (relay's test_reference metric):
2e-3 for the synthetic fp16-valued models, relay's own 2e-2 GPU bar for the Hugging Face
fixtures (bf16/fp32 checkpoints uploaded as fp16). The engine's own counters must agree too.
The binary is built where the reference tree exists (build()); without it these skip."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "oracle", "_ref", "relay_engine_hip")
FIX = os.path.join(REPO, "tests", "golden", "fixtures")


def engine(model, num_blocks, block_size, max_batch_tokens, max_seqs, prefix, requests, seed):
    if not os.path.exists(BIN):
        pytest.skip("oracle/_ref/relay_engine_hip was not built (needs the reference tree at build time)")
    args = [str(a) for a in (model, num_blocks, block_size, max_batch_tokens, max_seqs, int(prefix), requests, seed)]
    print("relay_engine_hip", " ".join(args), flush=True)
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-4000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print(out, flush=True)
    assert out["backend"] == "hip"
    return out


SYN64 = "synthetic:256,512,2,8,2,64,512,0"

CASES = {
    # chunked prefill (prompts longer than the 64-token budget) mixed with decode steps
    "chunked": (SYN64, 64, 16, 64, 8, False, "5:12,40:10,130:8,300:6,17:12", 1),
    # four prompts sharing a 64-token prefix
    "prefix_cache": (SYN64, 64, 16, 128, 8, True, "96:6:64,100:6:64,150:6:64,64:6:64", 2),
    # a cache of 12 blocks for three requests of 80 tokens: the youngest is preempted
    "preemption": (SYN64, 12, 16, 64, 8, False, "60:20,60:20,60:20", 3),
    # head size 128, qkv bias (Qwen2), block size 32, prefix caching (one request at a time)
    "d128_bias_bs32": ("synthetic:256,512,2,4,2,128,512,1", 64, 32, 96, 1, True, "70:8,72:8:64,75:8:64", 4),
    # head size 32 (the fast kernels at width 32), block size 8
    "d32_bs8": ("synthetic:128,256,2,4,4,32,256,0", 96, 8, 48, 4, False, "25:10,50:10,7:10", 5),
}


@pytest.mark.parametrize("name", list(CASES))
def test_relay_engine_on_hip_matches_cpu(dev, name):
    model, nb, bs, mbt, ms, prefix, reqs, seed = CASES[name]
    out = engine(model, nb, bs, mbt, ms, prefix, reqs, seed)
    assert out["tokens_equal"]
    assert out["rows"] > 0 and out["worst_rel"] < 2e-3
    assert out["steps"][0] == out["steps"][1]
    assert out["preemptions"][0] == out["preemptions"][1]
    assert out["prefix_hit_tokens"][0] == out["prefix_hit_tokens"][1]
    if name == "preemption":
        assert out["preemptions"][0] > 0
    if prefix:
        assert out["prefix_hit_tokens"][0] > 0


@pytest.mark.parametrize("fixture", ["llama3-rope", "qwen2-bias", "llama-gqa-tied-bf16"])
def test_relay_engine_on_hip_with_fixture_models(dev, fixture):
    """The reference's Hugging Face fixtures, loaded by relay's own HostWeights::load (head
    sizes 16 and 8: the fast kernels and the reference kernel)."""
    out = engine(os.path.join(FIX, fixture), 64, 16, 32, 4, True, "20:12,45:10:32,9:12,45:6:32", 7)
    assert out["tokens_equal"]
    assert out["worst_rel"] < 2e-2
    assert out["steps"][0] == out["steps"][1]


@pytest.mark.parametrize("blocks,block_size,mbt", [(18, 4, 64), (128, 1, 512), (8, 32, 512)])
def test_relay_batching_schedules_keep_greedy_tokens(dev, blocks, block_size, mbt):
    """The schedules of relay's test_batching.cpp:97-120 (a cache of 18 blocks of 4 tokens
    that forces preemption and recompute; block sizes 1 and 32) with its prompt lengths and
    token counts, all greedy: the HIP backend's tokens equal relay's CPU backend's under each
    schedule (the sampled requests of that program are not held bitwise across schedules on
    a non-exact backend, test_relay_suites_hip.py)."""
    reqs = ",".join(f"{n}:{3 + (i * 5) % 11}" for i, n in enumerate([1, 5, 17, 33, 2, 48, 9, 16]))
    out = engine(os.path.join(FIX, "llama-gqa-tied-bf16"), blocks, block_size, mbt, 8, False, reqs, 11)
    assert out["tokens_equal"]
    assert out["worst_rel"] < 2e-2
    assert out["steps"][0] == out["steps"][1] and out["preemptions"][0] == out["preemptions"][1]
    if blocks == 18:
        assert out["preemptions"][0] > 0

