"""The HIP backend end to end, with relay's own model-level tests as the pattern:

- test_reference.cpp: prompt logits and greedy continuations against the Hugging Face
  logits in the reference's fixtures (GPU tolerance 2e-2, relay's), and against the
  CPU oracle;
- test_attention.cpp: the comparison schedule (chunked prompts, offsets, mixed decode +
  prefill batches) -- fast kernels vs the CPU oracle, fast vs the reference kernel on
  the GPU (relay's M1-vs-M0), int8 vs fp16;
- test_kv_cache.cpp:67-102: KV blocks moved to another backend decode identically;
- update_weight and the error conventions of relay's backends.
The fixtures have head_dim 8 or 16, which the fast kernels do not cover (they run on
the reference kernel, as relay's M1 falls back to M0); the fast kernels are exercised
by synthetic models with head_dim 64 and 128.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from helpers import rel_err_rowmax
from relay_amd import HipBackend, HipOptions
from relay_amd.backend import ForwardBatch, SeqChunk
from relay_amd.engine import GreedyEngine
from relay_amd.model import HostWeights, ModelConfig
from schedule import blocks_needed, compare

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(__file__), "golden", "fixtures")
MODELS = ["chat-tiny", "llama-gqa-tied-bf16", "llama-mha", "llama3-rope", "qwen2-bias"]
FAST = HipOptions(False, False)
REF = HipOptions(True, False)


def small_model(D, heads, kv_heads, layers=2, vocab=512, hidden=256, inter=512, std=0.1, llama3=False, bias=False,
                seed=0):
    c = ModelConfig(hidden=hidden, intermediate=inter, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=D,
                    vocab=vocab, tie_embeddings=not bias, qkv_bias=bias, rope_theta=500000.0 if llama3 else 10000.0,
                    rope_llama3=llama3, rope_factor=8.0, model_type="qwen2" if bias else "llama")
    return HostWeights.synthetic(c, seed=seed, std=std, norm_one=False)


@pytest.mark.parametrize("model", MODELS)
def test_prompt_logits_match_transformers(dev, model):
    d = os.path.join(FIX, model)
    w = HostWeights.load(d)
    ref = json.load(open(os.path.join(d, "relay-reference.json")))
    p = ref["prompt"]
    be = HipBackend(w, 64, 16, options=FAST)
    b = ForwardBatch([SeqChunk(p, 0, list(range((len(p) + 15) // 16)), True)],
                     all_logits=not ref.get("prompt_logits_last_only", False))
    lg = be.forward(b)
    hf = np.array(ref["prompt_logits"], np.float32)
    err = rel_err_rowmax(lg[:len(hf)], hf)
    cpu = O.CpuBackend(w, 64, 16).forward(b)
    err_cpu = rel_err_rowmax(lg, cpu)
    print(f"{model}: vs transformers {err:.2e}, vs CPU oracle {err_cpu:.2e}")
    assert err < 2e-2 and err_cpu < 2e-2


@pytest.mark.parametrize("model", MODELS)
def test_greedy_generation_matches_transformers(dev, model):
    d = os.path.join(FIX, model)
    w = HostWeights.load(d)
    ref = json.load(open(os.path.join(d, "relay-reference.json")))
    be = HipBackend(w, 64, 16, max_batch_tokens=512, options=FAST)
    seen = []
    eng = GreedyEngine(be, 64, 16, max_batch_tokens=512, max_seqs=8, on_logits=lambda r, i, row: seen.append(row.copy()))
    eng.add(1, ref["prompt"], len(ref["generated"]))
    out = eng.run_all()
    worst = max(rel_err_rowmax(s, np.array(r, np.float32)) for s, r in zip(seen, ref["step_logits"]))
    print(f"{model}: generated {'identical' if out[1] == ref['generated'] else 'DIFFERENT'}, worst {worst:.2e}")
    assert out[1] == ref["generated"]
    assert worst < 2e-2


@pytest.mark.parametrize("D,heads,kv_heads", [(64, 8, 2), (64, 9, 3), (128, 8, 2), (64, 32, 4)])
def test_fast_kernels_match_cpu_oracle(dev, D, heads, kv_heads):
    """GPU vs the fp32 CPU oracle on relay's comparison schedule (test_attention.cpp:43-138) at
    relay's bar (1e-2). The synthetic weights are rounded to fp16 values first, so the oracle
    and the GPU see the same weights and the difference measures the GPU arithmetic (fp16
    activations and attention weights); with fp32 weights the fp16 upload alone puts the
    32/4-head case at ~1e-2."""
    w = small_model(D, heads, kv_heads, hidden=heads * D // 2)
    for L in w.layers:
        for f in ("attn_norm", "wqkv", "bqkv", "wo", "mlp_norm", "w_gate_up", "w_down"):
            a = getattr(L, f)
            if a is not None:
                np.copyto(a, a.astype(np.float16).astype(np.float32))
    for a in (w.embed, w.lm_head, w.final_norm):
        if a is not None:
            np.copyto(a, a.astype(np.float16).astype(np.float32))
    lens = [1, 17, 64, 200, 700, 1300]
    nb = blocks_needed(lens, 12)
    a = O.CpuBackend(w, nb, 16)
    b = HipBackend(w, nb, 16, max_batch_tokens=2048, options=FAST)
    worst, agree, total = compare(a, b, w.config.vocab, lens, 192, 12)
    print(f"D={D} G={heads // kv_heads}: worst relative logit difference {worst:.2e}, argmax {agree}/{total}")
    assert worst < 1e-2
    assert agree >= total - max(1, total // 50)


@pytest.mark.parametrize("D,heads,kv_heads,llama3,bias", [(64, 8, 2, False, False), (128, 8, 4, True, False),
                                                          (64, 6, 6, False, True)])
def test_fast_equals_reference_kernel(dev, D, heads, kv_heads, llama3, bias):
    """relay's m1_attention_equals_m0_attention: same GPU, two attention paths."""
    w = small_model(D, heads, kv_heads, hidden=256, llama3=llama3, bias=bias, seed=D)
    lens = [1, 37, 300, 700]
    nb = blocks_needed(lens, 8)
    a = HipBackend(w, nb, 16, max_batch_tokens=2048, options=REF)
    b = HipBackend(w, nb, 16, max_batch_tokens=2048, options=FAST)
    worst, agree, total = compare(a, b, w.config.vocab, lens, 256, 8)
    print(f"fast vs reference kernel D={D}: worst {worst:.2e}, argmax {agree}/{total}")
    assert worst < 1e-2
    assert agree >= total - max(1, total // 50)


def test_int8_weights_stay_close_to_fp16(dev):
    w = small_model(64, 8, 2, hidden=512, inter=1024)
    lens = [5, 60, 130]
    nb = blocks_needed(lens, 10)
    a = HipBackend(w, nb, 16, max_batch_tokens=2048, options=FAST)
    b = HipBackend(w, nb, 16, max_batch_tokens=2048, options=HipOptions(False, True))
    worst, agree, total = compare(a, b, w.config.vocab, lens, 64, 10)
    print(f"int8 vs fp16: relative logit difference {worst:.2e}, argmax {agree}/{total}")
    assert worst < 0.25


def test_kv_blocks_moved_to_another_backend_decode_identically(dev):
    w = small_model(64, 8, 2)
    prefill = HipBackend(w, 16, 4, options=FAST)
    decode = HipBackend(w, 16, 4, options=FAST)
    prompt = [5, 17, 99, 3, 42, 7, 64, 1, 8, 120, 33]
    src, dst = [0, 1, 2], [13, 6, 9]
    first = prefill.forward(ForwardBatch([SeqChunk(prompt, 0, src, True)]))
    nxt = int(np.argmax(first[0]))
    for l in range(w.config.layers):
        data = prefill.read_kv_layer(l, src)
        decode.write_kv_layer(l, dst, data)
        for i in range(len(src)):  # the block API sees the same bytes
            k, v = decode.read_kv_block(l, dst[i])
            bb = prefill.kv_block_bytes()
            assert np.array_equal(k, data[i * bb:(i + 1) * bb])
            assert np.array_equal(v, data[(len(src) + i) * bb:(len(src) + i + 1) * bb])
    for step in range(5):
        p = len(prompt) + step
        if p // 4 >= len(src):
            src.append(3 + step)
            dst.append(2 + step)
        la = prefill.forward(ForwardBatch([SeqChunk([nxt], p, list(src), True)]))
        lc = decode.forward(ForwardBatch([SeqChunk([nxt], p, list(dst), True)]))
        assert np.array_equal(la.view(np.uint32), lc.view(np.uint32))
        nxt = int(np.argmax(la[0]))


def test_update_weight_equals_a_rebuilt_backend(dev):
    w = small_model(64, 8, 2)
    be = HipBackend(w, 8, 16, options=FAST)
    rng = np.random.default_rng(4)
    batch = ForwardBatch([SeqChunk([1, 2, 3, 4, 5], 0, [0], True)])
    new_embed = (rng.standard_normal(w.embed.shape) * 0.1).astype(np.float32)
    new_wo = (rng.standard_normal(w.layers[1].wo.shape) * 0.1).astype(np.float32)
    be.update_weight("embed", new_embed)
    be.update_weight("layers.1.wo", new_wo)
    w.embed[...] = new_embed
    w.layers[1].wo[...] = new_wo
    fresh = HipBackend(w, 8, 16, options=FAST)
    assert np.array_equal(be.forward(batch).view(np.uint32), fresh.forward(batch).view(np.uint32))
    with pytest.raises(ValueError):
        be.update_weight("embed", new_embed[:10])
    with pytest.raises(ValueError):
        be.update_weight("layers.9.wo", new_wo)
    with pytest.raises(ValueError):
        be.update_weight("nonsense", new_wo)
    q8 = HipBackend(w, 8, 16, options=HipOptions(False, True))
    with pytest.raises(RuntimeError):
        q8.update_weight("layers.0.wqkv", w.layers[0].wqkv)


def test_errors_follow_relay_conventions(dev):
    w = small_model(64, 8, 2)
    be = HipBackend(w, 8, 16, max_batch_tokens=64, max_context=100, options=FAST)
    with pytest.raises(ValueError):  # block table too short
        be.forward(ForwardBatch([SeqChunk(list(range(20)), 0, [0], True)]))
    with pytest.raises(IndexError):  # token id out of range
        be.forward(ForwardBatch([SeqChunk([w.config.vocab], 0, [0], True)]))
    with pytest.raises(ValueError):  # more tokens than max_batch_tokens
        be.forward(ForwardBatch([SeqChunk([1] * 65, 0, list(range(5)), True)]))
    with pytest.raises(ValueError):  # longer than max_context
        be.forward(ForwardBatch([SeqChunk([1], 100, list(range(7)), True)]))
    assert be.forward(ForwardBatch([])).shape[0] == 0
    with pytest.raises(ValueError):  # an empty chunk that wants logits (relay's backends read another row)
        be.forward(ForwardBatch([SeqChunk([3, 4], 0, [0], True), SeqChunk([], 0, [1], True)]))
    # an empty chunk that wants none is skipped: same logits as without it
    a = be.forward(ForwardBatch([SeqChunk([3, 4], 0, [0], True)]))
    b = be.forward(ForwardBatch([SeqChunk([3, 4], 0, [0], True), SeqChunk([], 0, [1], False)]))
    assert a.shape == b.shape and np.array_equal(a, b)


def test_library_gemm_choices_agree(dev, monkeypatch):
    """Prompts above the skinny product's token range run their projections as library GEMMs:
    hipBLASLt with a timed kernel choice by default, rocBLAS' own choice with
    RELAY_HIP_GEMM=rocblas. Both are fp32 sums of the same fp16 products, so the logits agree
    to accumulation-order rounding and the greedy tokens are the same; both stay within 2e-3
    of the CPU oracle."""
    w = small_model(64, 8, 2, layers=2, hidden=512, inter=1024, vocab=1024, std=0.05, seed=5)
    for L in w.layers:  # fp16 values, so the oracle and the GPU see the same weights
        for f in ("attn_norm", "wqkv", "wo", "mlp_norm", "w_gate_up", "w_down"):
            a = getattr(L, f)
            np.copyto(a, a.astype(np.float16).astype(np.float32))
    for a in (w.embed, w.lm_head, w.final_norm):
        if a is not None:
            np.copyto(a, a.astype(np.float16).astype(np.float32))
    prompt = list(np.random.default_rng(1).integers(0, 1024, size=200))
    b = ForwardBatch([SeqChunk(prompt, 0, list(range(13)), True)], all_logits=True)
    got = {}
    for mode in ("default", "rocblas"):
        if mode == "rocblas":
            monkeypatch.setenv("RELAY_HIP_GEMM", "rocblas")
        else:
            monkeypatch.delenv("RELAY_HIP_GEMM", raising=False)
        print(f"library gemm mode {mode}: T={len(prompt)}", flush=True)
        be = HipBackend(w, 16, 16, max_batch_tokens=256, options=FAST)
        got[mode] = be.forward(b)
        be.close()
    cpu = O.CpuBackend(w, 16, 16).forward(b)
    # hipBLASLt's kernel is chosen by timing, so the pair's summation orders vary between runs
    # (measured up to 1.07e-3 apart); each is held to the oracle's 2e-3 below.
    assert rel_err_rowmax(got["default"], got["rocblas"]) < 2e-3
    assert (got["default"].argmax(axis=1) == got["rocblas"].argmax(axis=1)).mean() >= 0.98
    for mode in got:
        assert rel_err_rowmax(got[mode], cpu) < 2e-3, mode


@pytest.mark.parametrize("heads,hidden,n_seq", [(4, 256, 20), (8, 512, 32)])
def test_int8_paths_match_fp16_on_exactly_quantizable_weights(dev, heads, hidden, n_seq):
    """Weights of the form q * 2^-9 with a +-127 in every row quantize exactly (scale 2^-9,
    the same q back), so the int8 backend multiplies the same values as the fp16 one and the
    logits may differ only by fp32 summation order (amplified where an activation is rounded
    to fp16 between layers: measured 2e-4; a wrong product would be off by O(1)). intermediate 8192 and 20 decode
    sequences put gate_up (N 16384) and down (K 8192) on the split-K int8 GEMM at 20
    tokens; the prompts (100 tokens) take the large-tile int8 GEMM with its K split. At 32
    sequences the 512 x 512 o projection is split over K as well, merged by the MLP RMSNorm."""
    w = small_model(64, heads, 2, layers=1, hidden=hidden, inter=8192, vocab=512, seed=3)
    rng = np.random.default_rng(11)
    for L in w.layers:
        for f in ("wqkv", "wo", "w_gate_up", "w_down"):
            a = getattr(L, f)
            q = rng.integers(-127, 128, size=a.shape).astype(np.float32)
            q[:, 0] = np.where(rng.random(a.shape[0]) < 0.5, 127.0, -127.0)
            np.copyto(a, q * 2.0 ** -9)
    lens = [5] * n_seq
    nb = blocks_needed(lens, 4)
    a = HipBackend(w, nb, 16, max_batch_tokens=2048, options=FAST)
    b = HipBackend(w, nb, 16, max_batch_tokens=2048, options=HipOptions(False, True))
    worst, agree, total = compare(a, b, w.config.vocab, lens, 64, 4)
    print(f"int8 vs fp16, exactly quantizable weights: relative logit difference {worst:.2e}, argmax {agree}/{total}")
    assert worst < 1e-3 and agree >= total - 1


def test_read_kv_layer_into_a_caller_buffer(dev):
    """read_kv_layer into a buffer the caller keeps gives the same bytes as into a new one
    (relay's KVSender reuses its buffer), and a buffer of the wrong size is refused."""
    w = small_model(64, 8, 2)
    be = HipBackend(w, 64, 16, options=FAST)
    be.fill_kv_random(seed=2, std=1.0)
    blocks = [5, 0, 63, 17, 17, 40]
    fresh = be.read_kv_layer(1, blocks)
    buf = np.full_like(fresh, 0xAB)
    assert be.read_kv_layer(1, blocks, out=buf) is buf and np.array_equal(buf, fresh)
    with pytest.raises(ValueError):
        be.read_kv_layer(1, blocks, out=np.empty(fresh.size - 1, np.uint8))
    be.close()
