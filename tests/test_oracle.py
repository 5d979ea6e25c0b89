"""Pins the CPU oracle (oracle/cpu_oracle.cpp) before anything is checked against it.

- Whole model: bit-for-bit equal to relay's own CPU backend built from /root/reference
  (oracle/_ref; skipped where that build is absent) on every fixture and on a chunked,
  batched schedule; within relay's CPU tolerance (1e-4) of the Hugging Face logits the
  reference's fixtures hold, with identical greedy continuations; equal to the committed
  goldens made by the reference build (tests/golden/*.npz).
- fp32 -> fp16: equal to the reference build and to numpy's IEEE round-to-nearest-even
  cast on special values, halfway cases, subnormals and random bit patterns.
- RoPE frequencies: equal to the reference build; the unscaled ones to the closed form.
- Attention: against a double-precision brute force (a different summation route), and
  against what the mathematics fixes (equal keys give the mean of V; one dominant key
  gives its V row).
- int8 quantizer: the properties that define it (max maps to +-127, round half to even,
  reconstruction within half a step, zero rows).
- int8 GEMV oracle: exact rational arithmetic on a small case, closed forms.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle as O
from helpers import PagedCase, bits_to_f32, f16_bits, rel_err_rowmax
from relay_amd.backend import ForwardBatch, SeqChunk
from relay_amd.engine import GreedyEngine
from relay_amd.model import HostWeights, ModelConfig
from schedule import blocks_needed, compare

FIX = os.path.join(os.path.dirname(__file__), "golden", "fixtures")
MODELS = ["chat-tiny", "llama-gqa-tied-bf16", "llama-mha", "llama3-rope", "qwen2-bias"]
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no /root/reference here)")


def prompt_batch(ref):
    p = ref["prompt"]
    return ForwardBatch([SeqChunk(p, 0, list(range((len(p) + 15) // 16)), True)],
                        all_logits=not ref.get("prompt_logits_last_only", False))


@pytest.mark.parametrize("model", MODELS)
def test_prompt_logits_match_transformers(model):
    d = os.path.join(FIX, model)
    w = HostWeights.load(d)
    ref = json.load(open(os.path.join(d, "relay-reference.json")))
    lg = O.CpuBackend(w, 64, 16).forward(prompt_batch(ref))
    hf = np.array(ref["prompt_logits"], np.float32)
    assert rel_err_rowmax(lg[:len(hf)], hf) < 1e-4


@pytest.mark.parametrize("model", MODELS)
def test_greedy_generation_matches_transformers(model):
    d = os.path.join(FIX, model)
    w = HostWeights.load(d)
    ref = json.load(open(os.path.join(d, "relay-reference.json")))
    seen = []
    eng = GreedyEngine(O.CpuBackend(w, 64, 16), 64, 16, 512, 8, on_logits=lambda r, i, row: seen.append(row.copy()))
    eng.add(1, ref["prompt"], len(ref["generated"]))
    assert eng.run_all()[1] == ref["generated"]
    assert max(rel_err_rowmax(s, np.array(r, np.float32)) for s, r in zip(seen, ref["step_logits"])) < 1e-4


@needs_ref
@pytest.mark.parametrize("model", MODELS)
def test_bit_identical_to_the_reference_build(model):
    d = os.path.join(FIX, model)
    w = HostWeights.load(d)
    ref = json.load(open(os.path.join(d, "relay-reference.json")))
    b = prompt_batch(ref)
    assert np.array_equal(O.CpuBackend(w, 64, 16).forward(b).view(np.uint32),
                          O.RefBackend(d, 64, 16).forward(b).view(np.uint32))


@needs_ref
def test_bit_identical_to_the_reference_build_on_the_schedule():
    d = os.path.join(FIX, "chat-tiny")
    w = HostWeights.load(d)
    lens = [1, 17, 64, 200, 300]
    nb = blocks_needed(lens, 6)
    worst, agree, total = compare(O.RefBackend(d, nb, 16), O.CpuBackend(w, nb, 16), w.config.vocab, lens, 96, 6)
    assert worst == 0.0 and agree == total


def test_the_schedule_agrees_with_itself():
    """test_attention.cpp's the_comparison_schedule_runs_and_agrees_with_itself."""
    w = HostWeights.load(os.path.join(FIX, "chat-tiny"))
    lens = [1, 17, 64, 200, 700, 1300]
    nb = blocks_needed(lens, 12)
    worst, agree, total = compare(O.CpuBackend(w, nb, 16), O.CpuBackend(w, nb, 16), w.config.vocab, lens, 192, 12)
    assert worst == 0.0 and agree == total


def test_batched_equals_alone_bitwise():
    """relay's CPU contract (cpu_backend.cpp:1-6): a sequence's logits do not depend on
    what else is in the batch, or on the block size."""
    w = HostWeights.load(os.path.join(FIX, "llama-gqa-tied-bf16"))
    p1, p2 = list(range(1, 30)), list(range(40, 47))
    alone = O.CpuBackend(w, 16, 4).forward(ForwardBatch([SeqChunk(p1, 0, list(range(8)), True)]))
    both = O.CpuBackend(w, 16, 4).forward(ForwardBatch([SeqChunk(p2, 0, [8, 9], True),
                                                        SeqChunk(p1, 0, list(range(8)), True)]))
    other_bs = O.CpuBackend(w, 80, 1).forward(ForwardBatch([SeqChunk(p1, 0, list(range(40, 69)), True)]))
    assert np.array_equal(alone[0].view(np.uint32), both[1].view(np.uint32))
    assert np.array_equal(alone[0].view(np.uint32), other_bs[0].view(np.uint32))


def special_floats():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 18, dtype=np.uint64).astype(np.uint32)
    rnd = bits.view(np.float32)
    rnd = rnd[np.isfinite(rnd)]
    half = np.arange(0, 0x7C00, dtype=np.uint16)
    vals = bits_to_f32(half).astype(np.float64)
    ulp = np.diff(np.append(vals, 65536.0))
    mids = (vals + ulp / 2).astype(np.float32)  # every halfway point: ties to even
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e30, -1e30, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                     2.0 ** -26, 1e-45], np.float32)
    return np.concatenate([edge, rnd, mids, -mids])


def test_f32_to_f16_is_ieee_round_to_nearest_even():
    x = special_floats()
    assert np.array_equal(O.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


def test_round_f16_inplace_is_numpys_cast_round_trip():
    x = special_floats()
    y = O.round_f16_inplace(x.copy())
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(y), nan)
    assert np.array_equal(y[~nan].view(np.uint32), want[~nan].view(np.uint32))


@needs_ref
def test_f32_to_f16_equals_the_reference_build():
    import ctypes as C

    x = np.concatenate([special_floats(), np.array([np.nan], np.float32)])
    want = np.empty(x.size, np.uint16)
    O.ref_lib().ref_f32_to_f16(x.ctypes.data, want.ctypes.data, x.size)
    assert np.array_equal(O.f32_to_f16(x), want)


def test_f16_to_f32_is_exact():
    h = np.arange(0, 1 << 16, dtype=np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]  # finite values
    assert np.array_equal(O.f16_to_f32(h), h.view(np.float16).astype(np.float32))


def test_rope_inv_freq_closed_form():
    c = ModelConfig(hidden=64, intermediate=64, layers=1, heads=1, kv_heads=1, head_dim=128, vocab=8)
    got = O.rope_inv_freq(c).astype(np.float64)
    want = 10000.0 ** (-np.arange(0, 128, 2) / 128.0)
    assert np.abs(got / want - 1).max() < 4e-7


@needs_ref
@pytest.mark.parametrize("model", ["llama3-rope", "llama-mha"])
def test_rope_inv_freq_equals_the_reference_build(model):
    d = os.path.join(FIX, model)
    c = HostWeights.load(d).config
    assert np.array_equal(O.rope_inv_freq(c), O.RefBackend(d, 4, 16).rope_inv_freq(c.head_dim // 2))


@pytest.mark.parametrize("bs,heads,kvh,D", [(16, 8, 2, 64), (1, 4, 4, 16), (12, 6, 3, 128)])
def test_attention_against_double_precision(bs, heads, kvh, D):
    case = PagedCase([1, 70, 600], [1, 5, 3], heads, kvh, D, bs, seed=bs)
    args = (bits_to_f32(case.q), heads * D, case.kpool, case.vpool, case.meta, None, heads, kvh, D, bs, 1 / math.sqrt(D))
    a = O.paged_attention(*args)
    b = O.paged_attention(*args, f64=True)
    assert np.abs(a - b).max() <= 2e-6 * np.abs(b).max()


def test_attention_closed_forms():
    D, bs = 16, 4
    case = PagedCase([37], [1], 2, 1, D, bs, seed=1)
    # equal keys: uniform weights, output = mean of V over the 37 positions
    row0 = case.kpool[:D].copy()
    for b in range(case.num_blocks):
        for s in range(bs):
            case.kpool[(b * bs + s) * D:(b * bs + s + 1) * D] = row0
    v = bits_to_f32(case.vpool).reshape(-1, D)
    rows = [case.tables[p // bs] * bs + p % bs for p in range(37)]
    out = O.paged_attention(bits_to_f32(case.q), 2 * D, case.kpool, case.vpool, case.meta, None, 2, 1, D, bs, 0.25)
    assert np.allclose(out[0, :D], v[rows].mean(0), atol=1e-6)
    # one key far above the rest: output = its V row
    q = np.zeros((1, 2 * D), np.float32)
    q[0, 0] = 1.0
    k = np.zeros(case.kpool.size, np.float32)
    hot = rows[20]
    k[hot * D] = 200.0
    out = O.paged_attention(q, 2 * D, k, case.vpool, case.meta, None, 2, 1, D, bs, 1.0)
    assert np.allclose(out[0, :D], v[hot], atol=1e-6)


def test_quantizer_properties():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float32)
    w[7] = 0.0
    q, s = O.quantize_int8(w)
    assert s[7] == 1.0 and not q[7].any()
    live = np.arange(64) != 7
    mx = np.abs(w[live]).max(1)
    assert np.array_equal(s[live], (mx / np.float32(127.0)).astype(np.float32))
    assert (np.abs(q[live]).max(1) == 127).all()
    r = w[live] / s[live, None]
    assert (np.abs(r - q[live]) <= 0.5 + 1e-6).all()
    # ties go to the even integer
    t = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5]], np.float32)
    qt, st = O.quantize_int8(t)
    assert st[0] == 1.0 and qt[0].tolist() == [127, 0, 2, 2, 0, -2]


def test_gemv_oracle_is_exact_on_a_small_case():
    rng = np.random.default_rng(4)
    N, K, T = 5, 24, 3
    w8 = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.02, N).astype(np.float32)
    x = f16_bits(rng.standard_normal((T, K)).astype(np.float32))
    y = O.gemv_int8(w8, s, x)
    xf = bits_to_f32(x)
    for t in range(T):
        for n in range(N):
            exact = sum(Fraction(int(w8[n, k])) * Fraction(float(xf[t, k])) for k in range(K)) * Fraction(float(s[n]))
            assert abs(Fraction(y[t, n]) - exact) <= abs(exact) * Fraction(1, 2 ** 50) + Fraction(1, 2 ** 60)
    # all-ones weights sum the activations
    ones = np.ones((2, K), np.int8)
    y1 = O.gemv_int8(ones, np.ones(2, np.float32), x)
    assert np.allclose(y1[:, 0], xf.astype(np.float64).sum(1), rtol=1e-12)


GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("name", ["smollm2_135m", "tinyllama_2layer", "llama3_8b_2layer", "tinyllama_2layer_p2048"])
def test_oracle_equals_committed_goldens(name):
    """Goldens written by tests/golden/make_goldens.py from the reference build: the same
    greedy tokens and every logits row bit for bit (by SHA-256)."""
    import goldens

    path = os.path.join(GOLDEN, f"{name}.npz")
    g = np.load(path, allow_pickle=False)
    assert g["prompt"].tolist() == goldens.prompt_of(name)
    got = goldens.run_oracle(name, goldens.weights_for(name))
    assert got["tokens"].tolist() == g["tokens"].tolist()
    assert np.array_equal(goldens.row_sha(got["rows"]), g["row_sha256"])


@pytest.mark.parametrize("name", ["tinyllama_2layer_decode32", "llama3_8b_2layer_mixed"])
def test_oracle_equals_committed_step_goldens(name):
    """Step goldens (a 32-sequence decode step at context 2048; a mixed step of 48 decode
    sequences and a 512-token chunk), written from the reference build by
    tests/golden/make_goldens.py: every logits row bit for bit and the same greedy tokens."""
    import goldens

    g = np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False)
    got = goldens.run_step_oracle(name, goldens.weights_for(name))
    assert np.array_equal(got["tokens"], g["tokens"])
    assert np.array_equal(goldens.row_sha(got["rows"]), g["row_sha256"])
