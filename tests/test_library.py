"""The C-ABI library and the host-side logic, on the CPU (no compute calls on a GPU).

- librelay_hip.so loads and exports every function include/relay_hip.h declares;
- without a device the package refuses to run (there is no CPU fallback);
- config parsing matches relay's ModelConfig on the reference fixtures;
- the synthetic generator is deterministic and has the stated moments;
- relay's comparison schedule is self-consistent on the CPU oracle (its CPU-vs-CPU
  run agrees exactly, test_attention.cpp:169-175).
"""
import os
import re

import numpy as np
import pytest

from relay_amd import _lib
from relay_amd.model import HostWeights, ModelConfig, llama3_8b, read_safetensors

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "relay_hip.h")
FIX = os.path.join(REPO, "tests", "golden", "fixtures")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:rh|relay_hip)_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    for want in ("rh_paged_decode_attention", "rh_flash_prefill", "rh_gemv_int8", "rh_gemv_f16", "relay_hip_backend_forward",
                 "relay_hip_backend_read_kv_layer", "relay_hip_backend_update_weight"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert set(declared_functions()) == set(_lib.SIGNATURES), "the ctypes table and the header disagree"


def test_no_device_means_an_error_not_a_fallback():
    if _lib.lib().rh_device_available():
        pytest.skip("a GPU is present")
    with pytest.raises(_lib.RelayHipError):
        _lib.require_device()
    from relay_amd import HipBackend

    w = HostWeights.load(os.path.join(FIX, "llama-mha"))
    with pytest.raises(_lib.RelayHipError):
        HipBackend(w, 8, 16)


def test_kernel_launchers_validate_shapes_before_launching():
    lib = _lib.lib()
    assert lib.rh_gemv_int8(None, 64, None, 0, None, None, 0, 64, 64, 0.0, None) != 0
    assert lib.rh_gemv_int8_row_stride(4096) == 4096 + 256 and lib.rh_gemv_int8_row_stride(576) == 576
    assert lib.rh_gemv_int8_row_stride(14336) == 14336 + 256 and lib.rh_gemv_int8_row_stride(100) == 112
    assert "T must be" in _lib.last_error()
    assert lib.rh_flash_prefill(None, 64, None, None, None, None, 1, 4, 3, 64, 16, 0.1, None, 64, None) != 0
    assert lib.rh_prefill_tile_rows() == 128
    assert lib.rh_gemv_int8_max_tokens() == 64
    # a null weight pointer (an int8-only matrix passed to the fp16 product) is an error, not a launch
    assert lib.rh_gemv_f16_rmsnorm(None, 576, 16, 32, 1e-5, 48, 1, 576, 3072, 0.0, None) != 0
    assert "missing pointer" in _lib.last_error()
    assert lib.rh_gemv_int8(None, 576, 16, 0, 32, 48, 1, 576, 960, 0.0, None) != 0
    assert "missing pointer" in _lib.last_error()


def test_config_parsing_of_the_fixtures():
    c = ModelConfig.from_json_text(open(os.path.join(FIX, "llama3-rope", "config.json")).read())
    assert c.rope_llama3 and c.rope_factor > 1
    q = ModelConfig.from_json_text(open(os.path.join(FIX, "qwen2-bias", "config.json")).read())
    assert q.qkv_bias
    g = ModelConfig.from_json_text(open(os.path.join(FIX, "llama-gqa-tied-bf16", "config.json")).read())
    assert g.tie_embeddings and g.heads > g.kv_heads and g.head_dim == 8
    t = read_safetensors(os.path.join(FIX, "llama-gqa-tied-bf16", "model.safetensors"))
    assert all(a.dtype == np.float32 for a in t.values())


def test_synthetic_generator_is_deterministic_with_the_stated_moments():
    n = 1 << 20
    a, b = np.empty(n, np.float32), np.empty(n, np.float32)
    _lib.lib().rh_synth_normal_f32(a.ctypes.data, n, 0, 5, 0.0, 0.02)
    _lib.lib().rh_synth_normal_f32(b.ctypes.data, n, 0, 5, 0.0, 0.02)
    assert np.array_equal(a, b)
    c = np.empty(n, np.float32)
    _lib.lib().rh_synth_normal_f32(c.ctypes.data, n, 0, 6, 0.0, 0.02)
    assert not np.array_equal(a, c)
    assert abs(a.mean()) < 5 * 0.02 / np.sqrt(n) and abs(a.std() - 0.02) < 2e-4
    # the first elements do not depend on n (counter-based, any thread count)
    s = np.empty(1000, np.float32)
    _lib.lib().rh_synth_normal_f32(s.ctypes.data, 1000, 0, 5, 0.0, 0.02)
    assert np.array_equal(s, a[:1000])


def test_llama3_config_matches_the_stated_shape():
    c = llama3_8b()
    assert (c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim, c.intermediate, c.vocab) == \
        (4096, 32, 32, 8, 128, 14336, 128256)


@pytest.mark.parametrize("heads", [4, 32])
def test_prefill_plan_covers_every_row_once(heads):
    """rh_prefill_plan (host code): every row of every chunk in exactly one block of at
    most rh_prefill_tile_rows() rows, blocks inside their chunk with the chunk's positions
    and table, records heaviest first; a large step pairs light with heavy blocks."""
    rows = _lib.lib().rh_prefill_tile_rows()
    chunks = [(0, 2048, 0, 0), (2048, 300, 700, 130), (2348, 2, 5, 200), (2350, 129, 0, 210)]
    work = _lib.prefill_work(chunks, heads)
    seen, cost = [], []
    for rec in work:
        c = 0
        for t0, n, p0 in (rec[0:3], rec[3:6]):
            if n == 0:
                continue
            assert 0 < n <= rows
            ch = [x for x in chunks if x[0] <= t0 < x[0] + x[1]]
            assert len(ch) == 1 and t0 + n <= ch[0][0] + ch[0][1] and rec[6] == ch[0][3]
            assert p0 == ch[0][2] + (t0 - ch[0][0])
            seen.extend(range(t0, t0 + n))
            c += int(n) * int(p0 + n)
        cost.append(c)
    assert sorted(seen) == list(range(2479))
    assert cost == sorted(cost, reverse=True)
    paired = sum(1 for rec in work if rec[4] > 0)
    assert (paired > 0) == (heads == 32)


def test_prefill_plan_rejects_small_capacity():
    import numpy as np

    a = np.array([0], np.int32)
    n = np.array([1000], np.int32)
    work = np.zeros((1, 8), np.int32)
    assert _lib.lib().rh_prefill_plan(a.ctypes.data, n.ctypes.data, a.ctypes.data, a.ctypes.data, 1, 4,
                                      work.ctypes.data, 1) < 0
    assert "capacity" in _lib.last_error()


def test_work_planners_follow_their_rules():
    """The host-side planners (no device needed): rh_decode_slice_keys cuts contexts into
    whole chunks, kMergeBatch (8) slices of 2 to 8 chunks for few groups at head sizes 64 and
    128, one slice for a handful of
    short contexts, at least two otherwise, never below 8 chunks; rh_gemv_f16_split_plan splits K in two only for long K on few row tiles above 16 tokens;
    rh_gemv_int8_row_stride pads rows that are a multiple of 2 KB."""
    L = _lib.lib()
    for D in (16, 32, 64, 128):
        chunk = L.rh_decode_chunk_keys(D)
        assert chunk == {16: 128, 32: 128, 64: 64, 128: 32}[D]
        for n, kvh, g, ctx in [(32, 4, 8, 2048), (48, 8, 4, 8192), (1, 3, 3, 640), (1, 8, 4, 65536), (200, 8, 4, 100)]:
            sk = L.rh_decode_slice_keys(n, kvh, g, D, ctx)
            assert sk > 0 and sk % chunk == 0
            groups = n * kvh * ((g + 15) // 16)
            small = max(2 * chunk, -(-ctx // (8 * chunk)) * chunk)
            if D in (64, 128) and small <= 8 * chunk and groups * -(-ctx // small) <= 256:
                assert sk == small and -(-ctx // sk) <= 8  # few groups: short slices, one merge round
            elif groups <= 16 and ctx <= 16 * chunk:
                assert sk >= ctx  # one slice
            else:
                assert sk >= 8 * chunk and (ctx + sk - 1) // sk >= min(2, (ctx + 8 * chunk - 1) // (8 * chunk))
    assert L.rh_decode_slice_keys(32, 4, 8, 64, 2048) == 1024  # config 2: two slices of 1024 keys
    assert L.rh_decode_slice_keys(1, 3, 3, 64, 640) == 128  # config 1: five slices of 2 chunks
    assert L.rh_decode_slice_keys(1, 8, 4, 128, 2048) == 256  # 8 slices of 8 chunks at D128
    assert L.rh_decode_chunk_keys(96) == -1
    assert [L.rh_gemv_f16_split_plan(T, K, N) for T, K, N in
            [(32, 5632, 2048), (1, 5632, 2048), (32, 2048, 2048), (32, 4096, 4096), (8, 14336, 4096), (1, 4096, 1024)]] \
        == [2, 1, 1, 1, 1, 1]
    assert L.rh_gemv_f16_split_plan(0, 64, 64) == -1
    assert [L.rh_gemv_int8_row_stride(K) for K in (4096, 14336, 2048, 576, 100)] == [4352, 14592, 2304, 576, 112]
