"""Seeded random shapes for every kernel family, beyond the hand-picked cases of the other
test files: decode and prefill attention against the CPU oracle (2e-3 of max|ref|), the
int8 GEMV, the split-K fp16 product and the split-K int8 GEMM against their float64 bounds.
Each case prints its parameters first, so a failure names its shape."""
import numpy as np
import pytest

import oracle as O
import test_decode_attention as TD
import test_gemm_w8 as TW
import test_gemv_f16 as TF
import test_gemv_int8 as TG
import test_prefill as TP
from helpers import PagedCase

pytestmark = pytest.mark.gpu

COMBOS = [(8, 8), (9, 3), (32, 4), (32, 8), (16, 1), (40, 2), (64, 4), (12, 4), (48, 16)]


@pytest.mark.parametrize("seed", range(24))
def test_random_decode(torch_mod, dev, seed):
    rng = np.random.default_rng(1000 + seed)
    h, kv = COMBOS[rng.integers(len(COMBOS))]
    D = int(rng.choice([16, 32, 64, 128]))
    bs = int(rng.choice([1, 2, 4, 8, 12, 16, 32, 64]))
    ctxs = [int(c) for c in rng.integers(1, 3000, size=int(rng.integers(1, 24)))]
    from relay_amd import _lib

    chunk = _lib.lib().rh_decode_chunk_keys(D)
    sk = None if seed % 2 else chunk * int(rng.integers(1, 40))
    print(f"random decode {seed}: heads {h}/{kv} D {D} bs {bs} slice {sk} contexts {ctxs}", flush=True)
    case = PagedCase(ctxs, 1, h, kv, D, bs, seed=seed)
    got, _ = TD.run_decode(torch_mod, dev, case, slice_keys=sk)
    TD.check_close(got, TD.oracle_out(case))


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill(torch_mod, dev, seed):
    rng = np.random.default_rng(2000 + seed)
    h, kv = COMBOS[rng.integers(len(COMBOS))]
    D = int(rng.choice([16, 32, 64, 128]))
    bs = int(rng.choice([1, 4, 12, 16, 32]))
    ctxs = [int(c) for c in rng.integers(2, 700, size=int(rng.integers(1, 4)))]
    new = [int(rng.integers(1, c + 1)) for c in ctxs]
    print(f"random prefill {seed}: heads {h}/{kv} D {D} bs {bs} contexts {ctxs} new {new}", flush=True)
    case = PagedCase(ctxs, new, h, kv, D, bs, seed=seed)
    TP.check_close(TP.run_prefill(torch_mod, dev, case), TP.oracle_out(case))


@pytest.mark.parametrize("seed", range(16))
def test_random_products(torch_mod, dev, seed):
    rng = np.random.default_rng(3000 + seed)
    T, N, K = int(rng.integers(1, 65)), int(rng.integers(1, 3000)), 16 * int(rng.integers(1, 300))
    print(f"random int8 GEMV {seed}: T {T} N {N} K {K}", flush=True)
    w8, s, x = TG.make(N, K, T, seed=seed)
    assert (np.abs(TG.run(torch_mod, dev, w8, s, x) - O.gemv_int8(w8, s, x)) <= TG.bound(w8, s, x)).all()
    T, N, K = int(rng.integers(1, 33)), int(rng.integers(1, 3000)), 16 * int(rng.integers(1, 400))
    ks = int(rng.integers(1, min(8, (K + 63) // 64) + 1))
    print(f"random fp16 split product {seed}: T {T} N {N} K {K} ksplit {ks}", flush=True)
    w, x = TF.make(N, K, T, seed=seed)
    y, cnt = TF.run_split(torch_mod, dev, w, x, ks)
    TF.check(y, w, x)
    assert (cnt == 0).all()
    T, N, K = int(rng.integers(1, 65)), 4 * int(rng.integers(1, 1500)), 64 * int(rng.integers(1, 100))
    ks = int(rng.integers(1, min(8, K // (128 if K % 128 == 0 else 64)) + 1))
    print(f"random int8 split GEMM {seed}: T {T} N {N} K {K} ksplit {ks}", flush=True)
    q, sc, x = TW.make(N, K, T, seed=seed)
    TW.check(TW.run_skinny(torch_mod, dev, q, sc, x, ks), q, sc, x)


@pytest.mark.parametrize("seed", range(12))
def test_random_large_batch_int8(torch_mod, dev, seed):
    """The large-batch int8 GEMM (rh_gemm_w8 and its K split) over random T above the GEMV
    limit, N (any, or a multiple of 4 for a split) and K (a multiple of 64)."""
    rng = np.random.default_rng(4000 + seed)
    T, K = int(rng.integers(65, 700)), 64 * int(rng.integers(1, 80))
    ks = int(rng.integers(1, min(8, K // 64) + 1))
    N = int(rng.integers(1, 3000)) * (4 if ks > 1 else 1)
    print(f"random int8 large-batch GEMM {seed}: T {T} N {N} K {K} ksplit {ks}", flush=True)
    q, sc, x = TW.make(N, K, T, seed=seed)
    y = TW.run_split(torch_mod, dev, q, sc, x, ks) if ks > 1 else TW.run(torch_mod, dev, q, sc, x)
    TW.check(y, q, sc, x)
