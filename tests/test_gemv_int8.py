"""Weight-only int8 GEMV (rh_gemv_int8) against the double-precision oracle.

y[t, n] = scale[n] * sum_k W8[n, k] x[t, k] (+ beta y). Products of int8 and fp16 values
are exact in fp32, so the only error is fp32 accumulation over K terms: the bound used
is |y - y_exact| <= 4 K eps32 scale[n] sum_k |W8[n, k] x[t, k]| (+ the fp32 rounding of
the beta term), eps32 = 2^-24.
"""
import numpy as np
import pytest

import oracle as O
from helpers import bits_to_f32, f16_bits

pytestmark = pytest.mark.gpu

EPS32 = 2.0 ** -24


def run(torch, dev, w8, scale, x_bits, beta=0.0, y0=None, f16_scale=False, ldw=None):
    """ldw None: relay's dense rows; otherwise rows ldw bytes apart with junk in the padding."""
    from relay_amd import _lib

    N, K = w8.shape
    T = x_bits.shape[0]
    ldw = K if ldw is None else ldw
    padded = np.full((N, ldw), 0x7F, np.int8)
    padded[:, :K] = w8
    W = torch.from_numpy(padded).to(dev)
    if f16_scale:
        S = torch.from_numpy(f16_bits(scale).view(np.int16)).to(dev)
    else:
        S = torch.from_numpy(scale.astype(np.float32)).to(dev)
    X = torch.from_numpy(x_bits.view(np.int16)).to(dev)
    Y = torch.from_numpy(y0.copy()).to(dev) if y0 is not None else torch.full((T, N), float("nan"), device=dev)
    print(f"gemv case: T={T} K={K} N={N} ldw={ldw} beta={beta} f16_scale={f16_scale}", flush=True)
    rc = _lib.lib().rh_gemv_int8(W.data_ptr(), ldw, S.data_ptr(), int(f16_scale), X.data_ptr(), Y.data_ptr(), T, K,
                                 N, beta, None)
    _lib.check(rc, "rh_gemv_int8")
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def make(N, K, T, seed):
    rng = np.random.default_rng(seed)
    w8 = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    scale = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    x = f16_bits(rng.standard_normal((T, K), dtype=np.float32))
    return w8, scale, x


def bound(w8, scale, x_bits):
    ax = np.abs(bits_to_f32(x_bits)).astype(np.float64)
    mag = ax @ np.abs(w8.astype(np.float64)).T  # [T, N]
    K = w8.shape[1]
    return 4 * K * EPS32 * mag * scale[None, :].astype(np.float64) + 1e-30


@pytest.mark.parametrize("T", [1, 2, 3, 4, 7, 8, 9, 16, 17, 32, 33, 48, 64])
@pytest.mark.parametrize("N,K", [(64, 4096), (1000, 1024), (48, 80), (33, 160), (4096, 576), (6150, 256)])
def test_matches_oracle(torch_mod, dev, T, N, K):
    w8, s, x = make(N, K, T, seed=T * 1000 + N + K)
    y = run(torch_mod, dev, w8, s, x)
    exact = O.gemv_int8(w8, s, x)
    assert (np.abs(y - exact) <= bound(w8, s, x)).all()


@pytest.mark.parametrize("T", [1, 3, 4, 8, 9, 16])
@pytest.mark.parametrize("N", [4104, 4352, 11264, 14336, 28680, 57352])
def test_rows_split_evenly_over_the_cus(torch_mod, dev, T, N):
    """More row tiles than CUs: each workgroup takes an even share of rows (14, 24, 56 ...),
    so the last 16-row tile of a workgroup may be partly empty; every row must be computed
    once (y starts as NaN) and no row of a neighbour written."""
    K = 256
    w8, scale, x = make(N, K, T, seed=N + T)
    y0 = np.full((T, N), 0.5, np.float32)
    y = run(torch_mod, dev, w8, scale, x, beta=1.0, y0=y0)
    exact = O.gemv_int8(w8, scale, x, beta=1.0, y0=y0)
    assert np.isfinite(y).all()
    assert (np.abs(y - exact) <= bound(w8, scale, x) + 2 * EPS32 * np.abs(exact)).all()


def test_beta_accumulates(torch_mod, dev):
    w8, s, x = make(300, 512, 5, seed=1)
    y0 = np.random.default_rng(2).standard_normal((5, 300)).astype(np.float32)
    y = run(torch_mod, dev, w8, s, x, beta=1.0, y0=y0)
    exact = O.gemv_int8(w8, s, x, beta=1.0, y0=y0)
    assert (np.abs(y - exact) <= bound(w8, s, x) + 2 * EPS32 * np.abs(exact)).all()


def test_fp16_scales(torch_mod, dev):
    w8, s, x = make(512, 4096, 8, seed=3)
    s16 = bits_to_f32(f16_bits(s))
    y = run(torch_mod, dev, w8, s, x, f16_scale=True)
    exact = O.gemv_int8(w8, s16, x)
    assert (np.abs(y - exact) <= bound(w8, s16, x)).all()


@pytest.mark.parametrize("T", [8, 48])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_llama3_shapes(torch_mod, dev, N, K, T):
    """BASELINE config 4's projection shapes at T = 8 and at config 5's 48 decode tokens
    (fp16 scales), in the padded row layout the backend stores (rh_gemv_int8_row_stride)."""
    from relay_amd import _lib

    w8, s, x = make(N, K, T, seed=N + K + T)
    s16 = bits_to_f32(f16_bits(s))
    ldw = _lib.lib().rh_gemv_int8_row_stride(K)
    y = run(torch_mod, dev, w8, s, x, f16_scale=True, ldw=ldw)
    exact = O.gemv_int8(w8, s16, x)
    assert (np.abs(y - exact) <= bound(w8, s16, x)).all()


@pytest.mark.parametrize("ldw", [96, 160, 4096 + 256])
def test_row_stride_gives_the_same_bits(torch_mod, dev, ldw):
    """Rows ldw bytes apart (junk in the padding): bit-identical to the dense layout."""
    w8, s, x = make(300, 96, 4, seed=ldw)
    a = run(torch_mod, dev, w8, s, x)
    b = run(torch_mod, dev, w8, s, x, ldw=ldw)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rejects_bad_shapes(torch_mod, dev):
    from relay_amd import _lib

    assert _lib.lib().rh_gemv_int8(None, 64, None, 0, None, None, 65, 64, 64, 0.0, None) != 0
    assert _lib.lib().rh_gemv_int8(None, 72, None, 0, None, None, 1, 72, 64, 0.0, None) != 0
    assert _lib.lib().rh_gemv_int8(None, 48, None, 0, None, None, 1, 64, 64, 0.0, None) != 0
    assert "ldw" in _lib.last_error()
