"""fp16-weight skinny product (rh_gemv_f16) against a float64 reference.

y[t, n] = sum_k W16[n, k] x[t, k] (+ beta y). Products of two fp16 values are exact in
fp32, so the only error is fp32 accumulation over K terms; the bound used is
|y - y_exact| <= 4 K 2^-24 sum_k |W16[n, k] x[t, k]| (+ the fp32 rounding of the beta term).
The exact value is computed in float64 from the same fp16 values (numpy as the checker).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS32 = 2.0 ** -24


def run(torch, dev, w, x, beta=0.0, y0=None, ldw=None):
    from relay_amd import _lib

    N, K = w.shape
    T = x.shape[0]
    ldw = K if ldw is None else ldw
    padded = np.full((N, ldw), np.float16(7.0), np.float16)
    padded[:, :K] = w
    W = torch.from_numpy(padded.view(np.int16)).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    Y = torch.from_numpy(y0.copy()).to(dev) if y0 is not None else torch.full((T, N), float("nan"), device=dev)
    print(f"gemv_f16 case: T={T} K={K} N={N} ldw={ldw} beta={beta}", flush=True)
    _lib.check(_lib.lib().rh_gemv_f16(W.data_ptr(), ldw, X.data_ptr(), Y.data_ptr(), T, K, N, beta, None),
               "rh_gemv_f16")
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def make(N, K, T, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    x = rng.standard_normal((T, K)).astype(np.float16)
    return w, x


def check(y, w, x, beta=0.0, y0=None):
    wd, xd = w.astype(np.float64), x.astype(np.float64)
    exact = xd @ wd.T + (beta * y0.astype(np.float64) if beta else 0.0)
    bound = 4 * w.shape[1] * EPS32 * (np.abs(xd) @ np.abs(wd).T) + 2 * EPS32 * np.abs(exact) + 1e-30
    assert (np.abs(y - exact) <= bound).all()


@pytest.mark.parametrize("T", [1, 2, 5, 16, 17, 31, 32])
@pytest.mark.parametrize("N,K", [(960, 576), (576, 1536), (100, 48), (33, 16), (4096, 2048), (1000, 5632)])
def test_matches_float64(torch_mod, dev, T, N, K):
    w, x = make(N, K, T, seed=T * 7 + N + K)
    check(run(torch_mod, dev, w, x), w, x)


def test_beta_accumulates(torch_mod, dev):
    w, x = make(300, 512, 20, seed=1)
    y0 = np.random.default_rng(2).standard_normal((20, 300)).astype(np.float32)
    check(run(torch_mod, dev, w, x, beta=1.0, y0=y0), w, x, beta=1.0, y0=y0)


def test_row_stride_gives_the_same_bits(torch_mod, dev):
    w, x = make(200, 96, 9, seed=3)
    a = run(torch_mod, dev, w, x)
    b = run(torch_mod, dev, w, x, ldw=96 + 40)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rejects_bad_shapes(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_f16(None, 64, None, None, 33, 64, 64, 0.0, None) != 0 and "T must" in _lib.last_error()
    assert L.rh_gemv_f16(None, 72, None, None, 1, 72, 64, 0.0, None) != 0 and "K must" in _lib.last_error()
    assert L.rh_gemv_f16(None, 60, None, None, 1, 64, 64, 0.0, None) != 0 and "ldw" in _lib.last_error()
    assert L.rh_gemv_f16_max_tokens() == 32
