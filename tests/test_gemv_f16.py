"""fp16-weight skinny product (rh_gemv_f16) against a float64 reference.

y[t, n] = sum_k W16[n, k] x[t, k] (+ beta y). Products of two fp16 values are exact in
fp32, so the only error is fp32 accumulation over K terms; the bound used is
|y - y_exact| <= 4 K 2^-24 sum_k |W16[n, k] x[t, k]| (+ the fp32 rounding of the beta term).
The exact value is computed in float64 from the same fp16 values (numpy as the checker).
"""
import numpy as np
import pytest

# q_out scale passed to the fused q writers and to rh_qkv_post alike (the backend passes the
# softmax scale times log2(e); any value must give the same bytes on both paths)
QS = 0.125 * 1.4426950408889634

pytestmark = pytest.mark.gpu

EPS32 = 2.0 ** -24


def whole_line(T, N, K):
    """Whether rh_gemv_f16 takes a whole-line kernel (the vector-ALU one at one token from 2 Mi
    weights, the 8-row MFMA one at 1-8 tokens otherwise, the fused kernel's at 9-32) instead
    of the 16-row MFMA tile (which only the K split runs now)."""
    return 1 <= T <= 32


def fused_differs(T, N, K):
    """Whether a fused launch (producer or qkv epilogue) and the plain launch of the chain it
    replaces may sum in different orders: both run whole-line kernels, whose row groups and
    wave splits can differ."""
    return whole_line(T, N, K)


def gemv_bound(w_f16, x_f16):
    """fp32-accumulation bound of x w^T for fp16 operands (rows of x against rows of w)."""
    wd, xd = w_f16.astype(np.float64), x_f16.astype(np.float64)
    return 4 * w_f16.shape[1] * EPS32 * (np.abs(xd) @ np.abs(wd).T) + 1e-30


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


@pytest.mark.parametrize("N,K,ldw", [(49152, 576, 576), (11264, 2048, 2048 + 8), (3641, 1040, 1040), (2048, 1024, 1032),
                                     (513, 4096, 4096)])
def test_one_token_kernel(torch_mod, dev, N, K, ldw):
    """One token from 2 Mi weights up takes the vector-ALU kernel (4 waves at K <= 1024, else 8;
    SmolLM2's and TinyLlama's heads and gate_up, a row count not a multiple of 8, padded rows),
    with beta = 1 over a finite y."""
    w, x = make(N, K, 1, seed=N + K)
    y0 = np.random.default_rng(K).standard_normal((1, N)).astype(np.float32)
    check(run(torch_mod, dev, w, x, beta=1.0, y0=y0, ldw=ldw), w, x, beta=1.0, y0=y0)


@pytest.mark.parametrize("N,K,T,ldw", [(11264, 2048, 8, 2048), (576, 1536, 3, 1544), (2048, 5632, 2, 5632),
                                       (13, 4112, 7, 4120), (576, 576, 1, 584), (960, 576, 1, 576), (21, 1000 * 16, 1, 16008)])
def test_few_token_kernel(torch_mod, dev, N, K, T, ldw):
    """1-8 tokens (one token below 2 Mi weights) on the 8-row whole-line MFMA kernel (8 waves;
    4 below 256 workgroups), padded rows, a K that ends mid-step, a last workgroup with five
    rows, beta = 1 over a finite y."""
    w, x = make(N, K, T, seed=N + K + T)
    y0 = np.random.default_rng(K).standard_normal((T, N)).astype(np.float32)
    check(run(torch_mod, dev, w, x, beta=1.0, y0=y0, ldw=ldw), w, x, beta=1.0, y0=y0)


def test_row_stride_gives_the_same_bits(torch_mod, dev):
    w, x = make(200, 96, 9, seed=3)
    a = run(torch_mod, dev, w, x)
    b = run(torch_mod, dev, w, x, ldw=96 + 40)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_split(torch, dev, w, x, ks, beta=0.0, y0=None, ws=None, counters=None):
    """rh_gemv_f16_splitk; returns y and the counters after the call."""
    from relay_amd import _lib

    N, K = w.shape
    T = x.shape[0]
    W = torch.from_numpy(np.ascontiguousarray(w).view(np.int16)).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    Y = torch.from_numpy(y0.copy()).to(dev) if y0 is not None else torch.full((T, N), float("nan"), device=dev)
    ws = torch.full((ks * T * N,), float("nan"), device=dev) if ws is None else ws
    counters = torch.zeros((N + 15) // 16, dtype=torch.int32, device=dev) if counters is None else counters
    print(f"gemv_f16_splitk case: T={T} K={K} N={N} ksplit={ks} beta={beta}", flush=True)
    _lib.check(_lib.lib().rh_gemv_f16_splitk(W.data_ptr(), K, X.data_ptr(), Y.data_ptr(), T, K, N, beta, ks,
                                             ws.data_ptr(), counters.data_ptr(), None), "rh_gemv_f16_splitk")
    torch.cuda.synchronize()
    return Y.cpu().numpy(), counters.cpu().numpy()


@pytest.mark.parametrize("ks", [1, 2, 3, 8])
@pytest.mark.parametrize("T,N,K", [(1, 2048, 5632), (32, 2048, 5632), (17, 100, 1024), (5, 33, 512)])
def test_split_k_matches_float64(torch_mod, dev, T, N, K, ks):
    """Any K split stays within the fp32 accumulation bound; ksplit 1 is rh_gemv_f16 bit for
    bit; the counters are back at zero after the call."""
    w, x = make(N, K, T, seed=T + N + K + ks)
    y, cnt = run_split(torch_mod, dev, w, x, ks)
    check(y, w, x)
    assert (cnt == 0).all()
    if ks == 1:
        assert np.array_equal(y.view(np.uint32), run(torch_mod, dev, w, x).view(np.uint32))


def test_split_k_repeats_and_accumulates(torch_mod, dev):
    """The same workspace and counters over calls of different shapes: every call merges its
    own partials (same bits on a repeat), and beta != 0 adds the old y once."""
    ws = torch_mod.full((4 * 32 * 2048,), float("nan"), device=dev)
    counters = torch_mod.zeros(128, dtype=torch_mod.int32, device=dev)
    w, x = make(2048, 4096, 32, seed=11)
    a, _ = run_split(torch_mod, dev, w, x, 4, ws=ws, counters=counters)
    w2, x2 = make(1000, 1024, 3, seed=12)
    y0 = np.random.default_rng(3).standard_normal((3, 1000)).astype(np.float32)
    c, cnt = run_split(torch_mod, dev, w2, x2, 2, beta=1.0, y0=y0, ws=ws, counters=counters)
    check(c, w2, x2, beta=1.0, y0=y0)
    b, cnt = run_split(torch_mod, dev, w, x, 4, ws=ws, counters=counters)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)) and (cnt == 0).all()


def test_split_plan_and_limits(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_f16_split_plan(32, 5632, 2048) == 2
    assert L.rh_gemv_f16_split_plan(32, 2048, 2048) == 1
    assert L.rh_gemv_f16_split_plan(1, 4096, 14336) == 1
    assert L.rh_gemv_f16_splitk(None, 64, None, None, 1, 64, 64, 0.0, 9, None, None, None) != 0
    assert "ksplit must be in 1..8" in _lib.last_error()
    assert L.rh_gemv_f16_splitk(None, 128, None, None, 1, 128, 64, 0.0, 3, None, None, None) != 0
    assert "more K ranges" in _lib.last_error()
    assert L.rh_gemv_f16_splitk(None, 128, None, None, 1, 128, 64, 0.0, 2, None, None, None) != 0
    assert "workspace" in _lib.last_error()


def test_rejects_bad_shapes(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_f16(None, 64, None, None, 33, 64, 64, 0.0, None) != 0 and "T must" in _lib.last_error()
    assert L.rh_gemv_f16(None, 72, None, None, 1, 72, 64, 0.0, None) != 0 and "K must" in _lib.last_error()
    assert L.rh_gemv_f16(None, 60, None, None, 1, 64, 64, 0.0, None) != 0 and "ldw" in _lib.last_error()
    assert L.rh_gemv_f16_max_tokens() == 32


# Fused producers: rh_gemv_f16_rmsnorm / rh_gemv_f16_silu must give the same bits as the
# two-launch chain they replace (rh_rmsnorm or rh_silu_mul, then rh_gemv_f16), whose parts
# are checked against their own references (test_layer_ops.py and the tests above), where
# both take the 16-row tile; within the fp32 bound where they take different kernels.
def _chain_and_fused(torch, dev, kind, T, K, N, beta, seed):
    from relay_amd import _lib

    L = _lib.lib()
    rng = np.random.default_rng(seed)
    w16 = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    W = torch.from_numpy(w16.view(np.int16)).to(dev)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    want = torch.from_numpy(y0.copy()).to(dev)
    got = torch.from_numpy(y0.copy()).to(dev)
    xh = torch.empty((T, K), dtype=torch.int16, device=dev)
    print(f"gemv_f16 fused {kind}: T={T} K={K} N={N} beta={beta}", flush=True)
    if kind == "rmsnorm":
        x = torch.from_numpy((rng.standard_normal((T, K)) * 3).astype(np.float32)).to(dev)
        nw = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).to(dev)
        _lib.check(L.rh_rmsnorm(x.data_ptr(), None, T, nw.data_ptr(), K, 1e-5, xh.data_ptr(), None), "rh_rmsnorm")
        _lib.check(L.rh_gemv_f16_rmsnorm(W.data_ptr(), K, x.data_ptr(), nw.data_ptr(), 1e-5, got.data_ptr(), T, K, N,
                                         beta, None), "rh_gemv_f16_rmsnorm")
    else:
        gu = torch.from_numpy((rng.standard_normal((T, 2 * K)) * 2).astype(np.float32)).to(dev)
        _lib.check(L.rh_silu_mul(gu.data_ptr(), T, K, xh.data_ptr(), None), "rh_silu_mul")
        _lib.check(L.rh_gemv_f16_silu(W.data_ptr(), K, gu.data_ptr(), got.data_ptr(), T, K, N, beta, None),
                   "rh_gemv_f16_silu")
    _lib.check(L.rh_gemv_f16(W.data_ptr(), K, xh.data_ptr(), want.data_ptr(), T, K, N, beta, None), "rh_gemv_f16")
    torch.cuda.synchronize()
    return want.cpu().numpy(), got.cpu().numpy(), w16, xh.cpu().numpy().view(np.float16)


@pytest.mark.parametrize("kind", ["rmsnorm", "silu"])
@pytest.mark.parametrize("T,K,N,beta", [(1, 576, 960, 0.0), (16, 576, 3072, 0.0), (7, 1536, 576, 1.0),
                                        (32, 960, 100, 0.0), (3, 4096, 512, 1.0), (2, 14336, 256, 1.0), (5, 5632, 2048, 1.0),
                                        (16, 2032, 6144, 0.0),
                                        (17, 48, 33, 0.0)])
def test_fused_producers_match_the_chain(torch_mod, dev, kind, T, K, N, beta):
    from relay_amd import _lib

    assert _lib.lib().rh_gemv_f16_fused_fits(T, K)
    want, got, w16, xh = _chain_and_fused(torch_mod, dev, kind, T, K, N, beta, seed=T + K + N)
    if fused_differs(T, N, K):  # the two launches sum in different orders
        assert (np.abs(want - got) <= 2 * gemv_bound(w16, xh) + 4 * EPS32 * np.abs(want)).all()
    else:
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32))


def test_fused_limits(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_f16_fused_fits(16, 2040) and not L.rh_gemv_f16_fused_fits(16, 2048)
    assert L.rh_gemv_f16_fused_fits(2, 14336) and not L.rh_gemv_f16_fused_fits(33, 16)
    assert L.rh_gemv_f16_silu(None, 2048, None, None, 16, 2048, 64, 0.0, None) != 0
    assert "LDS" in _lib.last_error()


@pytest.mark.parametrize("T,heads,kvh,D,H,bs,with_bias,norm", [
    (1, 9, 3, 64, 576, 16, False, True), (15, 32, 4, 64, 2048, 16, True, True), (5, 32, 8, 128, 4096, 16, False, True),
    (20, 8, 2, 64, 320, 12, True, True), (3, 4, 4, 16, 64, 1, True, True),
    (32, 32, 4, 64, 2048, 16, False, False), (17, 9, 3, 64, 576, 16, True, False), (2, 32, 8, 128, 4096, 16, False, False)])
def test_fused_qkv_matches_the_chain(torch_mod, dev, T, heads, kvh, D, H, bs, with_bias, norm):
    """rh_gemv_f16_rmsnorm_qkv (norm) or rh_gemv_f16_qkv (x already normalised) against
    rh_rmsnorm -> rh_gemv_f16 -> rh_qkv_post.
    Without rotation (inv_freq = 0) every byte of qkv, q and both caches is equal where both
    launches take the 16-row tile (same sums, same placement); else the bounds below. With RoPE the two kernels' inlined sincosf/products round differently in
    the last bit (measured: ~20% of rotated values 1 ulp apart), so rotated fp32 values must
    agree within 4 ulp of the pair's magnitude and fp16 values within 1 ulp."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    rng = np.random.default_rng(T * 31 + D + H)
    N = (heads + 2 * kvh) * D
    assert not norm or L.rh_gemv_f16_fused_fits(T, H)
    pos = [int(p) for p in rng.permutation(5 * bs + 3)[:T]]  # distinct: one writer per cache slot
    seq = [t % 2 for t in range(T)]
    per = (5 * bs + 3) // bs + 1
    nblocks = 2 * per + 3
    tables = [int(b) for b in rng.permutation(nblocks)[:2 * per]]
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    w16 = (rng.standard_normal((N, H)) * 0.05).astype(np.float16)
    W = dt(w16.view(np.int16))
    x = dt((rng.standard_normal((T, H)) * 2).astype(np.float32))
    nw = dt(rng.uniform(0.5, 1.5, H).astype(np.float32))
    bias = dt(rng.standard_normal(N).astype(np.float32)) if with_bias else None
    P, S = dt(np.array(pos, np.int32)), dt(np.array(seq, np.int32))
    TO, TB = dt(np.array([0, per], np.int32)), dt(np.array(tables, np.int32))
    bp = bias.data_ptr() if bias is not None else None

    def run(fused, inv):
        kc = torch.full((nblocks * kvh * bs * D,), 0x7BFF, dtype=torch.int16, device=dev)
        vc = kc.clone()
        qo = torch.zeros(T * heads * D, dtype=torch.int16, device=dev)
        qkv = torch.full((T, N), float("nan"), device=dev)
        xn = torch.empty((T, H), dtype=torch.int16, device=dev)
        _lib.check(L.rh_rmsnorm(x.data_ptr(), None, T, nw.data_ptr(), H, 1e-5, xn.data_ptr(), None), "rh_rmsnorm")
        if fused and not norm:
            _lib.check(L.rh_gemv_f16_qkv(W.data_ptr(), H, xn.data_ptr(), qkv.data_ptr(), T, H, bp, inv.data_ptr(),
                                         P.data_ptr(), S.data_ptr(), TO.data_ptr(), TB.data_ptr(), kc.data_ptr(),
                                         vc.data_ptr(), qo.data_ptr(), QS, heads, kvh, D, bs, None), "rh_gemv_f16_qkv")
        elif fused:
            _lib.check(L.rh_gemv_f16_rmsnorm_qkv(W.data_ptr(), H, x.data_ptr(), nw.data_ptr(), 1e-5, qkv.data_ptr(), T, H,
                                                 bp, inv.data_ptr(), P.data_ptr(), S.data_ptr(), TO.data_ptr(),
                                                 TB.data_ptr(), kc.data_ptr(), vc.data_ptr(), qo.data_ptr(), QS, heads,
                                                 kvh, D, bs, None), "rh_gemv_f16_rmsnorm_qkv")
        else:
            _lib.check(L.rh_gemv_f16(W.data_ptr(), H, xn.data_ptr(), qkv.data_ptr(), T, H, N, 0.0, None), "rh_gemv_f16")
            _lib.check(L.rh_qkv_post(qkv.data_ptr(), T, bp, inv.data_ptr(), P.data_ptr(), S.data_ptr(), TO.data_ptr(),
                                     TB.data_ptr(), kc.data_ptr(), vc.data_ptr(), qo.data_ptr(), QS, heads, kvh, D,
                                     bs, None), "rh_qkv_post")
        torch.cuda.synchronize()
        return [a.cpu().numpy() for a in (qkv, kc, vc, qo, xn)]

    print(f"fused qkv: T={T} heads={heads}/{kvh} D={D} H={H} bs={bs} bias={with_bias} norm={norm}", flush=True)
    inv0 = dt(np.zeros(D // 2, np.float32))
    chain0, fused0 = run(False, inv0), run(True, inv0)
    # Where the chain's plain launch takes a whole-line kernel the two sum in different orders:
    # fp32 values within twice the accumulation bound, fp16 ones within that plus one rounding.
    loose = fused_differs(T, N, H)
    gb = 2 * gemv_bound(w16, chain0[4].view(np.float16)) if loose else np.zeros((T, N))
    if loose:
        assert (np.abs(chain0[0] - fused0[0]) <= gb + 2 * EPS32 * np.abs(chain0[0])).all()
        for name, a, b in zip(("k cache", "v cache", "q"), chain0[1:4], fused0[1:4]):
            f16_close(a, b, gb.max(), name)
    else:
        for name, a, b in zip(("qkv", "k cache", "v cache", "q"), chain0[:4], fused0[:4]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name
    inv = dt((1.0 / 10000.0 ** (np.arange(0, D, 2) / D)).astype(np.float32))
    (qa, ka, va, oa, _), (qb, kb, vb, ob, _) = run(False, inv), run(True, inv)
    # fp32: the magnitude of a rotated value is bounded by |a| + |b| of its pair
    pairs = lambda v: np.broadcast_to(np.abs(v.reshape(T, -1, 2, D // 2)).sum(axis=2, keepdims=True),
                                      (T, N // D, 2, D // 2)).reshape(T, N)
    bound = 4 * 2.0 ** -24 * pairs(qa) + 2 * pairs(gb)
    assert (np.abs(qa - qb) <= bound).all()
    for name, a, b in (("k cache", ka, kb), ("v cache", va, vb), ("q", oa, ob)):
        if loose:
            f16_close(a, b, 2 * gb.max(), name)
        else:
            diff = np.abs(a.astype(np.int32) - b.astype(np.int32))
            assert diff.max() <= 1 and (np.sign(a) == np.sign(b)).all(), name


def f16_close(a_bits, b_bits, tol, name):
    """fp16 outputs of two fp32 values at most tol apart: within tol plus one fp16 rounding."""
    va = a_bits.view(np.float16).astype(np.float64)
    vb = b_bits.view(np.float16).astype(np.float64)
    lim = tol + 2.0 ** -10 * np.maximum(np.abs(va), np.abs(vb)) + 2.0 ** -24
    assert (np.abs(va - vb) <= lim).all(), name


@pytest.mark.parametrize("T,I,K", [(1, 5632, 2048), (4, 1536, 576), (8, 5632, 2048), (12, 1536, 576), (16, 5632, 2048),
                                   (24, 1536, 576), (32, 1536, 576), (3, 102, 160), (17, 250, 1024)])
def test_gate_up_silu_matches_the_chain(torch_mod, dev, T, I, K):
    """rh_gemv_f16_gate_up_silu (the whole-line kernel with SiLU·mul in its epilogue, gate and
    up rows of each output in one workgroup) against rh_gemv_f16 over the fused [gate; up]
    matrix + rh_silu_mul: within the fp32 accumulation bound of g and u carried through
    SiLU·mul plus one fp16 rounding; I not a multiple of 8 included."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    rng = np.random.default_rng(T * 17 + I + K)
    w16 = (rng.standard_normal((2 * I, K)) * 0.05).astype(np.float16)
    x = (rng.standard_normal((T, K)) * 2).astype(np.float16)
    W = torch.from_numpy(w16.view(np.int16)).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    gu = torch.empty((T, 2 * I), device=dev)
    act_a = torch.empty((T, I), dtype=torch.int16, device=dev)
    act_b = torch.full((T, I), 0x7E00, dtype=torch.int16, device=dev)
    print(f"gemv_f16_gate_up_silu: T={T} I={I} K={K}", flush=True)
    _lib.check(L.rh_gemv_f16(W.data_ptr(), K, X.data_ptr(), gu.data_ptr(), T, K, 2 * I, 0.0, None), "rh_gemv_f16")
    _lib.check(L.rh_silu_mul(gu.data_ptr(), T, I, act_a.data_ptr(), None), "rh_silu_mul")
    _lib.check(L.rh_gemv_f16_gate_up_silu(W.data_ptr(), K, X.data_ptr(), act_b.data_ptr(), T, K, I, None),
               "rh_gemv_f16_gate_up_silu")
    torch.cuda.synchronize()
    exact = x.astype(np.float64) @ w16.astype(np.float64).T
    err = gemv_bound(w16, x) + 2 * EPS32 * np.abs(exact)
    g, u, dg, du = exact[:, :I], exact[:, I:], err[:, :I], err[:, I:]
    silu = g / (1.0 + np.exp(-g))
    f16_close(act_a.cpu().numpy(), act_b.cpu().numpy(), 2 * (1.1 * np.abs(u) * dg + np.abs(silu) * du + dg * du), "act")
    want = (silu * u).astype(np.float64)
    got = act_b.cpu().numpy().view(np.float16).astype(np.float64)
    assert (np.abs(got - want) <= 1.1 * np.abs(u) * dg + np.abs(silu) * du + dg * du
            + 2.0 ** -10 * np.abs(want) + 2.0 ** -24).all()


def test_gate_up_silu_limits(dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_f16_gate_up_silu(None, 64, None, None, 33, 64, 32, None) != 0
    assert "T must be in 1..32" in _lib.last_error()
    assert L.rh_gemv_f16_gate_up_silu(None, 64, None, None, 4, 64, 32, None) != 0
    assert "missing pointer" in _lib.last_error()
