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

# q_out scale passed to the fused q writers and to rh_qkv_post alike (the backend passes the
# softmax scale times log2(e); any value must give the same bytes on both paths)
QS = 0.125 * 1.4426950408889634

pytestmark = pytest.mark.gpu

EPS32 = 2.0 ** -24


def vector_alu(T, N, K):
    """Whether a fused int8 launch and the plain launch of the chain it replaces may sum in
    different orders: the fused forms run the whole-line MFMA kernel at 1-16 tokens (the qkv
    form up to 32) with their own row groups and wave splits, while rh_gemv_int8 keeps its
    row-tile kernels above 16 tokens and on more than 6144 rows at 9-16."""
    return 1 <= T <= 32


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


@pytest.mark.parametrize("T", [1, 4, 8, 48])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_llama3_shapes(torch_mod, dev, N, K, T):
    """Llama-3-8B projection shapes at config 4's batch sizes 1, 4 and 8 (the whole-line
    kernel: 8 rows per workgroup at one token and on 4096 -> 1024; 16 rows at 4 and 8 tokens
    where K and N exceed 2048) and config 5's 48 decode tokens, fp16 scales, in the padded
    row layout the backend stores (rh_gemv_int8_row_stride)."""
    from relay_amd import _lib

    w8, s, x = make(N, K, T, seed=N + K + T)
    s16 = bits_to_f32(f16_bits(s))
    ldw = _lib.lib().rh_gemv_int8_row_stride(K)
    y = run(torch_mod, dev, w8, s, x, f16_scale=True, ldw=ldw)
    exact = O.gemv_int8(w8, s16, x)
    assert (np.abs(y - exact) <= bound(w8, s16, x)).all()


@pytest.mark.parametrize("N,K", [(2560, 2048), (11264, 2048), (32000, 2048), (2048, 5632), (28672, 4096),
                                 (9, 16), (17, 4112)])
@pytest.mark.parametrize("f16_scale", [False, True])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6, 7, 8])
def test_whole_line_kernels(torch_mod, dev, N, K, f16_scale, T):
    """T = 1-8 on the whole-line MFMA kernel (16 rows per workgroup at 4-8 tokens where K and
    N exceed 2048, else 8): TinyLlama's and Llama-3's projections and LM heads, a K that ends mid-step,
    a last workgroup with one row, with beta = 1 over a finite y."""
    from relay_amd import _lib

    w8, s, x = make(N, K, T, seed=N * 7 + K + T)
    s_used = bits_to_f32(f16_bits(s)) if f16_scale else s
    y0 = np.random.default_rng(N).standard_normal((T, N)).astype(np.float32)
    y = run(torch_mod, dev, w8, s, x, beta=1.0, y0=y0, f16_scale=f16_scale, ldw=_lib.lib().rh_gemv_int8_row_stride(K))
    exact = O.gemv_int8(w8, s_used, x, beta=1.0, y0=y0)
    assert (np.abs(y - exact) <= bound(w8, s_used, x) + 2 * EPS32 * np.abs(exact)).all()


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
    # rows are addressed with 32-bit offsets from the workgroup's first row
    assert _lib.lib().rh_gemv_int8(None, 1 << 21, None, 0, None, None, 1, 64, 64, 0.0, None) != 0
    assert "2^21" in _lib.last_error()


# Fused producers and the qkv epilogue on the int8 GEMV: the same bits as the launches they
# replace (rh_rmsnorm / rh_silu_mul, rh_gemv_int8, rh_qkv_post), whose parts are checked
# against their own references (test_layer_ops.py and the tests above), wherever the two use
# the same kernel and wave split of K (the MFMA tile: above two tokens, or two above 4096 rows;
# every shape with at most 256 16-row tiles, the backend's use); against the float64 oracle elsewhere.
def _fused_vs_chain(torch, dev, kind, T, K, N, beta, f16_scale, seed):
    from relay_amd import _lib

    L = _lib.lib()
    rng = np.random.default_rng(seed)
    w8 = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    scale = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    ldw = L.rh_gemv_int8_row_stride(K)
    padded = np.full((N, ldw), 0x7F, np.int8)
    padded[:, :K] = w8
    W = torch.from_numpy(padded).to(dev)
    S = torch.from_numpy(f16_bits(scale).view(np.int16) if f16_scale else scale).to(dev)
    y0 = rng.standard_normal((T, N)).astype(np.float32)
    want = torch.from_numpy(y0.copy()).to(dev)
    got = torch.from_numpy(y0.copy()).to(dev)
    xh = torch.empty((T, K), dtype=torch.int16, device=dev)
    print(f"gemv_int8 fused {kind}: T={T} K={K} N={N} beta={beta} f16_scale={f16_scale}", flush=True)
    if kind == "rmsnorm":
        x = torch.from_numpy((rng.standard_normal((T, K)) * 3).astype(np.float32)).to(dev)
        nw = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).to(dev)
        _lib.check(L.rh_rmsnorm(x.data_ptr(), None, T, nw.data_ptr(), K, 1e-5, xh.data_ptr(), None), "rh_rmsnorm")
        _lib.check(L.rh_gemv_int8_rmsnorm(W.data_ptr(), ldw, S.data_ptr(), int(f16_scale), x.data_ptr(), nw.data_ptr(),
                                          1e-5, got.data_ptr(), T, K, N, beta, None), "rh_gemv_int8_rmsnorm")
    else:
        gu = torch.from_numpy((rng.standard_normal((T, 2 * K)) * 2).astype(np.float32)).to(dev)
        _lib.check(L.rh_silu_mul(gu.data_ptr(), T, K, xh.data_ptr(), None), "rh_silu_mul")
        _lib.check(L.rh_gemv_int8_silu(W.data_ptr(), ldw, S.data_ptr(), int(f16_scale), gu.data_ptr(), got.data_ptr(),
                                       T, K, N, beta, None), "rh_gemv_int8_silu")
    _lib.check(L.rh_gemv_int8(W.data_ptr(), ldw, S.data_ptr(), int(f16_scale), xh.data_ptr(), want.data_ptr(), T, K, N,
                              beta, None), "rh_gemv_int8")
    torch.cuda.synchronize()
    s_used = bits_to_f32(f16_bits(scale)) if f16_scale else scale
    return want.cpu().numpy(), got.cpu().numpy(), (w8, s_used, xh.cpu().numpy().view(np.uint16), y0)


@pytest.mark.parametrize("kind", ["rmsnorm", "silu"])
@pytest.mark.parametrize("T,K,N,beta,f16_scale", [(1, 576, 960, 0.0, False), (16, 576, 3072, 0.0, True),
                                                  (7, 1536, 576, 1.0, False), (3, 4096, 512, 1.0, True),
                                                  (2, 14336, 256, 1.0, False), (5, 5632, 2048, 1.0, True),
                                                  (16, 2032, 4096, 0.0, False), (9, 48, 33, 0.0, False),
                                                  (4, 2048, 4104, 0.0, True)])
def test_fused_producers_match_the_chain(torch_mod, dev, kind, T, K, N, beta, f16_scale):
    want, got, (w8, s, xb, y0) = _fused_vs_chain(torch_mod, dev, kind, T, K, N, beta, f16_scale, seed=T + K + N)
    if not vector_alu(T, N, K):
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
    else:
        # the plain launch runs the 8-row whole-line kernel, the fused one the 16-row tile
        exact = O.gemv_int8(w8, s, xb, beta=beta, y0=y0)
        tol = bound(w8, s, xb) + 2 * EPS32 * np.abs(exact)
        assert (np.abs(got - exact) <= tol).all() and (np.abs(want - exact) <= tol).all()


@pytest.mark.parametrize("kind", ["rmsnorm", "silu"])
def test_fused_producers_on_wide_matrices(torch_mod, dev, kind):
    """6144 rows at T = 8: the plain launch takes two row tiles per workgroup (16 waves), the
    fused one 16-row workgroups (8 waves), so the sums differ in order: both within the
    fp32-accumulation bound of the float64 product of the same fp16 operands."""
    T, K, N = 8, 1024, 6144
    want, got, (w8, s, xb, y0) = _fused_vs_chain(torch_mod, dev, kind, T, K, N, 1.0, False, seed=7)
    exact = O.gemv_int8(w8, s, xb, beta=1.0, y0=y0)
    tol = bound(w8, s, xb) + 2 * EPS32 * np.abs(exact)
    assert (np.abs(got - exact) <= tol).all() and (np.abs(want - exact) <= tol).all()


def test_fused_limits(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_int8_silu(None, 2048, None, 0, None, None, 16, 2048, 64, 0.0, None) != 0
    assert L.rh_gemv_int8_rmsnorm(None, 64, None, 0, None, None, 1e-5, None, 17, 64, 64, 0.0, None) != 0


def f16_close(a_bits, b_bits, tol, name):
    """fp16 outputs (caches, q) of two fp32 values that differ by at most tol (their sums'
    order): within tol plus one fp16 rounding of either."""
    va = bits_to_f32(a_bits.view(np.uint16)).astype(np.float64)
    vb = bits_to_f32(b_bits.view(np.uint16)).astype(np.float64)
    lim = tol + 2.0 ** -10 * np.maximum(np.abs(va), np.abs(vb)) + 2.0 ** -24
    assert (np.abs(va - vb) <= lim).all(), name


@pytest.mark.parametrize("T,heads,kvh,D,H,bs,with_bias,norm", [
    (1, 9, 3, 64, 576, 16, False, True), (15, 32, 4, 64, 2048, 16, True, False), (5, 16, 8, 128, 4096, 16, False, True),
    (8, 8, 2, 64, 320, 12, True, True), (3, 4, 4, 16, 64, 1, True, True), (16, 32, 4, 64, 2048, 16, False, False),
    (2, 16, 4, 128, 2048, 16, False, False), (24, 32, 4, 64, 2048, 16, True, False),
    (32, 32, 4, 64, 2048, 16, False, False), (17, 8, 2, 128, 512, 16, True, False)])
def test_fused_qkv_matches_the_chain(torch_mod, dev, T, heads, kvh, D, H, bs, with_bias, norm):
    """rh_gemv_int8_rmsnorm_qkv (norm) or rh_gemv_int8_qkv (x already normalised) against
    rh_rmsnorm -> rh_gemv_int8 -> rh_qkv_post. Without rotation (inv_freq = 0) every byte of
    qkv, q and both caches is equal (where rh_gemv_int8 takes the MFMA tile; else the bounds below). With RoPE the inlined sincosf/products of the two kernels
    round differently in the last bit, so rotated fp32 values must agree within 4 ulp of the
    pair's magnitude and fp16 values within 1 ulp."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    rng = np.random.default_rng(T * 37 + D + H)
    N = (heads + 2 * kvh) * D
    pos = [int(p) for p in rng.permutation(5 * bs + 3)[:T]]  # distinct: one writer per cache slot
    seq = [t % 2 for t in range(T)]
    per = (5 * bs + 3) // bs + 1
    nblocks = 2 * per + 3
    tables = [int(b) for b in rng.permutation(nblocks)[:2 * per]]
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ldw = L.rh_gemv_int8_row_stride(H)
    w8 = np.full((N, ldw), 0x7F, np.int8)
    w8[:, :H] = rng.integers(-127, 128, size=(N, H), dtype=np.int8)
    W = dt(w8)
    S = dt(rng.uniform(0.001, 0.02, size=N).astype(np.float32))
    x = dt((rng.standard_normal((T, H)) * 2).astype(np.float32))
    nw = dt(rng.uniform(0.5, 1.5, H).astype(np.float32))
    bias = dt(rng.standard_normal(N).astype(np.float32)) if with_bias else None
    P, Sq = dt(np.array(pos, np.int32)), dt(np.array(seq, np.int32))
    TO, TB = dt(np.array([0, per], np.int32)), dt(np.array(tables, np.int32))
    bp = bias.data_ptr() if bias is not None else None

    def run_qkv(fused, inv):
        kc = torch.full((nblocks * kvh * bs * D,), 0x7BFF, dtype=torch.int16, device=dev)
        vc = kc.clone()
        qo = torch.zeros(T * heads * D, dtype=torch.int16, device=dev)
        qkv = torch.full((T, N), float("nan"), device=dev)
        xn = torch.empty((T, H), dtype=torch.int16, device=dev)
        _lib.check(L.rh_rmsnorm(x.data_ptr(), None, T, nw.data_ptr(), H, 1e-5, xn.data_ptr(), None), "rh_rmsnorm")
        rope = (bp, inv.data_ptr(), P.data_ptr(), Sq.data_ptr(), TO.data_ptr(), TB.data_ptr(), kc.data_ptr(),
                vc.data_ptr(), qo.data_ptr(), QS, heads, kvh, D, bs, None)
        if fused and not norm:
            _lib.check(L.rh_gemv_int8_qkv(W.data_ptr(), ldw, S.data_ptr(), 0, xn.data_ptr(), qkv.data_ptr(), T, H, *rope),
                       "rh_gemv_int8_qkv")
        elif fused:
            _lib.check(L.rh_gemv_int8_rmsnorm_qkv(W.data_ptr(), ldw, S.data_ptr(), 0, x.data_ptr(), nw.data_ptr(), 1e-5,
                                                  qkv.data_ptr(), T, H, *rope), "rh_gemv_int8_rmsnorm_qkv")
        else:
            _lib.check(L.rh_gemv_int8(W.data_ptr(), ldw, S.data_ptr(), 0, xn.data_ptr(), qkv.data_ptr(), T, H, N, 0.0,
                                      None), "rh_gemv_int8")
            _lib.check(L.rh_qkv_post(qkv.data_ptr(), T, *rope), "rh_qkv_post")
        torch.cuda.synchronize()
        return [a.cpu().numpy() for a in (qkv, kc, vc, qo, xn)]

    print(f"int8 fused qkv: T={T} heads={heads}/{kvh} D={D} H={H} bs={bs} bias={with_bias} norm={norm}", flush=True)
    assert (N + 15) // 16 <= 256 and (not norm or L.rh_gemv_f16_fused_fits(T, H))
    inv0 = dt(np.zeros(D // 2, np.float32))
    chain0, fused0 = run_qkv(False, inv0), run_qkv(True, inv0)
    # Where the chain's plain product runs on the 8-row whole-line kernel and the fused qkv
    # product on the 16-row tile, their sums differ in order, each within
    # the fp32-accumulation bound of the same fp16 operands (gemv bound below, carried through
    # the rotation).
    pairs = lambda v: np.broadcast_to(np.abs(v.reshape(T, -1, 2, D // 2)).sum(axis=2, keepdims=True),
                                      (T, N // D, 2, D // 2)).reshape(T, N)
    if vector_alu(T, N, H):
        gb = 2 * bound(w8[:, :H], S.cpu().numpy(), chain0[4].view(np.uint16))
        assert (np.abs(chain0[0] - fused0[0]) <= gb + 2 * EPS32 * np.abs(chain0[0])).all()
        for name, a, b in zip(("k cache", "v cache", "q"), chain0[1:4], fused0[1:4]):
            f16_close(a, b, gb.max(), name)
    else:
        gb = 0.0
        for name, a, b in zip(("qkv", "k cache", "v cache", "q"), chain0[:4], fused0[:4]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name
    inv = dt((1.0 / 10000.0 ** (np.arange(0, D, 2) / D)).astype(np.float32))
    (qa, ka, va, oa, _), (qb, kb, vb, ob, _) = run_qkv(False, inv), run_qkv(True, inv)
    bound_q = 4 * 2.0 ** -24 * pairs(qa) + (2 * pairs(gb) if vector_alu(T, N, H) else 0.0)
    assert (np.abs(qa - qb) <= bound_q).all()
    for name, a, b in (("k cache", ka, kb), ("v cache", va, vb), ("q", oa, ob)):
        if vector_alu(T, N, H):
            f16_close(a, b, 2 * gb.max(), name)
        else:
            diff = np.abs(a.astype(np.int32) - b.astype(np.int32))
            assert diff.max() <= 1 and (np.sign(a) == np.sign(b)).all(), name


@pytest.mark.parametrize("T,I,K,f16_scale", [(1, 5632, 2048, False), (3, 5632, 2048, True), (8, 5632, 2048, False),
                                             (1, 14336, 4096, False), (4, 14336, 4096, False),
                                             (5, 14336, 4096, True), (8, 14336, 4096, False), (6, 1536, 576, False),
                                             (2, 102, 160, False), (7, 250, 4096, True), (9, 5632, 2048, False),
                                             (16, 14336, 4096, True), (12, 1536, 576, False), (13, 250, 4096, False)])
def test_gate_up_silu_equals_the_chain(torch_mod, dev, T, I, K, f16_scale):
    """rh_gemv_int8_gate_up_silu gives the bytes of rh_gemv_int8 over the fused [gate; up]
    matrix followed by rh_silu_mul, at every row grouping rh_gemv_int8 takes at 1-8 tokens
    (8, 16 and 32 rows per workgroup) and for I not a multiple of 4; at 9-16 tokens (the
    whole-line kernel) within the chain's fp32 accumulation bound through SiLU·mul."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    w8, scale, x = make(2 * I, K, T, seed=T * 31 + I + K)
    gu = run(torch, dev, w8, scale, x, f16_scale=f16_scale)
    GU = torch.from_numpy(gu).to(dev)
    act_a = torch.empty((T, I), dtype=torch.int16, device=dev)
    _lib.check(L.rh_silu_mul(GU.data_ptr(), T, I, act_a.data_ptr(), None), "rh_silu_mul")
    W = torch.from_numpy(w8).to(dev)
    S = (torch.from_numpy(f16_bits(scale).view(np.int16)) if f16_scale else torch.from_numpy(scale)).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    act_b = torch.full((T, I), 0x7E00, dtype=torch.int16, device=dev)
    print(f"gate_up_silu case: T={T} I={I} K={K} f16_scale={f16_scale}", flush=True)
    _lib.check(L.rh_gemv_int8_gate_up_silu(W.data_ptr(), K, S.data_ptr(), int(f16_scale), X.data_ptr(),
                                           act_b.data_ptr(), T, K, I, None), "rh_gemv_int8_gate_up_silu")
    torch.cuda.synchronize()
    if T <= 8:
        assert np.array_equal(act_a.cpu().numpy(), act_b.cpu().numpy())
    else:
        s_used = bits_to_f32(f16_bits(scale)) if f16_scale else scale
        exact = O.gemv_int8(w8, s_used, x).astype(np.float64)
        err = bound(w8, s_used, x) + 2 * EPS32 * np.abs(exact)
        g, u, dg, du = exact[:, :I], exact[:, I:], err[:, :I], err[:, I:]
        silu = g / (1.0 + np.exp(-g))
        f16_close(act_a.cpu().numpy(), act_b.cpu().numpy(), 1.1 * np.abs(u) * dg + np.abs(silu) * du + dg * du, "act")


@pytest.mark.parametrize("T,I,K,f16_scale", [(1, 5632, 2048, False), (4, 5632, 2048, True), (8, 5632, 2048, False),
                                             (1, 14336, 4096, False), (7, 14336, 4096, True), (3, 1536, 576, False),
                                             (2, 102, 160, False), (5, 250, 4096, True), (8, 2048, 64, False)])
def test_rmsnorm_gate_up_silu_matches_the_chain(torch_mod, dev, T, I, K, f16_scale):
    """rh_gemv_int8_rmsnorm_gate_up_silu against rh_rmsnorm -> rh_gemv_int8_gate_up_silu: the
    same bytes where the fused launch has >= 256 workgroups (the same K split); below that,
    within the chain's fp32 accumulation bound carried through SiLU·mul plus one fp16
    rounding."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    rng = np.random.default_rng(T * 131 + I + K)
    w8, scale, _ = make(2 * I, K, T, seed=T * 31 + I + K + 1)
    W = torch.from_numpy(w8).to(dev)
    S = (torch.from_numpy(f16_bits(scale).view(np.int16)) if f16_scale else torch.from_numpy(scale)).to(dev)
    x = torch.from_numpy((rng.standard_normal((T, K)) * 3).astype(np.float32)).to(dev)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).to(dev)
    xn = torch.empty((T, K), dtype=torch.int16, device=dev)
    act_a = torch.empty((T, I), dtype=torch.int16, device=dev)
    act_b = torch.full((T, I), 0x7E00, dtype=torch.int16, device=dev)
    print(f"rmsnorm_gate_up_silu case: T={T} I={I} K={K} f16_scale={f16_scale}", flush=True)
    _lib.check(L.rh_rmsnorm(x.data_ptr(), None, T, nw.data_ptr(), K, 1e-5, xn.data_ptr(), None), "rh_rmsnorm")
    _lib.check(L.rh_gemv_int8_gate_up_silu(W.data_ptr(), K, S.data_ptr(), int(f16_scale), xn.data_ptr(),
                                           act_a.data_ptr(), T, K, I, None), "rh_gemv_int8_gate_up_silu")
    _lib.check(L.rh_gemv_int8_rmsnorm_gate_up_silu(W.data_ptr(), K, S.data_ptr(), int(f16_scale), x.data_ptr(),
                                                   nw.data_ptr(), 1e-5, act_b.data_ptr(), T, K, I, None),
               "rh_gemv_int8_rmsnorm_gate_up_silu")
    torch.cuda.synchronize()
    a, b = act_a.cpu().numpy(), act_b.cpu().numpy()
    if (I + 7) // 8 >= 256:
        assert np.array_equal(a, b)
    else:
        xb = xn.cpu().numpy().view(np.uint16)
        s_used = bits_to_f32(f16_bits(scale)) if f16_scale else scale
        exact = O.gemv_int8(w8, s_used, xb).astype(np.float64)
        err = bound(w8, s_used, xb) + 2 * EPS32 * np.abs(exact)
        g, u, dg, du = exact[:, :I], exact[:, I:], err[:, :I], err[:, I:]
        silu = g / (1.0 + np.exp(-g))
        f16_close(a, b, 1.1 * np.abs(u) * dg + np.abs(silu) * du + dg * du, "act")


def test_rmsnorm_gate_up_silu_limits(dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_int8_rmsnorm_gate_up_silu(None, 64, None, 0, None, None, 1e-5, None, 9, 64, 32, None) != 0
    assert "T must be in 1..8" in _lib.last_error()
    assert L.rh_gemv_int8_rmsnorm_gate_up_silu(None, 64, None, 0, None, None, 1e-5, None, 4, 64, 32, None) != 0
    assert "missing pointer" in _lib.last_error()


def test_gate_up_silu_limits(dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemv_int8_gate_up_silu(None, 64, None, 0, None, None, 17, 64, 32, None) != 0
    assert "T must be in 1..16" in _lib.last_error()
    assert L.rh_gemv_int8_gate_up_silu(None, 64, None, 0, None, None, 4, 64, 32, None) != 0
    assert "missing pointer" in _lib.last_error()
