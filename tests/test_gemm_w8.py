"""Weight-only int8 GEMM (rh_gemm_w8) against a float64 reference.

y[t, n] = scale[n] * sum_k q[n, k] x[t, k] (+ beta y). The products q * x are exact in fp32,
so the error is the fp32 accumulation over K terms plus the rounding of the scale multiply
(and of the beta term): |y - y_exact| <= (4 K 2^-24 + 2^-23) |scale[n]| sum_k |q x| (+ 2^-23
|beta y|). The exact value is computed in float64 from the same int8/fp16 values (numpy as
the checker). Sizes cover partial token and row tiles, T above and below the GEMV limit, and
the shapes of the Llama-3-8B mixed batch (T = 560), and the K-split form (rh_gemm_w8_split).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS32 = 2.0 ** -24


def make(N, K, T, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    scale = (rng.uniform(0.5, 2.0, N) * 1e-3).astype(np.float32)
    x = rng.standard_normal((T, K)).astype(np.float16)
    return q, scale, x


def run(torch, dev, q, scale, x, beta=0.0, y0=None, ldw=None):
    from relay_amd import _lib

    N, K = q.shape
    T = x.shape[0]
    ldw = K if ldw is None else ldw
    padded = np.full((N, ldw), 99, np.int8)
    padded[:, :K] = q
    W = torch.from_numpy(padded).to(dev)
    S = torch.from_numpy(scale).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    Y = torch.from_numpy(y0.copy()).to(dev) if y0 is not None else torch.full((T, N), float("nan"), device=dev)
    print(f"gemm_w8 case: T={T} K={K} N={N} ldw={ldw} beta={beta}", flush=True)
    _lib.check(_lib.lib().rh_gemm_w8(W.data_ptr(), ldw, S.data_ptr(), X.data_ptr(), Y.data_ptr(), T, K, N, beta, None),
               "rh_gemm_w8")
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def run_split(torch, dev, q, scale, x, ks):
    from relay_amd import _lib

    N, K = q.shape
    T = x.shape[0]
    W = torch.from_numpy(q).to(dev)
    S = torch.from_numpy(scale).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    Y = torch.full((T, N), float("nan"), device=dev)
    ws = torch.full((ks * T * N,), float("nan"), device=dev)
    print(f"gemm_w8_split case: T={T} K={K} N={N} ksplit={ks}", flush=True)
    _lib.check(_lib.lib().rh_gemm_w8_split(W.data_ptr(), K, S.data_ptr(), X.data_ptr(), Y.data_ptr(), T, K, N, 0.0, ks,
                                           ws.data_ptr(), None), "rh_gemm_w8_split")
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def check(y, q, scale, x, beta=0.0, y0=None, rows=None):
    """rows: check only these output rows n (float64 over all of a large matrix is slow)."""
    if rows is not None:
        y, q, scale = y[:, rows], q[rows], scale[rows]
        y0 = None if y0 is None else y0[:, rows]
    qd, xd, sd = q.astype(np.float64), x.astype(np.float64), scale.astype(np.float64)
    dot = xd @ qd.T
    mag = (np.abs(xd) @ np.abs(qd).T) * np.abs(sd)
    exact = dot * sd + (beta * y0.astype(np.float64) if beta else 0.0)
    bound = (4 * q.shape[1] * EPS32 + 2 * EPS32) * mag + 1e-30
    if beta:
        bound = bound + 2 * EPS32 * np.abs(beta * y0.astype(np.float64)) + 2 * EPS32 * np.abs(exact)
    err = np.abs(y - exact)
    assert np.isfinite(y).all()
    assert (err <= bound).all(), f"worst excess {np.max(err - bound):.3e}"


@pytest.mark.parametrize("T", [1, 17, 100, 128, 129, 300])
@pytest.mark.parametrize("N,K", [(64, 64), (100, 128), (576, 1536), (1000, 5632)])
def test_matches_float64(torch_mod, dev, T, N, K):
    q, s, x = make(N, K, T, seed=T * 13 + N + K)
    check(run(torch_mod, dev, q, s, x), q, s, x)


@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 4096), (4096, 14336)])
def test_llama3_shapes_at_the_mixed_batch(torch_mod, dev, N, K):
    q, s, x = make(N, K, 560, seed=N + K)
    check(run(torch_mod, dev, q, s, x), q, s, x)


def test_wide_matrix_at_the_mixed_batch(torch_mod, dev):
    """Llama-3-8B's gate_up (28672 x 4096) at T = 560 runs the 256 x 96 tile; 1536 rows
    spread over the matrix are checked against float64."""
    from relay_amd import _lib

    assert _lib.lib().rh_gemm_w8_kernel(560, 4096, 28672, 1) == 1
    q, s, x = make(28672, 4096, 560, seed=7)
    rows = np.sort(np.random.default_rng(8).choice(28672, 1536, replace=False))
    check(run(torch_mod, dev, q, s, x), q, s, x, rows=rows)


@pytest.mark.parametrize("ks", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("T,N,K", [(300, 576, 1536), (65, 256, 4096), (129, 1000, 5632), (560, 4096, 1024)])
def test_split_matches_float64(torch_mod, dev, ks, T, N, K):
    """rh_gemm_w8_split: K cut into 1-8 ranges (a range of 2 steps at K = 1024, ks = 8),
    ranges added in order by the merge launch."""
    q, s, x = make(N, K, T, seed=T + N + K + ks)
    check(run_split(torch_mod, dev, q, s, x, ks), q, s, x)


def test_split_is_deterministic(torch_mod, dev):
    q, s, x = make(512, 4096, 200, seed=9)
    a = run_split(torch_mod, dev, q, s, x, 4)
    b = run_split(torch_mod, dev, q, s, x, 4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_plan(dev):
    from relay_amd import _lib

    L = _lib.lib()
    # Llama-3-8B at config 5's 560 tokens: qkv, wo, gate_up, down
    shapes = ((6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336))
    assert [L.rh_gemm_w8_plan(560, k, n) for n, k in shapes] == [1, 1, 1, 3]
    assert [L.rh_gemm_w8_kernel(560, k, n, L.rh_gemm_w8_plan(560, k, n)) for n, k in shapes] == [2, 3, 1, 2]
    # merged by the consumer (o, down, gate_up): unsplit grids under 256 workgroups take K ranges
    assert [L.rh_gemm_w8_partials_plan(560, k, n) for n, k in shapes] == [2, 3, 1, 3]
    assert L.rh_gemm_w8_kernel(560, 4096, 4096, 3) == 2 and L.rh_gemm_w8_partials_plan(0, 64, 64) == -1
    assert L.rh_gemm_w8_partials_plan(48, 4096, 4096) == L.rh_gemm_w8_plan(48, 4096, 4096)
    # TinyLlama at 512-token prefill chunks: qkv, wo, gate_up, down
    shapes = ((2560, 2048), (2048, 2048), (11264, 2048), (2048, 5632))
    assert [L.rh_gemm_w8_plan(512, k, n) for n, k in shapes] == [1, 2, 1, 4]
    assert [L.rh_gemm_w8_partials_plan(512, k, n) for n, k in shapes] == [2, 2, 1, 4]
    assert L.rh_gemm_w8_plan(560, 100, 64) == -1 and L.rh_gemm_w8_plan(0, 64, 64) == -1
    assert L.rh_gemm_w8_plan(100, 128, 4096) == 1  # ranges of at least two 128-k steps
    # K not a multiple of 128: the 64-k step kernels; at most 64 tokens: the 128 x 128 tile
    assert L.rh_gemm_w8_kernel(300, 576, 1536, 1) == 0 and L.rh_gemm_w8_kernel(64, 4096, 4096, 2) == 0
    assert L.rh_gemm_w8_kernel(300, 1024, 1024, 9) == -1 and L.rh_gemm_w8_kernel(300, 1024, 1024, 8) in (2, 3)


WIDE_CASES = [(65, 256, 4096, 4), (97, 1000, 1280, 3), (200, 250, 640, 1), (300, 512, 128, 1), (450, 132, 1152, 5),
              (560, 2048, 2048, 2), (128, 4096, 640, 5), (250, 4096, 1280, 3), (512, 2048, 1152, 3)]


@pytest.mark.parametrize("T,N,K,ks", WIDE_CASES)
def test_wide_step_kernels(torch_mod, dev, T, N, K, ks):
    """The 128-k step kernels (128 x 128 and 128 x 96 tiles): odd step counts per range (the
    paired loop's zero step), one step, partial row and token tiles, N not a multiple of 4
    (scalar stores), several K ranges; within the fp32 bound and the same bits on a repeat."""
    from relay_amd import _lib

    cfg = _lib.lib().rh_gemm_w8_kernel(T, K, N, ks)
    assert cfg in (2, 3), cfg
    q, s, x = make(N, K, T, seed=T * 7 + N + K + ks)
    y = run_split(torch_mod, dev, q, s, x, ks)
    check(y, q, s, x)
    assert np.array_equal(y.view(np.uint32), run_split(torch_mod, dev, q, s, x, ks).view(np.uint32))


def test_wide_step_kernels_cover_both_tiles(dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert {L.rh_gemm_w8_kernel(T, K, N, ks) for T, N, K, ks in WIDE_CASES} == {2, 3}


def test_beta_accumulates(torch_mod, dev):
    q, s, x = make(300, 512, 150, seed=1)
    y0 = np.random.default_rng(2).standard_normal((150, 300)).astype(np.float32)
    check(run(torch_mod, dev, q, s, x, beta=1.0, y0=y0), q, s, x, beta=1.0, y0=y0)


def test_row_stride_gives_the_same_bits(torch_mod, dev):
    q, s, x = make(200, 256, 40, seed=3)
    a = run(torch_mod, dev, q, s, x)
    b = run(torch_mod, dev, q, s, x, ldw=256 + 272)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_agrees_with_the_gemv_on_its_range(torch_mod, dev):
    """Both int8 paths compute scale * (fp32 sum of exact products): on T <= 16 they may
    differ only by accumulation order."""
    from relay_amd import _lib

    torch = torch_mod
    q, s, x = make(512, 1024, 16, seed=4)
    a = run(torch, dev, q, s, x)
    W = torch.from_numpy(q).to(dev)
    S = torch.from_numpy(s).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    Y = torch.empty((16, 512), device=dev)
    _lib.check(_lib.lib().rh_gemv_int8(W.data_ptr(), 1024, S.data_ptr(), 0, X.data_ptr(), Y.data_ptr(), 16, 1024, 512,
                                       0.0, None), "rh_gemv_int8")
    torch.cuda.synchronize()
    b = Y.cpu().numpy()
    mag = (np.abs(x.astype(np.float64)) @ np.abs(q.astype(np.float64)).T) * s
    assert (np.abs(a - b) <= 8 * 1024 * EPS32 * mag + 1e-30).all()


def test_rejects_bad_shapes(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemm_w8(None, 96, None, None, None, 4, 96, 64, 0.0, None) != 0 and "K must" in _lib.last_error()
    assert L.rh_gemm_w8(None, 72, None, None, None, 4, 64, 64, 0.0, None) != 0 and "ldw" in _lib.last_error()
    assert L.rh_gemm_w8(None, 64, None, None, None, 0, 64, 64, 0.0, None) == 0  # nothing to do
    assert L.rh_gemm_w8_split(None, 64, None, None, None, 4, 64, 64, 0.0, 2, None, None) != 0  # 2 ranges of 1 step
    assert "ksplit" in _lib.last_error()
    assert L.rh_gemm_w8_split(None, 128, None, None, None, 4, 128, 64, 0.0, 2, None, None) != 0
    assert "workspace" in _lib.last_error()
    assert L.rh_gemm_w8_split(None, 128, None, None, None, 4, 128, 66, 0.0, 2, None, None) != 0


def run_skinny(torch, dev, q, scale, x, ks, beta=0.0, y0=None, ldw=None):
    from relay_amd import _lib

    N, K = q.shape
    T = x.shape[0]
    ldw = K if ldw is None else ldw
    padded = np.full((N, ldw), 99, np.int8)
    padded[:, :K] = q
    W = torch.from_numpy(padded).to(dev)
    S = torch.from_numpy(scale).to(dev)
    X = torch.from_numpy(x.view(np.int16)).to(dev)
    Y = torch.from_numpy(y0.copy()).to(dev) if y0 is not None else torch.full((T, N), float("nan"), device=dev)
    ws = torch.full((ks * T * N,), float("nan"), device=dev)
    print(f"gemm_w8_skinny case: T={T} K={K} N={N} ldw={ldw} ksplit={ks} beta={beta}", flush=True)
    _lib.check(_lib.lib().rh_gemm_w8_skinny(W.data_ptr(), ldw, S.data_ptr(), X.data_ptr(), Y.data_ptr(), T, K, N, beta,
                                            ks, ws.data_ptr(), None), "rh_gemm_w8_skinny")
    torch.cuda.synchronize()
    return Y.cpu().numpy()


@pytest.mark.parametrize("ks", [1, 2, 3, 8])
@pytest.mark.parametrize("T,N,K", [(1, 64, 1024), (17, 200, 2048), (48, 1000, 4096), (64, 4096, 14336 // 4), (20, 256, 640),
                                   (33, 132, 1088)])
def test_skinny_split_k_matches_float64(torch_mod, dev, T, N, K, ks):
    """rh_gemm_w8_skinny at any K split (ranges of whole 64-k steps) stays within the
    fp32 bound; the split adds the ranges in order, so a repeat gives the same bits."""
    q, scale, x = make(N, K, T, seed=T + N + K + ks)
    y = run_skinny(torch_mod, dev, q, scale, x, ks)
    check(y, q, scale, x)
    assert np.array_equal(y.view(np.uint32), run_skinny(torch_mod, dev, q, scale, x, ks).view(np.uint32))


def test_skinny_accumulates_and_limits(torch_mod, dev):
    from relay_amd import _lib

    q, scale, x = make(300, 2048, 40, seed=9)
    y0 = np.random.default_rng(4).standard_normal((40, 300)).astype(np.float32)
    check(run_skinny(torch_mod, dev, q, scale, x, 4, beta=1.0, y0=y0), q, scale, x, beta=1.0, y0=y0)
    L = _lib.lib()
    assert L.rh_gemm_w8_split_plan(48, 14336, 4096) == 8 and L.rh_gemm_w8_split_plan(48, 4096, 28672) == 1
    assert L.rh_gemm_w8_split_plan(65, 4096, 4096) == -1
    assert L.rh_gemm_w8_skinny(None, 128, None, None, None, 65, 128, 64, 0.0, 1, None, None) != 0
    assert "T must be in 1..64" in _lib.last_error()
    assert L.rh_gemm_w8_skinny(None, 64, None, None, None, 8, 64, 64, 0.0, 2, None, None) != 0
    assert "ksplit" in _lib.last_error()
    assert L.rh_gemm_w8_skinny(None, 256, None, None, None, 8, 256, 64, 0.0, 2, None, None) != 0
    assert "workspace" in _lib.last_error()


@pytest.mark.parametrize("T,I,H,ks", [(17, 1024, 512, 2), (32, 5632, 2048, 3), (48, 2048, 4096, 8), (100, 1536, 576, 4),
                                      (200, 1024, 1024, 3), (560, 4096, 4096, 3)])
def test_merge_fused_consumers_equal_the_chain(torch_mod, dev, T, I, H, ks):
    """rh_gemm_w8_partials + rh_w8_merge_silu equals the split product + rh_silu_mul, and
    rh_gemm_w8_partials + rh_w8_merge_rmsnorm equals the split product accumulated into the
    residual (beta = 1) + rh_rmsnorm, byte for byte (same partials, same merge arithmetic)."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    rng = np.random.default_rng(T + I + H + ks)
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    split = (lambda *a: L.rh_gemm_w8_skinny(*a)) if T <= 64 else (lambda *a: L.rh_gemm_w8_split(*a))
    print(f"fused merges: T={T} I={I} H={H} ksplit={ks}", flush=True)
    # gate_up [2I, H] then SiLU
    q, s, x = make(2 * I, H, T, seed=T + 1)
    Wg, Sg, X = dt(q), dt(s), dt(x.view(np.int16))
    ws = torch.empty(ks * T * 2 * I, device=dev)
    gu = torch.empty((T, 2 * I), device=dev)
    act_a = torch.empty((T, I), dtype=torch.int16, device=dev)
    act_b = torch.empty((T, I), dtype=torch.int16, device=dev)
    _lib.check(split(Wg.data_ptr(), H, Sg.data_ptr(), X.data_ptr(), gu.data_ptr(), T, H, 2 * I, 0.0, ks, ws.data_ptr(),
                     None), "split product")
    _lib.check(L.rh_silu_mul(gu.data_ptr(), T, I, act_a.data_ptr(), None), "rh_silu_mul")
    _lib.check(L.rh_gemm_w8_partials(Wg.data_ptr(), H, X.data_ptr(), T, H, 2 * I, ks, ws.data_ptr(), None), "partials")
    _lib.check(L.rh_w8_merge_silu(ws.data_ptr(), ks, T, I, Sg.data_ptr(), act_b.data_ptr(), None), "merge_silu")
    torch.cuda.synchronize()
    assert np.array_equal(act_a.cpu().numpy(), act_b.cpu().numpy())
    # down [H, I] into the residual, then RMSNorm
    q, s, a8 = make(H, I, T, seed=T + 2)
    Wd, Sd, A = dt(q), dt(s), dt(a8.view(np.int16))
    x0 = rng.standard_normal((T, H)).astype(np.float32)
    nw = dt(rng.uniform(0.5, 1.5, H).astype(np.float32))
    xa, xb = dt(x0), dt(x0)
    ws2 = torch.empty(ks * T * H, device=dev)
    na = torch.empty((T, H), dtype=torch.int16, device=dev)
    nb = torch.empty((T, H), dtype=torch.int16, device=dev)
    _lib.check(split(Wd.data_ptr(), I, Sd.data_ptr(), A.data_ptr(), xa.data_ptr(), T, I, H, 1.0, ks, ws2.data_ptr(),
                     None), "split product (beta 1)")
    _lib.check(L.rh_rmsnorm(xa.data_ptr(), None, T, nw.data_ptr(), H, 1e-5, na.data_ptr(), None), "rh_rmsnorm")
    _lib.check(L.rh_gemm_w8_partials(Wd.data_ptr(), I, A.data_ptr(), T, I, H, ks, ws2.data_ptr(), None), "partials")
    _lib.check(L.rh_w8_merge_rmsnorm(ws2.data_ptr(), ks, T, H, Sd.data_ptr(), xb.data_ptr(), nw.data_ptr(), 1e-5,
                                     nb.data_ptr(), None), "merge_rmsnorm")
    torch.cuda.synchronize()
    assert np.array_equal(xa.cpu().numpy().view(np.uint32), xb.cpu().numpy().view(np.uint32))
    assert np.array_equal(na.cpu().numpy(), nb.cpu().numpy())
    check(xa.cpu().numpy() - x0, q, s, a8)  # and the product itself within the fp32 bound


def test_merge_fused_limits(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_w8_merge_rmsnorm_fits(4096) and not L.rh_w8_merge_rmsnorm_fits(4100) and not L.rh_w8_merge_rmsnorm_fits(8192)
    assert L.rh_gemm_w8_partials(None, 128, None, 4, 128, 64, 1, None, None) != 0 and "ksplit" in _lib.last_error()
    assert L.rh_w8_merge_silu(None, 2, 4, 12, None, None, None) != 0


@pytest.mark.parametrize("T,I,K", [(560, 14336, 4096), (512, 5632, 2048), (100, 1000, 256), (129, 250, 128),
                                   (300, 1536, 576), (65, 130, 64), (1, 64, 64), (97, 8, 192)])
def test_gate_up_silu_equals_the_chain(torch_mod, dev, T, I, K):
    """rh_gemm_w8_gate_up_silu against rh_gemm_w8 into an fp32 [T, 2 I] buffer + rh_silu_mul:
    the same bytes where the chain's product runs the same 256 x 96 tile (rh_gemm_w8_kernel
    = 1); elsewhere within the fp32 accumulation bound of g and u carried through SiLU·mul
    plus one fp16 rounding (checked on sampled outputs). Covers partial row and token tiles
    and I not a multiple of 4 (scalar stores)."""
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    q, s, x = make(2 * I, K, T, seed=T * 7 + I + K)
    W, S, X = dt(q), dt(s), dt(x.view(np.int16))
    gu = torch.empty((T, 2 * I), device=dev)
    act_a = torch.empty((T, I), dtype=torch.int16, device=dev)
    act_b = torch.full((T, I), 0x7E00, dtype=torch.int16, device=dev)
    print(f"gemm_w8_gate_up_silu case: T={T} I={I} K={K}", flush=True)
    _lib.check(L.rh_gemm_w8(W.data_ptr(), K, S.data_ptr(), X.data_ptr(), gu.data_ptr(), T, K, 2 * I, 0.0, None),
               "rh_gemm_w8")
    _lib.check(L.rh_silu_mul(gu.data_ptr(), T, I, act_a.data_ptr(), None), "rh_silu_mul")
    _lib.check(L.rh_gemm_w8_gate_up_silu(W.data_ptr(), K, S.data_ptr(), X.data_ptr(), act_b.data_ptr(), T, K, I, None),
               "rh_gemm_w8_gate_up_silu")
    torch.cuda.synchronize()
    a, b = act_a.cpu().numpy(), act_b.cpu().numpy()
    if L.rh_gemm_w8_kernel(T, K, 2 * I, 1) == 1:
        assert np.array_equal(a, b)
    rows = np.unique(np.random.default_rng(I).integers(0, I, size=min(I, 256)))
    qd, xd, sd = q.astype(np.float64), x.astype(np.float64), s.astype(np.float64)
    cols = np.concatenate([rows, I + rows])
    dot = (xd @ qd[cols].T) * sd[cols]
    err = (4 * K * EPS32 + 2 * EPS32) * (np.abs(xd) @ np.abs(qd[cols]).T) * sd[cols] + 1e-30
    n = len(rows)
    g, u, eg, eu = dot[:, :n], dot[:, n:], err[:, :n], err[:, n:]
    silu = g / (1.0 + np.exp(-g))
    tol = 1.1 * np.abs(u) * eg + np.abs(silu) * eu + eg * eu
    want = silu * u
    for got in (a, b):
        v = got[:, rows].view(np.float16).astype(np.float64)
        lim = tol + 2.0 ** -10 * np.maximum(np.abs(v), np.abs(want)) + 2.0 ** -24
        assert (np.abs(v - want) <= lim).all()


def test_gate_up_silu_limits(dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_gemm_w8_gate_up_silu(None, 128, None, None, None, 4, 128, 64, None) != 0
    assert "missing pointer" in _lib.last_error()
