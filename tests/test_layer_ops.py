"""The small layer kernels: bit-exact conversions and indexing, tolerances elsewhere.

- rh_f32_to_f16 vs relay's f32_to_f16 (the oracle's restatement, itself pinned against
  the reference build): every bit equal, including subnormals, ties and overflow.
- rh_quantize_int8 vs relay's host quantizer: identical int8 values and scales.
- rh_kv_gather / rh_kv_scatter: round trips are the identity on bytes.
- rh_qkv_post: with inv_freq = 0 (no rotation) the cache write is fp16(k) at exactly
  table[p / bs], slot p % bs -- bit-exact placement; with real frequencies, RoPE within
  fp32 rounding of the oracle's.
"""
import numpy as np
import pytest

import oracle as O
from helpers import bits_to_f32, f16_bits

pytestmark = pytest.mark.gpu


def special_floats():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e10, -1e10, np.inf, -np.inf,
            2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -26, 1.5 * 2.0 ** -24, 2.0 ** -15 * 1.5,
            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -12, 0.1, 1e-8, -5e-8]
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    rnd = bits.view(np.float32)
    rnd = rnd[np.isfinite(rnd)]
    # every halfway point between consecutive fp16 values in [1, 2) and in the subnormals
    half = np.arange(0x3C00, 0x4000, dtype=np.uint16)
    mids = (bits_to_f32(half).astype(np.float64) + 2.0 ** -11).astype(np.float32)
    sub = np.arange(1, 1024, dtype=np.float64) * 2.0 ** -24 + 2.0 ** -25
    return np.concatenate([np.array(vals, np.float32), rnd, mids, sub.astype(np.float32),
                           rng.standard_normal(100000).astype(np.float32)])


@pytest.mark.parametrize("shift,count", [(0, None), (1, None), (0, 7), (3, 21)])
def test_f32_to_f16_bit_exact(torch_mod, dev, shift, count):
    """Aligned (8-wide path plus scalar tail), misaligned (scalar path) and short inputs."""
    from relay_amd import _lib

    x = special_floats()
    n = x.size - shift if count is None else count
    X = torch_mod.from_numpy(x).to(dev)
    Y = torch_mod.full((x.size,), 0x7E00, dtype=torch_mod.int16, device=dev)
    _lib.check(_lib.lib().rh_f32_to_f16(X.data_ptr() + 4 * shift, Y.data_ptr() + 2 * shift, n, None))
    torch_mod.cuda.synchronize()
    got = Y.cpu().numpy().view(np.uint16)
    want = O.f32_to_f16(x[shift:shift + n])
    assert np.array_equal(got[shift:shift + n], want), f"{np.count_nonzero(got[shift:shift + n] != want)} of {n} differ"
    assert (got[:shift] == 0x7E00).all() and (got[shift + n:] == 0x7E00).all()


def test_quantize_int8_bit_exact(torch_mod, dev):
    from relay_amd import _lib

    rng = np.random.default_rng(1)
    w = (rng.standard_normal((257, 1000)) * 0.02).astype(np.float32)
    w[3] = 0.0  # an all-zero row: scale 1
    w[5, :7] = [0.5, -0.5, 0.25, 1.0, -1.0, 127.0 / 254.0, 3.0 / 254.0]  # halfway cases for rint
    q_want, s_want = O.quantize_int8(w)
    W = torch_mod.from_numpy(w).to(dev)
    ldq = 1024 + 256  # padded rows: the bytes past K stay as they were
    Q = torch_mod.full((w.shape[0], ldq), 55, dtype=torch_mod.int8, device=dev)
    S = torch_mod.empty(w.shape[0], dtype=torch_mod.float32, device=dev)
    _lib.check(_lib.lib().rh_quantize_int8(W.data_ptr(), w.shape[0], w.shape[1], Q.data_ptr(), ldq, S.data_ptr(), None))
    torch_mod.cuda.synchronize()
    assert np.array_equal(S.cpu().numpy().view(np.uint32), s_want.view(np.uint32))
    q = Q.cpu().numpy()
    assert np.array_equal(q[:, :w.shape[1]], q_want) and (q[:, w.shape[1]:] == 55).all()
    # dequant from the padded rows: fp16(q * scale), dense output
    D = torch_mod.empty(w.shape, dtype=torch_mod.float16, device=dev)
    _lib.check(_lib.lib().rh_dequant_int8(Q.data_ptr(), ldq, S.data_ptr(), w.shape[0], w.shape[1], D.data_ptr(), None))
    torch_mod.cuda.synchronize()
    want = (q_want.astype(np.float32) * s_want[:, None]).astype(np.float16)
    assert np.array_equal(D.cpu().numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("N,K,ldq", [(300, 4096, 4096 + 256), (64, 14336, 14336 + 256), (33, 48, 64), (5, 40, 40)])
def test_dequant_int8_bit_exact(torch_mod, dev, N, K, ldq):
    """fp16(fp32(q * scale)) for every element, from padded rows (K % 16 == 0: 16 weights per
    thread; otherwise one per thread)."""
    from relay_amd import _lib

    rng = np.random.default_rng(K + N)
    q = rng.integers(-127, 128, size=(N, ldq)).astype(np.int8)
    s = (rng.uniform(1e-4, 1e-2, N)).astype(np.float32)
    Q, S = torch_mod.from_numpy(q).to(dev), torch_mod.from_numpy(s).to(dev)
    D = torch_mod.empty((N, K), dtype=torch_mod.float16, device=dev)
    print(f"dequant: N={N} K={K} ldq={ldq}", flush=True)
    _lib.check(_lib.lib().rh_dequant_int8(Q.data_ptr(), ldq, S.data_ptr(), N, K, D.data_ptr(), None), "rh_dequant_int8")
    torch_mod.cuda.synchronize()
    want = (q[:, :K].astype(np.float32) * s[:, None]).astype(np.float16)
    assert np.array_equal(D.cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_kv_gather_scatter_round_trip(torch_mod, dev):
    from relay_amd import _lib

    rng = np.random.default_rng(2)
    nb, bb = 40, 4 * 16 * 64 * 2
    k = rng.integers(0, 2 ** 16, size=nb * bb // 2, dtype=np.uint16)
    v = rng.integers(0, 2 ** 16, size=nb * bb // 2, dtype=np.uint16)
    K = torch_mod.from_numpy(k.view(np.int16)).to(dev)
    V = torch_mod.from_numpy(v.view(np.int16)).to(dev)
    ids = [7, 3, 39, 0, 12]
    I = torch_mod.tensor(ids, dtype=torch_mod.int32, device=dev)
    buf = torch_mod.empty(2 * len(ids) * bb // 2, dtype=torch_mod.int16, device=dev)
    _lib.check(_lib.lib().rh_kv_gather(K.data_ptr(), V.data_ptr(), I.data_ptr(), len(ids), bb, buf.data_ptr(), None))
    torch_mod.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16).reshape(2, len(ids), bb // 2)
    for i, b in enumerate(ids):
        assert np.array_equal(got[0, i], k[b * bb // 2:(b + 1) * bb // 2])
        assert np.array_equal(got[1, i], v[b * bb // 2:(b + 1) * bb // 2])
    K2 = torch_mod.zeros_like(K)
    V2 = torch_mod.zeros_like(V)
    _lib.check(_lib.lib().rh_kv_scatter(K2.data_ptr(), V2.data_ptr(), I.data_ptr(), len(ids), bb, buf.data_ptr(), None))
    torch_mod.cuda.synchronize()
    k2, v2 = K2.cpu().numpy().view(np.uint16), V2.cpu().numpy().view(np.uint16)
    for b in ids:
        assert np.array_equal(k2[b * bb // 2:(b + 1) * bb // 2], k[b * bb // 2:(b + 1) * bb // 2])
        assert np.array_equal(v2[b * bb // 2:(b + 1) * bb // 2], v[b * bb // 2:(b + 1) * bb // 2])


@pytest.mark.parametrize("bs", [1, 16, 12])
def test_qkv_post_places_kv_bit_exact(torch_mod, dev, bs):
    from relay_amd import _lib

    heads, kvh, D = 8, 2, 64
    Q, KV = heads * D, kvh * D
    QKV = Q + 2 * KV
    rng = np.random.default_rng(bs)
    # two chunks: positions 0..40 of seq 0, positions 17..19 of seq 1
    pos = list(range(41)) + [17, 18, 19]
    seq = [0] * 41 + [1] * 3
    nb0, nb1 = (41 + bs - 1) // bs, (20 + bs - 1) // bs
    nblocks = nb0 + nb1 + 2
    perm = rng.permutation(nblocks)
    tables = [int(b) for b in perm[:nb0 + nb1]]
    toff = [0, nb0]
    T = len(pos)
    qkv = rng.standard_normal((T, QKV)).astype(np.float32)
    bias = rng.standard_normal(QKV).astype(np.float32)
    dt = lambda a: torch_mod.from_numpy(np.ascontiguousarray(a)).to(dev)
    QKVt, B = dt(qkv), dt(bias)
    inv0 = dt(np.zeros(D // 2, np.float32))
    P, S, TO, TB = dt(np.array(pos, np.int32)), dt(np.array(seq, np.int32)), dt(np.array(toff, np.int32)), \
        dt(np.array(tables, np.int32))
    kc = torch_mod.zeros(nblocks * kvh * bs * D, dtype=torch_mod.int16, device=dev)
    vc = torch_mod.zeros_like(kc)
    qo = torch_mod.empty(T * Q, dtype=torch_mod.int16, device=dev)
    _lib.check(_lib.lib().rh_qkv_post(QKVt.data_ptr(), T, B.data_ptr(), inv0.data_ptr(), P.data_ptr(), S.data_ptr(),
                                      TO.data_ptr(), TB.data_ptr(), kc.data_ptr(), vc.data_ptr(), qo.data_ptr(), 1.0,
                                      heads, kvh, D, bs, None))
    torch_mod.cuda.synchronize()
    row = qkv + bias  # fp32 adds, as the kernel does
    k_cache = kc.cpu().numpy().view(np.uint16)
    v_cache = vc.cpu().numpy().view(np.uint16)
    for t in range(T):
        blk = tables[toff[seq[t]] + pos[t] // bs]
        for h in range(kvh):
            off = ((blk * kvh + h) * bs + pos[t] % bs) * D
            assert np.array_equal(k_cache[off:off + D], O.f32_to_f16(row[t, Q + h * D:Q + (h + 1) * D]))
            assert np.array_equal(v_cache[off:off + D], O.f32_to_f16(row[t, Q + KV + h * D:Q + KV + (h + 1) * D]))
    assert np.array_equal(qo.cpu().numpy().view(np.uint16).reshape(T, Q), O.f32_to_f16(row[:, :Q]))


def test_qkv_post_rope_matches_oracle(torch_mod, dev):
    """RoPE with real frequencies (Llama 3 scaling): within fp32 rounding of cosf/sinf."""
    from relay_amd import _lib
    from relay_amd.model import llama3_8b

    c = llama3_8b()
    heads, kvh, D = 4, 2, c.head_dim
    inv = O.rope_inv_freq(c)
    Q, KV = heads * D, kvh * D
    rng = np.random.default_rng(9)
    pos = [0, 1, 100, 4095, 8191, 20000]
    T = len(pos)
    qkv = rng.standard_normal((T, Q + 2 * KV)).astype(np.float32)
    dt = lambda a: torch_mod.from_numpy(np.ascontiguousarray(a)).to(dev)
    X = dt(qkv)
    # every token its own sequence whose table maps all positions to block 0 (bs 16)
    bs = 16
    tables, toff = [], []
    for p in pos:
        toff.append(len(tables))
        tables.extend([0] * (p // bs + 1))
    kc = torch_mod.zeros(kvh * bs * D, dtype=torch_mod.int16, device=dev)
    vc = torch_mod.zeros_like(kc)
    # keep every device buffer referenced until the kernel has run (a temporary's memory
    # goes back to torch's caching allocator as soon as its data_ptr() is taken)
    INV, POS, SEQ = dt(inv), dt(np.array(pos, np.int32)), dt(np.arange(T, dtype=np.int32))
    TOFF, TABS = dt(np.array(toff, np.int32)), dt(np.array(tables, np.int32))
    _lib.check(_lib.lib().rh_qkv_post(X.data_ptr(), T, None, INV.data_ptr(), POS.data_ptr(), SEQ.data_ptr(),
                                      TOFF.data_ptr(), TABS.data_ptr(), kc.data_ptr(), vc.data_ptr(), None,
                                      1.0, heads, kvh, D, bs, None))
    torch_mod.cuda.synchronize()
    got = X.cpu().numpy()
    half = D // 2
    for t, p in enumerate(pos):
        ang = np.float32(p) * inv
        cs, sn = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
        for h in range(heads + kvh):
            a, b = qkv[t, h * D:h * D + half].astype(np.float64), qkv[t, h * D + half:(h + 1) * D].astype(np.float64)
            want = np.concatenate([a * cs - b * sn, b * cs + a * sn])
            # angle pos * inv_freq is rounded to fp32 on both sides; cos/sin of it agree to ~1 ulp
            assert np.abs(got[t, h * D:(h + 1) * D] - want).max() <= 4e-6 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("H", [576, 2048, 4096, 102, 8192])
def test_rmsnorm_bit_exact(torch_mod, dev, H):
    """out[r] = fp16(w * (x[rows[r]] * inv)), inv = 1 / sqrt(fp32(sum x^2 / H) + eps) with the sum
    in double (cpu_backend.cpp:47-52); fp32 division and square root are correctly rounded, so
    numpy reproduces every bit. H = 576..4096 take the vectorised kernel, 102 and 8192 the
    strided one."""
    from relay_amd import _lib

    rng = np.random.default_rng(H)
    R, rows_n = 7, 11
    x = (rng.standard_normal((rows_n, H)) * rng.uniform(0.1, 30, (rows_n, 1))).astype(np.float32)
    w = rng.uniform(0.2, 2.0, H).astype(np.float32)
    rows = rng.permutation(rows_n)[:R].astype(np.int32)
    eps = np.float32(1e-5)
    xd = x[rows].astype(np.float64)
    ss = (xd * xd).sum(axis=1)
    inv = np.float32(1.0) / np.sqrt((ss / H).astype(np.float32) + eps)
    want = (w[None, :] * (x[rows] * inv[:, None])).astype(np.float16)
    dt = lambda a: torch_mod.from_numpy(np.ascontiguousarray(a)).to(dev)
    X, Wt, RW = dt(x), dt(w), dt(rows)
    out = torch_mod.empty((R, H), dtype=torch_mod.int16, device=dev)
    print(f"rmsnorm: H={H}", flush=True)
    _lib.check(_lib.lib().rh_rmsnorm(X.data_ptr(), RW.data_ptr(), R, Wt.data_ptr(), H, float(eps), out.data_ptr(), None),
               "rh_rmsnorm")
    torch_mod.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want.view(np.int16))


@pytest.mark.parametrize("T,I", [(1, 1536), (32, 5632), (5, 14336), (3, 100)])
def test_silu_mul_within_one_fp16_ulp(torch_mod, dev, T, I):
    """act = fp16(g / (1 + exp(-g)) * u) (cpu_backend.cpp:193): within one fp16 ulp of the
    float64 value rounded to fp16 (expf is not correctly rounded). I = 100 takes the strided
    kernel, the others the vectorised one."""
    from relay_amd import _lib

    rng = np.random.default_rng(T + I)
    gu = (rng.standard_normal((T, 2 * I)) * 3).astype(np.float32)
    g, u = gu[:, :I].astype(np.float64), gu[:, I:].astype(np.float64)
    want = (g / (1 + np.exp(-g)) * u).astype(np.float16)
    G = torch_mod.from_numpy(gu).to(dev)
    out = torch_mod.empty((T, I), dtype=torch_mod.int16, device=dev)
    print(f"silu_mul: T={T} I={I}", flush=True)
    _lib.check(_lib.lib().rh_silu_mul(G.data_ptr(), T, I, out.data_ptr(), None), "rh_silu_mul")
    torch_mod.cuda.synchronize()
    got = out.cpu().numpy().view(np.float16)
    ulp = np.abs(np.spacing(want.astype(np.float16)).astype(np.float64))
    assert (np.abs(got.astype(np.float64) - want.astype(np.float64)) <= ulp + 1e-30).all()


@pytest.mark.parametrize("bs", [16, 12])
def test_qkv_post_to_cache_matches_qkv_post(torch_mod, dev, bs):
    """rh_qkv_post_to_cache writes the same q (fp16) and cache bytes as rh_qkv_post, with
    real RoPE frequencies and a bias, and leaves qkv as it was."""
    from relay_amd import _lib
    from relay_amd.model import tinyllama_1b

    heads, kvh, D = 8, 2, 64
    Q, KV = heads * D, kvh * D
    QKV = Q + 2 * KV
    rng = np.random.default_rng(bs + 7)
    pos = list(range(30)) + [100, 101, 333]
    seq = [0] * 30 + [1] * 3
    nb0, nb1 = (30 + bs - 1) // bs, (334 + bs - 1) // bs
    nblocks = nb0 + nb1 + 3
    tables = [int(b) for b in rng.permutation(nblocks)[:nb0 + nb1]]
    T = len(pos)
    qkv = rng.standard_normal((T, QKV)).astype(np.float32)
    inv = O.rope_inv_freq(tinyllama_1b())
    dt = lambda a: torch_mod.from_numpy(np.ascontiguousarray(a)).to(dev)
    B, INV = dt(rng.standard_normal(QKV).astype(np.float32)), dt(inv)
    P, S, TO, TB = dt(np.array(pos, np.int32)), dt(np.array(seq, np.int32)), dt(np.array([0, nb0], np.int32)), \
        dt(np.array(tables, np.int32))
    outs = []
    q_scale = 0.125 * 1.4426950408889634  # softmax scale * log2(e) at head size 64, as the backend passes
    for fn in ("rh_qkv_post", "rh_qkv_post_to_cache"):
        X = dt(qkv)
        kc = torch_mod.full((nblocks * kvh * bs * D,), 0x7BFF, dtype=torch_mod.int16, device=dev)
        vc = kc.clone()
        qo = torch_mod.zeros(T * Q, dtype=torch_mod.int16, device=dev)
        print(f"{fn}: T={T} bs={bs}", flush=True)
        _lib.check(getattr(_lib.lib(), fn)(X.data_ptr(), T, B.data_ptr(), INV.data_ptr(), P.data_ptr(), S.data_ptr(),
                                           TO.data_ptr(), TB.data_ptr(), kc.data_ptr(), vc.data_ptr(), qo.data_ptr(),
                                           q_scale, heads, kvh, D, bs, None), fn)
        torch_mod.cuda.synchronize()
        outs.append([a.cpu().numpy() for a in (X, kc, vc, qo)])
    (x0, k0, v0, q0), (x1, k1, v1, q1) = outs
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1) and np.array_equal(q0, q1)
    assert np.array_equal(x1, qkv) and not np.array_equal(x0, qkv)
    # q_out = fp16(rotated q * q_scale), the product rounded once
    want_q = (x0[:, :Q] * np.float32(q_scale)).astype(np.float16)
    assert np.array_equal(q0.view(np.float16).reshape(T, Q), want_q)
    assert _lib.lib().rh_qkv_post_to_cache(None, 1, None, None, None, None, None, None, None, None, None, 1.0, 8, 2, 64,
                                           16, None) != 0
    assert "q_out is required" in _lib.last_error()
