"""Split-context paged decode attention (rh_paged_decode_attention) against the CPU
oracle, plus the bit-exact properties of block-table gathering.

Oracle: oracle.paged_attention, the fp32 arithmetic of relay's CPU backend
(cpu_backend.cpp:152-180) on the same fp16 Q/K/V values. Tolerance: the kernel rounds
the softmax weights and its output to fp16, so |gpu - oracle| <= 2e-3 * max|oracle|
(fp16's unit roundoff is 4.9e-4).
Bit-exact: the same logical cache under any block-table permutation, any block size,
or inside any batch gives identical output bits.
"""
import copy
import math

import numpy as np
import pytest

import oracle as O
from helpers import PagedCase, bits_to_f32, f16_bits

pytestmark = pytest.mark.gpu


LN2 = 0.6931471805599453  # scale * log2(e) rounds to exactly 1.0f: q taken as already scaled


def run_decode(torch, dev, case, slice_keys=None, tokens=None, counters=None, exp2_q=False):
    """slice_keys None: the planner's choice (rh_decode_slice_keys). exp2_q: q in the backend's
    form, fp16(fp32(q * scale * log2(e))), with scale = ln 2."""
    from relay_amd import _lib

    if exp2_q:
        case = copy.copy(case)
        cl = np.float32(np.float32(1.0 / math.sqrt(case.D)) * np.float32(1.4426950408889634))
        case.q = f16_bits(bits_to_f32(case.q) * cl)
    d = case.to_device(torch, dev)
    toks = list(range(case.T)) if tokens is None else tokens
    n = len(toks)
    H, KVH, D = case.heads, case.kv_heads, case.D
    G = H // KVH
    if slice_keys is None:
        slice_keys = _lib.lib().rh_decode_slice_keys(n, KVH, G, D, max(case.pos[t] + 1 for t in toks))
    max_parts = max(1, max(math.ceil((case.pos[t] + 1) / slice_keys) for t in toks))
    dec = torch.from_numpy(case.dec_meta(toks)).to(dev)
    part_o = torch.empty(n * H * max_parts * D, dtype=torch.float32, device=dev)
    part_ml = torch.empty(n * H * max_parts * 2, dtype=torch.float32, device=dev)
    if counters is None:
        counters = torch.zeros(n * KVH * ((G + 15) // 16), dtype=torch.int32, device=dev)
    out = torch.full((case.T, H * D), float("nan"), dtype=torch.float16, device=dev)
    print(f"decode case: T={case.T} H={H} KVH={KVH} D={D} bs={case.bs} slice={slice_keys}", flush=True)
    rc = _lib.lib().rh_paged_decode_attention(
        d["q"].data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(), dec.data_ptr(), d["tables"].data_ptr(), n,
        H, KVH, D, case.bs, slice_keys, max_parts, LN2 if exp2_q else 1.0 / math.sqrt(D), part_o.data_ptr(),
        part_ml.data_ptr(),
        counters.data_ptr(), out.data_ptr(), H * D, None)
    _lib.check(rc, "rh_paged_decode_attention")
    torch.cuda.synchronize()
    res = out.cpu().numpy().astype(np.float32)
    return res[toks], counters


def oracle_out(case, tokens=None):
    toks = list(range(case.T)) if tokens is None else tokens
    return O.paged_attention(bits_to_f32(case.q), case.heads * case.D, case.kpool, case.vpool, case.meta, toks,
                             case.heads, case.kv_heads, case.D, case.bs, 1.0 / math.sqrt(case.D))


def check_close(g, o, tol=2e-3):
    assert np.isfinite(g).all()
    err = np.abs(g - o).max()
    assert err <= tol * np.abs(o).max() + 1e-5, f"max abs err {err}, scale {np.abs(o).max()}"


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(8, 8), (9, 3), (32, 4), (32, 8), (16, 1), (40, 2)])
def test_matches_oracle_heads(torch_mod, dev, D, heads, kv_heads):
    case = PagedCase([1, 37, 512, 513, 1500], 1, heads, kv_heads, D, 16, seed=heads + D)
    g, _ = run_decode(torch_mod, dev, case)
    check_close(g, oracle_out(case))


@pytest.mark.parametrize("D", [16, 32, 64, 128])
def test_exp2_domain_q_matches_oracle(torch_mod, dev, D):
    """The backend's call: q already scaled by softmax scale * log2(e) and scale = ln 2 (a
    unit multiplier inside the kernel), against the oracle on the unscaled q."""
    case = PagedCase([1, 200, 513, 2048, 3001], 1, 32, 8, D, 16, seed=D + 7)
    g, _ = run_decode(torch_mod, dev, case, exp2_q=True)
    check_close(g, oracle_out(case))


@pytest.mark.parametrize("ctx", [1, 2, 15, 16, 17, 31, 32, 33, 127, 128, 129, 511, 512, 513, 1024, 1025, 2048, 3001])
def test_context_lengths(torch_mod, dev, ctx):
    case = PagedCase([ctx, max(1, ctx // 3)], 1, 32, 4, 64, 16, seed=ctx)
    g, _ = run_decode(torch_mod, dev, case)
    check_close(g, oracle_out(case))


@pytest.mark.parametrize("D,slice_keys", [(16, 128), (16, 1024), (32, 128), (32, 384), (32, 2048),
                                          (64, 128), (64, 384), (64, 512), (64, 1024), (64, 2048), (64, 4096),
                                          (128, 64), (128, 192), (128, 512), (128, 1024), (128, 4096)])
def test_slice_sizes(torch_mod, dev, D, slice_keys):
    """Every split of the context (1 to 66 slices; 4 or 8 waves) gives the same attention."""
    case = PagedCase([100, 700, 2100], 1, 16, 2, D, 16, seed=slice_keys)
    g, _ = run_decode(torch_mod, dev, case, slice_keys=slice_keys)
    check_close(g, oracle_out(case))


@pytest.mark.parametrize("D", [16, 64])
@pytest.mark.parametrize("bs", [1, 2, 4, 8, 16, 32, 64, 12])
def test_block_sizes(torch_mod, dev, bs, D):
    case = PagedCase([5, 300, 1030], 1, 8, 2, D, bs, seed=bs)
    g, _ = run_decode(torch_mod, dev, case)
    check_close(g, oracle_out(case))


def _relayout(case, bs, seed):
    """The same logical K/V rows in a new pool with block size bs and a new permutation."""
    new = PagedCase([p + 1 for p in case.pos], 1, case.heads, case.kv_heads, case.D, bs, seed=seed)
    D, KVH = case.D, case.kv_heads
    for s in range(case.T):
        ctx = case.pos[s] + 1
        for p in range(ctx):
            ob = case.tables[case.table_off[s] + p // case.bs]
            nb = new.tables[new.table_off[s] + p // bs]
            for h in range(KVH):
                o0 = ((ob * KVH + h) * case.bs + p % case.bs) * D
                n0 = ((nb * KVH + h) * bs + p % bs) * D
                new.kpool[n0:n0 + D] = case.kpool[o0:o0 + D]
                new.vpool[n0:n0 + D] = case.vpool[o0:o0 + D]
    new.q = case.q.copy()
    return new


@pytest.mark.parametrize("bs", [16, 1, 32])
def test_block_table_gather_is_bit_exact(torch_mod, dev, bs):
    """Any permutation of the pool's blocks and any block size: identical bits."""
    case = PagedCase([600, 77, 1200], 1, 32, 4, 64, 16, seed=3)
    a, _ = run_decode(torch_mod, dev, case, slice_keys=512)
    b, _ = run_decode(torch_mod, dev, _relayout(case, bs, seed=99 + bs), slice_keys=512)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_batch_invariance_is_bit_exact(torch_mod, dev):
    """A sequence alone or in a batch of others: identical bits."""
    case = PagedCase([900, 40, 2049, 513], 1, 32, 8, 128, 16, seed=5)
    together, _ = run_decode(torch_mod, dev, case, slice_keys=512)
    for t in range(case.T):
        alone, _ = run_decode(torch_mod, dev, case, tokens=[t], slice_keys=512)
        assert np.array_equal(alone[0].view(np.uint32), together[t].view(np.uint32))


def test_repeated_calls_reset_counters(torch_mod, dev):
    case = PagedCase([1900, 1300], 1, 32, 4, 64, 16, seed=11)
    a, ctr = run_decode(torch_mod, dev, case, slice_keys=256)
    assert int(ctr.abs().sum().item()) == 0
    b, ctr = run_decode(torch_mod, dev, case, counters=ctr, slice_keys=256)
    c, _ = run_decode(torch_mod, dev, case, counters=ctr, slice_keys=256)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)) and np.array_equal(a.view(np.uint32), c.view(np.uint32))


def test_config2_full_size(torch_mod, dev):
    """32 sequences x 2048 context, 32 q / 4 kv heads, D 64, bs 16."""
    case = PagedCase([2048] * 32, 1, 32, 4, 64, 16, seed=0, extra_blocks=0)
    want = oracle_out(case)
    for sk in (None, 512):
        g, _ = run_decode(torch_mod, dev, case, slice_keys=sk)
        check_close(g, want)


def test_config5_full_size(torch_mod, dev):
    """BASELINE config 5's decode part at full size: 48 sequences x 8192 context, 32 q / 8 kv
    heads, D 128, bs 16 (1.6 GB of K+V for the layer)."""
    case = PagedCase([8192] * 48, 1, 32, 8, 128, 16, seed=5, extra_blocks=0)
    g, _ = run_decode(torch_mod, dev, case)
    check_close(g, oracle_out(case))


def test_rejects_unsupported_shapes(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    rc = L.rh_paged_decode_attention(None, 64, None, None, None, None, 1, 4, 4, 80, 16, 512, 1, 0.1, None, None, None,
                                     None, 64, None)
    assert rc != 0 and "head_dim" in _lib.last_error()
    rc = L.rh_paged_decode_attention(None, 256, None, None, None, None, 1, 4, 4, 64, 16, 100, 1, 0.1, None, None, None,
                                     None, 256, None)
    assert rc != 0 and "slice_keys" in _lib.last_error()


def test_slice_merge_is_stable_over_many_launches(torch_mod, dev):
    """The last-arriving workgroup of each (sequence, kv head) merges the other slices'
    partials through relaxed device-scope accesses ordered only by waiting for its own stores
    before the counter increment. A merge that read a stale partial would change the output
    of some launch: 300 back-to-back launches at config 2's shape with 512-key slices (4
    partials per group) must give the first launch's bits every time, and that must match
    the oracle."""
    from relay_amd import _lib

    torch = torch_mod
    case = PagedCase([2048] * 32, 1, 32, 4, 64, 16, seed=3, extra_blocks=0)
    d = case.to_device(torch, dev)
    H, KVH, D, n, sk = 32, 4, 64, 32, 512
    parts = 4
    dec = torch.from_numpy(case.dec_meta()).to(dev)
    part_o = torch.empty(n * H * parts * D, device=dev)
    part_ml = torch.empty(n * H * parts * 2, device=dev)
    ctr = torch.zeros(n * KVH, dtype=torch.int32, device=dev)
    outs = [torch.empty((n, H * D), dtype=torch.float16, device=dev) for _ in range(2)]
    L = _lib.lib()
    print("decode merge stability: 32 x 2048, 512-key slices, 300 launches", flush=True)

    def launch(out):
        _lib.check(L.rh_paged_decode_attention(d["q"].data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(),
                                               dec.data_ptr(), d["tables"].data_ptr(), n, H, KVH, D, 16, sk, parts,
                                               1.0 / math.sqrt(D), part_o.data_ptr(), part_ml.data_ptr(),
                                               ctr.data_ptr(), out.data_ptr(), H * D, None), "decode")

    launch(outs[0])
    torch.cuda.synchronize()
    check_close(outs[0].cpu().numpy().astype(np.float32), oracle_out(case))
    first = outs[0].clone()
    bad = torch.zeros((), dtype=torch.int32, device=dev)
    for i in range(300):
        launch(outs[1])
        bad += (outs[1].view(torch.int16) != first.view(torch.int16)).any().to(torch.int32)
    torch.cuda.synchronize()
    assert int(bad.item()) == 0, f"{int(bad.item())} of 300 launches differed from the first"
    assert int(ctr.abs().sum().item()) == 0
