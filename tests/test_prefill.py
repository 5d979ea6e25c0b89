"""Flash prefill attention (rh_flash_prefill) and the reference attention kernel
(rh_reference_attention) against the CPU oracle.

Each case is a batch of chunks: chunk s holds the last n_new[s] positions of a
sequence of context ctx[s] (a chunk at an offset sees the earlier chunks' keys through
the paged cache, as with relay's chunked prefill). Oracle and tolerance as for decode.
"""
import copy
import math

import numpy as np
import pytest

import oracle as O
from helpers import PagedCase, bits_to_f32, f16_bits

pytestmark = pytest.mark.gpu


def chunks_of(case):
    """(first row, rows, first position, table offset) of each chunk of the case."""
    chunks, t = [], 0
    for s in range(len(case.table_off)):
        n = case.seq.count(s)
        if n:
            chunks.append((t, n, case.pos[t], case.table_off[s]))
        t += n
    return chunks


LN2 = 0.6931471805599453  # scale * log2(e) rounds to exactly 1.0f: q taken as already scaled


def exp2_domain_q(case):
    """The backend's form of q: fp16(fp32(q * scale * log2(e))), as its q writers store it."""
    cl = np.float32(np.float32(1.0 / math.sqrt(case.D)) * np.float32(1.4426950408889634))
    return f16_bits(bits_to_f32(case.q) * cl)


def run_prefill(torch, dev, case, exp2_q=False):
    from relay_amd import _lib

    L = _lib.lib()
    if exp2_q:
        case = copy.copy(case)
        case.q = exp2_domain_q(case)
    d = case.to_device(torch, dev)
    H, KVH, D = case.heads, case.kv_heads, case.D
    work = torch.from_numpy(_lib.prefill_work(chunks_of(case), H)).to(dev)
    out = torch.full((case.T, H * D), float("nan"), dtype=torch.float16, device=dev)
    print(f"prefill case: T={case.T} work={work.shape[0]} H={H} KVH={KVH} D={D} bs={case.bs}", flush=True)
    rc = L.rh_flash_prefill(d["q"].data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(), d["tables"].data_ptr(),
                            work.data_ptr(), work.shape[0], H, KVH, D, case.bs, LN2 if exp2_q else 1.0 / math.sqrt(D),
                            out.data_ptr(),
                            H * D, None)
    _lib.check(rc, "rh_flash_prefill")
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.float32)


def run_reference(torch, dev, case):
    from relay_amd import _lib

    d = case.to_device(torch, dev)
    H, KVH, D = case.heads, case.kv_heads, case.D
    q32 = torch.from_numpy(bits_to_f32(case.q)).to(dev)
    out = torch.full((case.T, H * D), float("nan"), dtype=torch.float16, device=dev)
    rc = _lib.lib().rh_reference_attention(q32.data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(),
                                           d["pos"].data_ptr(), d["seq"].data_ptr(), d["table_off"].data_ptr(),
                                           d["tables"].data_ptr(), None, case.T, H, KVH, D, case.bs,
                                           1.0 / math.sqrt(D), out.data_ptr(), H * D, None)
    _lib.check(rc, "rh_reference_attention")
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.float32)


def oracle_out(case):
    return O.paged_attention(bits_to_f32(case.q), case.heads * case.D, case.kpool, case.vpool, case.meta, None,
                             case.heads, case.kv_heads, case.D, case.bs, 1.0 / math.sqrt(case.D))


def check_close(g, o, tol=2e-3):
    assert np.isfinite(g).all()
    err = np.abs(g - o).max()
    assert err <= tol * np.abs(o).max() + 1e-5, f"max abs err {err}, scale {np.abs(o).max()}"


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (9, 3), (32, 4), (16, 2)])
def test_matches_oracle(torch_mod, dev, D, heads, kv_heads):
    # whole prompts, a chunk at an offset, a 2-token chunk, tiles crossing 128-row bounds
    case = PagedCase([300, 700, 50, 129], [300, 200, 2, 129], heads, kv_heads, D, 16, seed=D + heads)
    check_close(run_prefill(torch_mod, dev, case), oracle_out(case))


@pytest.mark.parametrize("bs", [1, 4, 16, 32, 12])
def test_block_sizes(torch_mod, dev, bs):
    case = PagedCase([257, 90], [200, 90], 8, 2, 64, bs, seed=bs)
    check_close(run_prefill(torch_mod, dev, case), oracle_out(case))


@pytest.mark.parametrize("n", [2, 31, 32, 33, 64, 127, 128, 129, 255, 256, 257, 1300])
def test_chunk_lengths(torch_mod, dev, n):
    case = PagedCase([n, n + 517], [n, n], 8, 1, 128, 16, seed=n)
    check_close(run_prefill(torch_mod, dev, case), oracle_out(case))


def test_config3_shape(torch_mod, dev):
    """BASELINE config 3's prefill: one 2048-token prompt, 32 q / 4 kv heads, D 64."""
    case = PagedCase([2048], [2048], 32, 4, 64, 16, seed=0)
    check_close(run_prefill(torch_mod, dev, case), oracle_out(case))


@pytest.mark.parametrize("D", [16, 32, 64, 128])
def test_exp2_domain_q_matches_oracle(torch_mod, dev, D):
    """The backend's call: q already scaled by softmax scale * log2(e) and scale = ln 2 (a
    unit multiplier inside the kernel), against the oracle on the unscaled q."""
    case = PagedCase([700, 300, 129], [700, 200, 129], 32, 4, D, 16, seed=D + 5)
    check_close(run_prefill(torch_mod, dev, case, exp2_q=True), oracle_out(case))


@pytest.mark.parametrize("D", [64, 128])
def test_paired_blocks(torch_mod, dev, D):
    """A step large enough that rh_prefill_plan pairs light and heavy blocks: an odd block
    count, a chunk at an offset, a ragged last block."""
    case = PagedCase([1300, 900, 40], [1300, 700, 40], 32, 4, D, 16, seed=D + 1)
    check_close(run_prefill(torch_mod, dev, case), oracle_out(case))


def test_gather_is_bit_exact_under_permutation(torch_mod, dev):
    case = PagedCase([400], [400], 8, 2, 64, 16, seed=1)
    a = run_prefill(torch_mod, dev, case)
    # the same rows with the pool's blocks permuted
    rng = np.random.default_rng(7)
    perm = rng.permutation(case.num_blocks)
    be = case.kv_heads * case.bs * case.D
    k2, v2 = np.empty_like(case.kpool), np.empty_like(case.vpool)
    for old, new in enumerate(perm):
        k2[new * be:(new + 1) * be] = case.kpool[old * be:(old + 1) * be]
        v2[new * be:(new + 1) * be] = case.vpool[old * be:(old + 1) * be]
    case.kpool, case.vpool = k2, v2
    case.tables = [int(perm[b]) for b in case.tables]
    case.meta["tables"] = np.array(case.tables, np.int32)
    b = run_prefill(torch_mod, dev, case)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("D", [16, 64, 128, 96])
def test_reference_kernel_matches_oracle(torch_mod, dev, D):
    case = PagedCase([1, 300, 600], [1, 100, 3], 6, 2, D, 16, seed=D)
    check_close(run_reference(torch_mod, dev, case), oracle_out(case))


def test_rejects_unsupported_head_dim(torch_mod, dev):
    from relay_amd import _lib

    rc = _lib.lib().rh_flash_prefill(None, 64, None, None, None, None, 1, 4, 4, 48, 16, 0.1, None, 64, None)
    assert rc != 0 and "head_dim" in _lib.last_error()
