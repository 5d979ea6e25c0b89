"""Edge cases across the kernels: empty calls, ragged batches, the longest prefill.

- Empty inputs (no decode tokens, no prefill work, T = 0 products) return success and
  write nothing (the output buffers keep their sentinel bytes).
- A ragged decode batch (contexts 1 .. 3000, across block, slice and chunk boundaries)
  in one call, against the CPU oracle at the decode tolerance (2e-3 * max|oracle|).
- Prefill of one 8192-token chunk (32 q / 4 kv heads, D 64; 4x config 3's prompt): the CPU
  oracle takes minutes there, so the checker is a float32 PyTorch attention on the same
  fp16 values (q K^T / sqrt(D), causal mask, softmax, @ V, all fp32) at the same tolerance.
"""
import math

import numpy as np
import pytest

from helpers import PagedCase, bits_to_f32
from test_decode_attention import check_close, oracle_out, run_decode
from test_prefill import chunks_of, run_prefill

pytestmark = pytest.mark.gpu


def test_empty_calls_write_nothing(torch_mod, dev):
    from relay_amd import _lib

    torch = torch_mod
    L = _lib.lib()
    out = torch.full((64,), 0x7BFF, dtype=torch.int16, device=dev)
    y = torch.full((64,), 3.0, device=dev)
    print("empty calls", flush=True)
    # No decode tokens.
    assert L.rh_paged_decode_attention(None, 64, None, None, None, None, 0, 4, 4, 64, 16, 64, 1, 0.125, None, None,
                                       None, out.data_ptr(), 64, None) == 0
    # No prefill work.
    assert L.rh_flash_prefill(None, 64, None, None, None, None, 0, 4, 4, 64, 16, 0.125, out.data_ptr(), 64, None) == 0
    # No tokens for the int8 GEMM.
    assert L.rh_gemm_w8(None, 64, None, None, y.data_ptr(), 0, 64, 64, 0.0, None) == 0
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 0x7BFF).all() and (y.cpu().numpy() == 3.0).all()


@pytest.mark.parametrize("D,heads,kv_heads", [(64, 32, 4), (128, 32, 8)])
def test_ragged_decode_batch(torch_mod, dev, D, heads, kv_heads):
    ctxs = [1, 2, 15, 16, 17, 63, 64, 65, 511, 512, 513, 1023, 1024, 1025, 2047, 3000]
    case = PagedCase(ctxs, 1, heads, kv_heads, D, 16, seed=D + len(ctxs))
    got, _ = run_decode(torch_mod, dev, case)
    check_close(got, oracle_out(case))


def _torch_causal_attention(torch, dev, case):
    """float32 attention of one chunk holding every position 0 .. T-1 of one sequence."""
    H, KVH, D, bs, T = case.heads, case.kv_heads, case.D, case.bs, case.T
    tables = np.array(case.tables, np.int64)
    p = np.arange(T)
    rows = ((tables[p // bs][:, None] * KVH + np.arange(KVH)[None, :]) * bs + (p % bs)[:, None])  # [T, KVH]
    k = bits_to_f32(case.kpool).reshape(-1, D)[rows]  # [T, KVH, D]
    v = bits_to_f32(case.vpool).reshape(-1, D)[rows]
    q = torch.from_numpy(bits_to_f32(case.q).reshape(T, H, D)).to(dev)
    kt, vt = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    out = torch.empty((T, H, D), dtype=torch.float32, device=dev)
    G = H // KVH
    for h in range(H):
        kh, vh = kt[:, h // G, :], vt[:, h // G, :]
        for r0 in range(0, T, 1024):
            qr = q[r0:r0 + 1024, h, :]
            s = (qr @ kh.T) / math.sqrt(D)
            idx = torch.arange(r0, r0 + qr.shape[0], device=dev)[:, None]
            s = s.masked_fill(torch.arange(T, device=dev)[None, :] > idx, float("-inf"))
            out[r0:r0 + qr.shape[0], h, :] = torch.softmax(s, dim=1) @ vh
    torch.cuda.synchronize()
    return out.reshape(T, H * D).cpu().numpy()


def test_prefill_8192_tokens_against_fp32_torch(torch_mod, dev):
    case = PagedCase([8192], [8192], 32, 4, 64, 16, seed=81)
    assert chunks_of(case) == [(0, 8192, 0, 0)]
    got = run_prefill(torch_mod, dev, case)
    want = _torch_causal_attention(torch_mod, dev, case)
    check_close(got, want)


def test_decode_64k_context(torch_mod, dev):
    """One sequence at 65536 keys (D 128, 32 q / 8 kv heads): the planner splits it into
    more slices than one batched merge takes, so the general merge loop runs."""
    from relay_amd import _lib

    case = PagedCase([65536], 1, 32, 8, 128, 16, seed=64)
    slice_keys = _lib.lib().rh_decode_slice_keys(1, 8, 4, 128, 65536)
    assert math.ceil(65536 / slice_keys) > 8
    got, _ = run_decode(torch_mod, dev, case)
    check_close(got, oracle_out(case))
