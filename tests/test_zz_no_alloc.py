"""rh_paged_decode_attention_noalloc (static scratch, no allocation) against
rh_paged_decode_attention with caller buffers: the same kernels, so identical bits, on two
calls in a row (the second smaller, so it runs on what the first left in the scratch), and
the size limit is enforced."""
import math

import numpy as np
import pytest

from helpers import PagedCase

pytestmark = pytest.mark.gpu


def _call(torch, dev, case, slice_keys, noalloc):
    from relay_amd import _lib

    L = _lib.lib()
    d = case.to_device(torch, dev)
    H, KVH, D, n = case.heads, case.kv_heads, case.D, case.T
    max_parts = max(math.ceil((p + 1) / slice_keys) for p in case.pos)
    dec = torch.from_numpy(case.dec_meta()).to(dev)
    out = torch.full((n, H * D), float("nan"), dtype=torch.float16, device=dev)
    print(f"no-alloc case: T={n} H={H}/{KVH} D={D} slice={slice_keys} noalloc={noalloc}", flush=True)
    if noalloc:
        rc = L.rh_paged_decode_attention_noalloc(d["q"].data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(),
                                                 dec.data_ptr(), d["tables"].data_ptr(), n, H, KVH, D, case.bs,
                                                 slice_keys, max_parts, 1 / math.sqrt(D), out.data_ptr(), H * D, None)
    else:
        po = torch.empty(n * H * max_parts * D, device=dev)
        pml = torch.empty(n * H * max_parts * 2, device=dev)
        ctr = torch.zeros(n * KVH * ((H // KVH + 15) // 16), dtype=torch.int32, device=dev)
        rc = L.rh_paged_decode_attention(d["q"].data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(),
                                         dec.data_ptr(), d["tables"].data_ptr(), n, H, KVH, D, case.bs, slice_keys,
                                         max_parts, 1 / math.sqrt(D), po.data_ptr(), pml.data_ptr(), ctr.data_ptr(),
                                         out.data_ptr(), H * D, None)
    _lib.check(rc, "decode attention")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_equals_buffered(torch_mod, dev):
    big = PagedCase([2048] * 24 + [3001, 17, 600], 1, 32, 8, 128, 16, seed=21)
    small = PagedCase([1500, 1, 513, 900], 1, 32, 4, 64, 16, seed=22)
    for case, sk in ((big, 512), (small, 256)):
        a = _call(torch_mod, dev, case, sk, noalloc=True)
        b = _call(torch_mod, dev, case, sk, noalloc=False)
        assert np.isfinite(a.astype(np.float32)).all()
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_noalloc_rejects_oversize(torch_mod, dev):
    from relay_amd import _lib

    L = _lib.lib()
    assert L.rh_decode_noalloc_scratch_bytes() == 16 << 20
    # 4 * (16384 + 512 * 32 * 64 * 130) bytes is far above 16 MiB.
    rc = L.rh_paged_decode_attention_noalloc(None, 4096, None, None, None, None, 512, 32, 8, 128, 16, 128, 64,
                                             0.1, None, 4096, None)
    assert rc != 0 and "static scratch" in _lib.last_error()


def test_noalloc_refuses_an_overlapping_call_on_another_stream(torch_mod, dev):
    """While the previous call's stream still has work queued, a call on another stream is
    refused with an error (both would use the GPU's one scratch array); once that stream has
    drained, the other stream's call runs and gives the buffered entry point's bits."""
    from relay_amd import _lib

    torch = torch_mod
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep is not available")
    L = _lib.lib()
    case = PagedCase([700, 1, 513, 1500], 1, 32, 4, 64, 16, seed=23)
    d = case.to_device(torch, dev)
    H, KVH, D, n, sk = case.heads, case.kv_heads, case.D, case.T, 256
    max_parts = max(math.ceil((p + 1) / sk) for p in case.pos)
    dec = torch.from_numpy(case.dec_meta()).to(dev)
    out = torch.full((n, H * D), float("nan"), dtype=torch.float16, device=dev)

    def call(stream):
        return L.rh_paged_decode_attention_noalloc(d["q"].data_ptr(), H * D, d["k"].data_ptr(), d["v"].data_ptr(),
                                                   dec.data_ptr(), d["tables"].data_ptr(), n, H, KVH, D, case.bs, sk,
                                                   max_parts, 1 / math.sqrt(D), out.data_ptr(), H * D,
                                                   stream.cuda_stream)

    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    print("no-alloc overlap guard: busy stream A, then a call on stream B", flush=True)
    with torch.cuda.stream(sa):
        torch.cuda._sleep(200_000_000)  # ~0.1 s of queued work on stream A
    _lib.check(call(sa), "decode attention (no-alloc) on stream A")
    rc = call(sb)
    busy = sa.query() is False
    torch.cuda.synchronize()
    if busy:
        assert rc != 0 and "must not overlap" in _lib.last_error()
    _lib.check(call(sb), "decode attention (no-alloc) on stream B after A drained")
    torch.cuda.synchronize()
    want = _call(torch, dev, case, sk, noalloc=False)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want.view(np.uint16))
