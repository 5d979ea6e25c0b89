#!/usr/bin/env python3
"""relay's attention + int8 GEMV hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]

Prints ONE JSON line. Headline: paged split-context decode
attention with the fused log-sum-exp merge, 32 sequences x 2048 context, 32 query / 4 KV
heads, head_dim 64, block size 16, 512-key slices (the config's own split; the slice size
the host planner picks for this shape, rh_decode_slice_keys, is timed beside it as
`decode_attention_planner`), fp16 Q/K/V ~ N(0, 1), block tables a seeded random
permutation of the pool. value = algorithmic bytes per launch
(K + V + Q + O + tables = 67,387,392 B) / average launch time, with inputs resident in
HBM; the K steps rotate over enough pool copies (> 256 MB) that the 256 MB Infinity
Cache cannot hold the working set between launches.

Also reported in the same line: flash prefill attention TFLOP/s (config 3's 2048-token
prompt, 32 / 4 heads, D 64, causal), int8 GEMV GB/s at Llama-3-8B shapes (config 4),
TinyLlama-1.1B decode tok/s at 32 x 2048 (config 3b, whole forward pass), config 1's
SmolLM2-135M 512-token prompt + 128 greedy steps (tok/s), config 5's Llama-3-8B mixed
step (48 decode sequences at 8192 + one 512-token chunk; fp16 and int8 weights), and the
CPU oracle's attention on a bounded sample of config 2 (cpu_baseline).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
METRIC = "decode-attn HBM GB/s (% peak); prefill-attn TFLOP/s (% MFMA); decode tok/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the stream the kernels are launched on."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def run(self, fn, steps, warmup, min_warm_s=0.25):
        """At least `warmup` untimed launches, continued until min_warm_s of sustained launches
        have passed: the GPU's clocks ramp up under load over a few hundred milliseconds, and a
        handful of 20-40 us launches would otherwise be timed at the idle clock."""
        t0 = time.perf_counter()
        i = 0
        while i < warmup or time.perf_counter() - t0 < min_warm_s:
            fn(i)
            i += 1
            if i % 64 == 0:
                self.torch.cuda.synchronize()
        self.torch.cuda.synchronize()
        warmup = self.last_warmup = i
        a = self.torch.cuda.Event(enable_timing=True)
        b = self.torch.cuda.Event(enable_timing=True)
        a.record(self.stream)
        for i in range(steps):
            fn(warmup + i)
        b.record(self.stream)
        self.torch.cuda.synchronize()
        return a.elapsed_time(b) / steps  # ms per step


# ---- config 2: decode attention -------------------------------------------------------

def decode_case(seed, n_seq=32, ctx=2048, heads=32, kvh=4, D=64, bs=16):
    rng = np.random.default_rng(seed)
    per = ctx // bs
    nblocks = n_seq * per
    tables = rng.permutation(nblocks).astype(np.int32)
    return nblocks, tables


def bench_decode(torch, dev, stream, steps, warmup, n_seq=32, ctx=2048, heads=32, kvh=4, D=64, bs=16,
                 slice_keys=None, table_per_copy=True):
    from relay_amd import _lib

    L = _lib.lib()
    per = ctx // bs
    nblocks = n_seq * per
    pool_bytes = 2 * nblocks * kvh * bs * D * 2
    copies = max(2, math.ceil(1.5 * MALL_BYTES / pool_bytes) + 1)
    log(f"decode: {copies} pool copies of {pool_bytes / 1e6:.1f} MB")
    pools = []
    for c in range(copies):
        k = torch.empty(nblocks * kvh * bs * D, dtype=torch.float16, device=dev)
        v = torch.empty_like(k)
        _lib.check(L.rh_fill_normal_f16(k.data_ptr(), k.numel(), 1234, 2 * c, 0.0, 1.0, None))
        _lib.check(L.rh_fill_normal_f16(v.data_ptr(), v.numel(), 1234, 2 * c + 1, 0.0, 1.0, None))
        if table_per_copy or c == 0:
            tab = torch.from_numpy(np.random.default_rng(c).permutation(nblocks).astype(np.int32)).to(dev)
        pools.append((k, v, tab))
    q = torch.empty(n_seq * heads * D, dtype=torch.float16, device=dev)
    _lib.check(L.rh_fill_normal_f16(q.data_ptr(), q.numel(), 1234, 999, 0.0, 1.0, None))
    meta = np.array([[i, ctx, i * per, 0] for i in range(n_seq)], np.int32)
    dec = torch.from_numpy(meta).to(dev)
    if slice_keys is None:
        slice_keys = L.rh_decode_slice_keys(n_seq, kvh, heads // kvh, D, ctx)
    parts = math.ceil(ctx / slice_keys)
    part_o = torch.empty(n_seq * heads * parts * D, dtype=torch.float32, device=dev)
    part_ml = torch.empty(n_seq * heads * parts * 2, dtype=torch.float32, device=dev)
    G = heads // kvh
    counters = torch.zeros(n_seq * kvh * ((G + 15) // 16), dtype=torch.int32, device=dev)
    out = torch.empty(n_seq * heads * D, dtype=torch.float16, device=dev)
    torch.cuda.synchronize()
    sp = stream.cuda_stream

    def step(i):
        k, v, tab = pools[i % copies]
        rc = L.rh_paged_decode_attention(q.data_ptr(), heads * D, k.data_ptr(), v.data_ptr(), dec.data_ptr(),
                                         tab.data_ptr(), n_seq, heads, kvh, D, bs, slice_keys, parts,
                                         1.0 / math.sqrt(D), part_o.data_ptr(), part_ml.data_ptr(),
                                         counters.data_ptr(), out.data_ptr(), heads * D, sp)
        if rc:
            raise RuntimeError(_lib.last_error())

    ms = Timer(torch, stream).run(step, steps, warmup)
    kv_bytes = 2 * n_seq * ctx * kvh * D * 2
    algo = kv_bytes + 2 * n_seq * heads * D * 2 + n_seq * per * 4
    return {"ms": ms, "bytes": algo, "gbs": algo / ms / 1e6, "copies": copies, "slice_keys": slice_keys}


# ---- config 3a: flash prefill attention -----------------------------------------------

def bench_prefill(torch, dev, stream, steps, warmup, S=2048, heads=32, kvh=4, D=64, bs=16):
    from relay_amd import _lib

    L = _lib.lib()
    nblocks = S // bs
    k = torch.empty(nblocks * kvh * bs * D, dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    q = torch.empty(S * heads * D, dtype=torch.float16, device=dev)
    for i, t in enumerate((k, v, q)):
        _lib.check(L.rh_fill_normal_f16(t.data_ptr(), t.numel(), 77, i, 0.0, 1.0, None))
    tab = torch.from_numpy(np.random.default_rng(5).permutation(nblocks).astype(np.int32)).to(dev)
    work = torch.from_numpy(_lib.prefill_work([(0, S, 0, 0)], heads)).to(dev)
    out = torch.empty(S * heads * D, dtype=torch.float16, device=dev)
    sp = stream.cuda_stream

    def step(i):
        rc = L.rh_flash_prefill(q.data_ptr(), heads * D, k.data_ptr(), v.data_ptr(), tab.data_ptr(), work.data_ptr(),
                                work.shape[0], heads, kvh, D, bs, 1.0 / math.sqrt(D), out.data_ptr(), heads * D, sp)
        if rc:
            raise RuntimeError(_lib.last_error())

    ms = Timer(torch, stream).run(step, steps, warmup)
    flops = 4.0 * D * heads * S * (S + 1) / 2
    return {"ms": ms, "flops": flops, "tflops": flops / ms / 1e9}


# ---- config 4: int8 GEMV ---------------------------------------------------------------

GEMV_SHAPES = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]  # (K, N)


def bench_gemv(torch, dev, stream, steps, warmup, Ts=(1, 4, 8)):
    from relay_amd import _lib

    L = _lib.lib()
    res = {}
    sp = stream.cuda_stream
    for K, N in GEMV_SHAPES:
        wbytes = N * K
        copies = max(2, math.ceil(1.5 * MALL_BYTES / wbytes) + 1)
        ws = []
        ldw = L.rh_gemv_int8_row_stride(K)  # the backend's int8 layout
        for c in range(copies):
            w = torch.randint(-127, 128, (N, ldw), dtype=torch.int8, device=dev)
            s = (torch.rand(N, device=dev) * 0.019 + 0.001).half()
            ws.append((w, s))
        for T in Ts:
            x = torch.randn(T, K, device=dev).half()
            y = torch.empty(T, N, device=dev)

            def step(i):
                w, s = ws[i % copies]
                rc = L.rh_gemv_int8(w.data_ptr(), ldw, s.data_ptr(), 1, x.data_ptr(), y.data_ptr(), T, K, N, 0.0, sp)
                if rc:
                    raise RuntimeError(_lib.last_error())

            algo = N * K + 2 * N + 2 * T * K + 4 * T * N
            timer = Timer(torch, stream)
            ms = timer.run(step, steps, warmup)
            res[f"{K}x{N}_T{T}"] = {"us": round(ms * 1e3, 2), "gbs": round(algo / ms / 1e6, 1),
                                    "frac": round(algo / ms / 1e6 / HBM_PEAK_GBS, 3), "warmup": timer.last_warmup}
        del ws
        torch.cuda.empty_cache()
    return res


# ---- config 3b: TinyLlama decode step --------------------------------------------------

def bench_tinyllama_decode(steps, int8=False, n_seq=32, ctx=2048, model="tinyllama"):
    from relay_amd import HipBackend, HipOptions, smollm2_135m, tinyllama_1b
    from relay_amd.backend import ForwardBatch, SeqChunk

    c = smollm2_135m() if model == "smollm2" else tinyllama_1b()
    bs = 16
    per = (ctx + 64 + bs - 1) // bs
    be = HipBackend(None, n_seq * per + 1, bs, max_batch_tokens=512, max_context=per * bs,
                    options=HipOptions(False, int8), config=c, synthetic_seed=0, synthetic_std=0.02)
    be.fill_kv_random(seed=3, std=1.0)
    rng = np.random.default_rng(0)
    times = []
    for r in range(steps + 2):
        batch = ForwardBatch([SeqChunk([int(rng.integers(c.vocab))], ctx + r, list(range(i * per, (i + 1) * per)), True)
                              for i in range(n_seq)])
        t0 = time.perf_counter()
        be.forward(batch)
        wall = (time.perf_counter() - t0) * 1e3
        if r >= 2:
            times.append((wall, be.last_forward_ms()))
    be.close()
    wall = float(np.median([t[0] for t in times]))
    dev_ms = float(np.median([t[1] for t in times]))
    return {"ms_wall": round(wall, 3), "ms_device": round(dev_ms, 3), "tok_s": round(n_seq / wall * 1e3, 1)}


def bench_tinyllama_prefill(steps, S=2048):
    """Config 3(a) as a whole forward pass: one S-token prompt in one chunk through all 22
    layers (attention + rocBLAS GEMMs + layer kernels), synthetic fp16 weights; the dense
    GEMM FLOPs 2 S (params) are reported next to the attention FLOPs."""
    from relay_amd import HipBackend, HipOptions, tinyllama_1b
    from relay_amd.backend import ForwardBatch, SeqChunk

    c = tinyllama_1b()
    bs = 16
    nb = S // bs + 1
    be = HipBackend(None, nb, bs, max_batch_tokens=S, max_context=nb * bs,
                    options=HipOptions(False, False), config=c, synthetic_seed=0, synthetic_std=0.02)
    rng = np.random.default_rng(0)
    times = []
    for r in range(steps + 2):
        batch = ForwardBatch([SeqChunk(rng.integers(0, c.vocab, size=S).tolist(), 0, list(range(nb)), True)])
        t0 = time.perf_counter()
        be.forward(batch)
        wall = (time.perf_counter() - t0) * 1e3
        if r >= 2:
            times.append((wall, be.last_forward_ms()))
    be.close()
    wall = float(np.median([t[0] for t in times]))
    dev_ms = float(np.median([t[1] for t in times]))
    params = c.layers * (c.hidden * (c.q_dim + 2 * c.kv_dim) + c.q_dim * c.hidden +
                         3 * c.hidden * c.intermediate) + c.hidden * c.vocab
    gemm_flops = 2.0 * S * (params - c.hidden * c.vocab) + 2.0 * c.hidden * c.vocab  # lm_head: last row only
    attn_flops = 4.0 * c.head_dim * c.heads * S * (S + 1) / 2 * c.layers
    return {"ms_wall": round(wall, 3), "ms_device": round(dev_ms, 3), "prompt_tok_s": round(S / wall * 1e3, 1),
            "dense_gemm_tflop": round(gemm_flops / 1e12, 2), "attention_tflop": round(attn_flops / 1e12, 3),
            "tflops_device": round((gemm_flops + attn_flops) / dev_ms / 1e9, 1)}


def bench_prefill_chunked(steps, length, int8=False, chunk=512):
    """A length-token TinyLlama prompt in chunk-token chunks, one forward per chunk, as
    relay's attention bench times it (tools/relay_attention_bench.cpp:37-60); wall ms of the
    whole prompt (host included) and device ms summed over the chunks."""
    from relay_amd import HipBackend, HipOptions, tinyllama_1b
    from relay_amd.backend import ForwardBatch, SeqChunk

    c = tinyllama_1b()
    bs = 16
    nb = (length + bs - 1) // bs + 1
    be = HipBackend(None, nb, bs, max_batch_tokens=chunk, max_context=nb * bs, options=HipOptions(False, int8),
                    config=c, synthetic_seed=0, synthetic_std=0.02)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, c.vocab, size=length).tolist()
    walls, devs = [], []
    for r in range(steps + 1):  # the first run warms up
        t0 = time.perf_counter()
        dev = 0.0
        for s0 in range(0, length, chunk):
            be.forward(ForwardBatch([SeqChunk(prompt[s0:s0 + chunk], s0, list(range(nb)), True)]))
            dev += be.last_forward_ms()
        if r:
            walls.append((time.perf_counter() - t0) * 1e3)
            devs.append(dev)
    be.close()
    return {"ms_wall": round(float(np.median(walls)), 3), "ms_device": round(float(np.median(devs)), 3)}


def bench_reference_points(steps=5):
    """The measurement points relay publishes for TinyLlama-1.1B (results/t4/m1-2026-10-04.txt:
    51-59): prefill of 512 and 2048 tokens in 512-token chunks, and decode steps at batch 1, 8
    and 32 and context 512 and 2048, each with fp16 and with int8 weights."""
    out = {}
    for int8 in (False, True):
        tag = "int8" if int8 else "fp16"
        for n in (512, 2048):
            out[f"prefill_{n}_{tag}"] = bench_prefill_chunked(steps, n, int8)
        for ctx in (512, 2048):
            for b in (1, 8, 32):
                r = bench_tinyllama_decode(steps, int8=int8, n_seq=b, ctx=ctx)
                out[f"decode_b{b}_ctx{ctx}_{tag}"] = r
    return out


# ---- config 1: SmolLM2-135M, 512-token prompt + 128 greedy steps --------------------------

def bench_config1(prompt_len=512, new_tokens=128):
    """Greedy generation through relay's batch composition (relay_amd.engine.GreedyEngine)
    on the HIP backend with synthetic device weights; wall clock including the host loop
    (logits to the host, argmax) as relay-generate measures it (relay_generate.cpp:61-96)."""
    from relay_amd import HipBackend, HipOptions, smollm2_135m
    from relay_amd.engine import GreedyEngine

    c = smollm2_135m()
    bs = 16
    nb = (prompt_len + new_tokens) // bs + 2
    be = HipBackend(None, nb, bs, max_batch_tokens=2048, options=HipOptions(False, False), config=c,
                    synthetic_seed=0, synthetic_std=0.02)
    prompt = np.random.default_rng(0).integers(0, c.vocab, size=prompt_len).tolist()
    marks, dev_ms = [], []
    runs = []
    for rep in range(3):  # the first run warms up
        marks.clear()
        dev_ms.clear()

        def seen(rid, i, row):
            marks.append(time.perf_counter())
            dev_ms.append(be.last_forward_ms())

        eng = GreedyEngine(be, nb, bs, 2048, 8, on_logits=seen)
        eng.add(1, prompt, new_tokens)
        t0 = time.perf_counter()
        out = eng.run_all()[1]
        t1 = time.perf_counter()
        assert len(out) == new_tokens
        runs.append((marks[0] - t0, t1 - marks[0], t1 - t0))
    be.close()
    prefill, decode, total = (float(np.median([r[i] for r in runs[1:]])) for i in range(3))
    return {"prompt_ms": round(prefill * 1e3, 2), "decode_tok_s": round((new_tokens - 1) / decode, 1),
            "decode_step_ms_device": round(float(np.median(dev_ms[1:])), 3),
            "total_s": round(total, 4), "gen_tok_s": round(new_tokens / total, 1)}


# ---- config 5: Llama-3-8B mixed step ------------------------------------------------------

def bench_llama3_mixed(steps, int8=False, n_dec=48, ctx=8192, chunk=512):
    """One forward step: n_dec decode sequences at context ctx plus one chunk-token prefill
    chunk at position 0, synthetic fp16 (or int8) device weights and a random KV cache."""
    from relay_amd import HipBackend, HipOptions, llama3_8b
    from relay_amd.backend import ForwardBatch, SeqChunk

    c = llama3_8b()
    bs = 16
    per = (ctx + bs) // bs + 1
    nb = n_dec * per + chunk // bs + 1
    be = HipBackend(None, nb, bs, max_batch_tokens=n_dec + chunk, max_context=per * bs,
                    options=HipOptions(False, int8), config=c, synthetic_seed=0, synthetic_std=0.02)
    be.fill_kv_random(seed=5, std=1.0)
    rng = np.random.default_rng(1)
    ptable = list(range(n_dec * per, n_dec * per + chunk // bs))
    times = []
    for r in range(steps + 2):
        seqs = [SeqChunk([int(rng.integers(c.vocab))], ctx - 1, list(range(i * per, (i + 1) * per)), True)
                for i in range(n_dec)]
        if chunk:
            seqs.append(SeqChunk(rng.integers(0, c.vocab, size=chunk).tolist(), 0, ptable, True))
        t0 = time.perf_counter()
        be.forward(ForwardBatch(seqs))
        wall = (time.perf_counter() - t0) * 1e3
        if r >= 2:
            times.append((wall, be.last_forward_ms()))
    be.close()
    wall = float(np.median([t[0] for t in times]))
    dev_ms = float(np.median([t[1] for t in times]))
    kv = 2 * n_dec * ctx * c.kv_heads * c.head_dim * 2 * c.layers
    roof_ms = (kv + (8.0e9 if int8 else 15.0e9)) / HBM_PEAK_GBS / 1e6
    return {"ms_wall": round(wall, 3), "ms_device": round(dev_ms, 3), "decode_tok_s": round(n_dec / wall * 1e3, 1),
            "roofline_ms": round(roof_ms, 2), "frac_roofline": round(roof_ms / dev_ms, 4)}


def bench_kv_io(steps=5, ctx=8192):
    """The KV-I/O half of the boundary (relay's KVSender / KVReceiver calls): read_kv_layer
    and write_kv_layer of one sequence's blocks (Llama-3-8B layer shape, ctx positions) to
    and from host memory, through the gather/scatter kernels and pinned staging on the copy
    stream. Host-inclusive GB/s of the 2 * blocks * kv_block_bytes moved per call; the round
    trip is checked byte for byte."""
    import dataclasses

    from relay_amd import HipBackend, HipOptions, llama3_8b

    c = dataclasses.replace(llama3_8b(), layers=2)
    bs = 16
    n = ctx // bs + 1
    nb = 2 * n + 7
    be = HipBackend(None, nb, bs, max_batch_tokens=64, config=c, synthetic_seed=0, synthetic_std=0.02,
                    options=HipOptions(False, False))
    be.fill_kv_random(seed=5, std=1.0)
    blocks = np.random.default_rng(3).permutation(nb)[:n].tolist()
    nbytes = 2 * n * be.kv_block_bytes()
    data = be.read_kv_layer(1, blocks)  # into a buffer the caller keeps (as the engine's sender does)
    t0 = time.perf_counter()
    for _ in range(steps):
        be.read_kv_layer(1, blocks, out=data)
    rd = (time.perf_counter() - t0) / steps
    other = np.random.default_rng(4).permutation(nb)[:n].tolist()
    be.write_kv_layer(0, other, data)
    t0 = time.perf_counter()
    for _ in range(steps):
        be.write_kv_layer(0, other, data)
    be.wait_kv_written(0)
    wr = (time.perf_counter() - t0) / steps
    same = bool(np.array_equal(be.read_kv_layer(0, other), data))
    # update_weight (relay_engine_update_tensor's path): one down projection, fp32 -> fp16
    # on the device, from host memory and from a device buffer.
    import torch

    wd = np.random.default_rng(5).standard_normal((c.hidden, c.intermediate)).astype(np.float32)
    be.update_weight("layers.1.w_down", wd)
    t0 = time.perf_counter()
    be.update_weight("layers.1.w_down", wd)
    uh = time.perf_counter() - t0
    wdev = torch.from_numpy(wd).to("cuda:0")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    be.update_weight("layers.1.w_down", wdev)
    ud = time.perf_counter() - t0
    be.close()
    return {"blocks": n, "bytes": nbytes, "read_ms": round(rd * 1e3, 3), "read_gbs": round(nbytes / rd / 1e9, 1),
            "write_ms": round(wr * 1e3, 3), "write_gbs": round(nbytes / wr / 1e9, 1), "round_trip_exact": same,
            "update_weight_fp32_bytes": wd.nbytes, "update_weight_host_gbs": round(wd.nbytes / uh / 1e9, 1),
            "update_weight_device_gbs": round(wd.nbytes / ud / 1e9, 1)}


# ---- CPU baseline ----------------------------------------------------------------------

def cpu_baseline(sample_seqs=8, ctx=2048, heads=32, kvh=4, D=64, bs=16):
    """The CPU oracle's attention (relay's CPU-backend arithmetic) on sample_seqs of
    config 2's 32 sequences, timed on this host; GB/s of the same fp16 K/V bytes."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    rng = np.random.default_rng(0)
    per = ctx // bs
    nb = sample_seqs * per
    k = rng.standard_normal(nb * kvh * bs * D, dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal(nb * kvh * bs * D, dtype=np.float32).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((sample_seqs, heads * D), dtype=np.float32).astype(np.float16).astype(np.float32)
    meta = {"pos": np.full(sample_seqs, ctx - 1, np.int32), "seq": np.arange(sample_seqs, dtype=np.int32),
            "table_off": (np.arange(sample_seqs) * per).astype(np.int32),
            "tables": rng.permutation(nb).astype(np.int32)}
    O.paged_attention(q[:1], heads * D, k, v, {**meta, "pos": meta["pos"][:1]}, None, heads, kvh, D, bs, 0.125)
    reps, t = 0, 0.0
    t0 = time.perf_counter()
    while t < 10.0 and reps < 50:
        O.paged_attention(q, heads * D, k, v, meta, None, heads, kvh, D, bs, 1.0 / math.sqrt(D))
        reps += 1
        t = time.perf_counter() - t0
    per_call = t / reps
    byts = 2 * sample_seqs * ctx * kvh * D * 2
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(byts / per_call / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{sample_seqs} of config 2's 32 sequences (ctx {ctx}, 32q/4kv, D64), {reps} calls, "
                      f"{per_call * 1e3:.1f} ms each"}


def host_cpu():
    """This host's core count (as the OpenMP oracle uses them) and CPU model name (lscpu)."""
    import subprocess

    model = ""
    try:
        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except Exception:  # noqa: BLE001 - lscpu missing: report no name
        pass
    return {"nproc": os.cpu_count(), "omp_threads": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
            "model": model}


def cpu_config1(prompt_len=512, new_tokens=128):
    """Config 1 end to end on the CPU oracle (relay's fp32 CPU backend, OpenMP on this host's
    cores): SmolLM2-135M shape, synthetic fp32 weights, 512-token prompt + 128 greedy steps
    through relay's batch composition."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    from relay_amd import smollm2_135m
    from relay_amd.engine import GreedyEngine
    from relay_amd.model import HostWeights

    c = smollm2_135m()
    bs = 16
    nb = (prompt_len + new_tokens) // bs + 2
    w = HostWeights.synthetic(c, seed=0)
    cpu = O.CpuBackend(w, nb, bs)
    prompt = np.random.default_rng(0).integers(0, c.vocab, size=prompt_len).tolist()
    marks = []
    eng = GreedyEngine(cpu, nb, bs, 2048, 8, on_logits=lambda rid, i, row: marks.append(time.perf_counter()))
    eng.add(1, prompt, new_tokens)
    t0 = time.perf_counter()
    out = eng.run_all()[1]
    t1 = time.perf_counter()
    assert len(out) == new_tokens
    return {"prompt_s": round(marks[0] - t0, 3), "decode_tok_s": round((new_tokens - 1) / (t1 - marks[0]), 2),
            "total_s": round(t1 - t0, 3), "gen_tok_s": round(new_tokens / (t1 - t0), 2)}


def cpu_tinyllama_decode(n_seq=32, ctx=2048, layers=22):
    """Config 3(b) on the CPU oracle: one decode step of n_seq sequences at context ctx
    through all `layers` TinyLlama layers (synthetic fp32 weights); the step alone is timed.
    The cache is left as constructed (zeros): the oracle's work does not depend on the
    values, and writing 2.9 GB of fp32 blocks through the per-block call would take longer
    than the step."""
    import dataclasses

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    from relay_amd import tinyllama_1b
    from relay_amd.backend import ForwardBatch, SeqChunk
    from relay_amd.model import HostWeights

    c = dataclasses.replace(tinyllama_1b(), layers=layers)
    bs = 16
    per = ctx // bs + 1
    w = HostWeights.synthetic(c, seed=0)
    cpu = O.CpuBackend(w, n_seq * per, bs)
    rng = np.random.default_rng(3)
    batch = ForwardBatch([SeqChunk([int(rng.integers(c.vocab))], ctx - 1, list(range(i * per, (i + 1) * per)), True)
                          for i in range(n_seq)])
    times = []
    for _ in range(2):  # the same step twice (it rewrites the same cache slots); the faster counts
        t0 = time.perf_counter()
        cpu.forward(batch)
        times.append((time.perf_counter() - t0) * 1e3)
    ms = min(times)
    return {"layers": layers, "ms": round(ms, 1), "tok_s": round(n_seq / ms * 1e3, 2)}


TRAFFIC_FILE = os.path.join(REPO, "profiles", "decode_attention_config2_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the decode kernel, from the rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE runs summarised in profiles/ (scaled by the copy-kernel calibration there);
    None until that summary exists."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("traffic_bytes_per_launch"):
            return int(float(line.split("=")[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--slice-keys", type=int, default=512,
                    help="keys per split of the headline decode launch (config 2 specifies 512; 0 = the planner's)")
    ap.add_argument("--leg", choices=["prefill", "prefill128", "kvio", "gemv", "config1", "llama3", "llama3int8", "llama3dec",
                                           "llama3decint8", "tinyllama", "tinyllamaprefill", "refpoints"],
                    help="run only this part (for profiling) and print its numbers as one JSON line")
    ap.add_argument("--nseq", type=int, default=32, help="--leg tinyllama: decode batch")
    ap.add_argument("--ctx", type=int, default=2048, help="--leg tinyllama: context")
    ap.add_argument("--model", choices=["tinyllama", "smollm2"], default="tinyllama",
                    help="--leg tinyllama: the model shape (SmolLM2-135M for config 1's layers)")
    ap.add_argument("--int8", action="store_true", help="--leg tinyllama: int8 weights")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device-to-device copy 20 times (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's hot path (decode/prefill attention, int8 GEMV) runs on one "
              "MI355X; the path is not sharded across GPUs in this build", file=sys.stderr)
        sys.exit(2)
    import torch

    from relay_amd import _lib

    _lib.require_device()
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    if args.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": 256 << 20, "launches": 20}))
        return

    if args.leg:
        if args.leg == "prefill":
            r = bench_prefill(torch, dev, stream, args.steps, args.warmup)
        elif args.leg == "prefill128":
            r = bench_prefill(torch, dev, stream, args.steps, args.warmup, heads=32, kvh=8, D=128)
        elif args.leg == "gemv":
            r = bench_gemv(torch, dev, stream, args.steps, args.warmup)
        elif args.leg == "config1":
            r = bench_config1()
        elif args.leg == "tinyllama":
            r = bench_tinyllama_decode(args.steps, int8=args.int8, n_seq=args.nseq, ctx=args.ctx, model=args.model)
        elif args.leg == "refpoints":
            r = bench_reference_points(max(1, min(args.steps, 10)))
        elif args.leg == "tinyllamaprefill":
            r = bench_tinyllama_prefill(args.steps)
        elif args.leg == "kvio":
            r = bench_kv_io(max(1, args.steps))
        elif args.leg.startswith("llama3"):
            r = bench_llama3_mixed(args.steps, int8=args.leg.endswith("int8"),
                                   chunk=0 if args.leg.startswith("llama3dec") else 512)
        print(json.dumps({"leg": args.leg, **r}), flush=True)
        return

    dec = bench_decode(torch, dev, stream, args.steps, args.warmup, slice_keys=args.slice_keys or None)
    log(f"decode attention ({dec['slice_keys']}-key slices): {dec['ms'] * 1e3:.2f} us/launch, {dec['gbs']:.0f} GB/s")
    extra = {}
    plan = bench_decode(torch, dev, stream, args.steps, args.warmup)
    log(f"decode attention (planner, {plan['slice_keys']}-key slices): {plan['ms'] * 1e3:.2f} us/launch, "
        f"{plan['gbs']:.0f} GB/s")
    extra["decode_attention_planner"] = {"slice_keys": plan["slice_keys"], "us": round(plan["ms"] * 1e3, 2),
                                         "gbs": round(plan["gbs"], 1), "frac": round(plan["gbs"] / HBM_PEAK_GBS, 4)}
    if not args.quick:
        pre = bench_prefill(torch, dev, stream, 50, 20)  # enough warmup for the clocks to settle
        log(f"prefill attention: {pre['ms'] * 1e3:.1f} us, {pre['tflops']:.1f} TFLOP/s")
        extra["prefill_attention"] = {"workload": "2048-token causal prefill, 32q/4kv heads, D64 (config 3)",
                                      "us": round(pre["ms"] * 1e3, 2), "tflops": round(pre["tflops"], 1),
                                      "frac_fp16_mfma": round(pre["tflops"] / FP16_PEAK_TFLOPS, 4)}
        extra["gemv_int8"] = bench_gemv(torch, dev, stream, max(20, args.steps // 4), 5)
        log(f"gemv: {extra['gemv_int8']}")
        td = bench_tinyllama_decode(10)
        log(f"tinyllama decode 32x2048: {td}")
        extra["tinyllama_decode_32x2048"] = td
        td8 = bench_tinyllama_decode(10, int8=True)
        extra["tinyllama_decode_32x2048_int8"] = td8
        rp = bench_reference_points(5)
        log(f"relay's TinyLlama measurement points: {rp}")
        extra["tinyllama_reference_points"] = rp
        tp = bench_tinyllama_prefill(5)
        log(f"tinyllama 2048-token prefill forward: {tp}")
        extra["tinyllama_prefill_2048"] = tp
        kv = bench_kv_io(5)
        log(f"KV layer I/O (Llama-3-8B layer, 8192 positions): {kv}")
        extra["kv_layer_io_llama3_8192"] = kv
        c1 = bench_config1()
        log(f"config 1 (SmolLM2 512 + 128 greedy): {c1}")
        extra["smollm2_512_plus_128_greedy"] = c1
        for int8 in (False, True):
            l3 = bench_llama3_mixed(5, int8=int8)
            log(f"llama3-8b mixed step (48 x 8192 decode + 512 chunk){' int8' if int8 else ''}: {l3}")
            extra["llama3_8b_mixed_step" + ("_int8" if int8 else "")] = l3
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline()
        cpu["host"] = host_cpu()
        log(f"cpu baseline (attention): {cpu}")
        if not args.quick:
            c1 = cpu_config1()
            log(f"cpu config 1: {c1}")
            td = cpu_tinyllama_decode()
            log(f"cpu tinyllama 32 x 2048 decode step: {td}")
            cpu["config1_smollm2_512_plus_128"] = c1
            cpu["tinyllama_decode_32x2048"] = td
    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "paged decode attention, 32 seqs x 2048 ctx, 32q/4kv heads, D64, bs16, split "
                               "context + fused LSE merge (BASELINE config 2)",
                   "slice_keys": dec["slice_keys"], "pool_copies": dec["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
