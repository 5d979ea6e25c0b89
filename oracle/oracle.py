"""TEST INFRASTRUCTURE ONLY: Python binding of the CPU oracle (liboracle.so, built from
cpu_oracle.cpp) and of the reference CPU backend built from /root/reference
(_ref/librelay_ref.so, present only where that tree was available at build time).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
as the checker or the timed CPU baseline. The product (relay_amd) never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "librelay_ref.so")

P, I, F, D, SZ = C.c_void_p, C.c_int, C.c_float, C.c_double, C.c_size_t
IP = C.POINTER(C.c_int)

_o = None
_r = None


def lib() -> C.CDLL:
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"{ORACLE_LIB} is missing: run `make -C oracle`")
        l = C.CDLL(ORACLE_LIB)
        sig = {
            "oracle_last_error": (C.c_char_p, []),
            "oracle_model_new": (P, [P, P, P, P, P, P, P, P, P, P, P, I, I]),
            "oracle_model_free": (None, [P]),
            "oracle_forward": (I, [P, I, IP, IP, IP, IP, IP, IP, I, P, SZ]),
            "oracle_read_kv_block": (I, [P, I, I, P, P]),
            "oracle_write_kv_block": (I, [P, I, I, P, P]),
            "oracle_rope_inv_freq": (I, [P, P]),
            "oracle_f32_to_f16": (None, [P, P, SZ]),
            "oracle_f16_to_f32": (None, [P, P, SZ]),
            "oracle_round_f16_inplace": (None, [P, SZ]),
            "oracle_quantize_int8": (None, [P, I, I, P, P]),
            "oracle_paged_attention": (None, [P, C.c_long, P, P, P, P, P, P, P, I, I, I, I, I, F, P]),
            "oracle_paged_attention_f64": (None, [P, C.c_long, P, P, P, P, P, P, P, I, I, I, I, I, D, P]),
            "oracle_gemv_int8": (None, [P, P, P, I, I, I, D, P, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(l, name)
            f.restype, f.argtypes = res, args
        _o = l
    return _o


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref_lib() -> C.CDLL:
    global _r
    if _r is None:
        l = C.CDLL(REF_LIB)
        sig = {
            "ref_last_error": (C.c_char_p, []),
            "ref_model_load": (P, [C.c_char_p, I, I]),
            "ref_model_free": (None, [P]),
            "ref_model_vocab": (I, [P]),
            "ref_forward": (I, [P, I, IP, IP, IP, IP, IP, IP, I, P, SZ]),
            "ref_generate": (I, [P, IP, I, I, I, IP, P]),
            "ref_f32_to_f16": (None, [P, P, SZ]),
            "ref_rope_inv_freq": (I, [P, P]),
            "ref_write_kv_block": (I, [P, I, I, P, P]),
            "ref_weight": (C.c_long, [P, C.c_char_p, P, SZ]),
        }
        for name, (res, args) in sig.items():
            f = getattr(l, name)
            f.restype, f.argtypes = res, args
        _r = l
    return _r


def _flat(batch):
    S = len(batch.seqs)
    tokens = [t for s in batch.seqs for t in s.tokens]
    tables = [b for s in batch.seqs for b in s.block_table]
    arr = lambda xs: (C.c_int * max(len(xs), 1))(*xs)
    rows = len(tokens) if batch.all_logits else sum(1 for s in batch.seqs if s.want_logits and s.tokens)
    return (S, arr([len(s.tokens) for s in batch.seqs]), arr(tokens), arr([s.start_pos for s in batch.seqs]),
            arr([len(s.block_table) for s in batch.seqs]), arr(tables), arr([int(s.want_logits) for s in batch.seqs]),
            rows)


class CpuBackend:
    """The fp32 CPU oracle behind the same forward / KV-block surface as HipBackend
    (relay's make_cpu_backend). Borrows the HostWeights' arrays: keep them alive."""

    def __init__(self, weights, num_blocks: int, block_size: int):
        self.w = weights
        c = weights.config
        self._cfg = c.to_c()
        self._hw, self._keep = weights.c_views()
        hw = self._hw
        self._h = lib().oracle_model_new(C.byref(self._cfg), hw.embed, hw.final_norm, hw.lm_head, hw.attn_norm,
                                         hw.wqkv, hw.bqkv, hw.wo, hw.mlp_norm, hw.w_gate_up, hw.w_down, num_blocks,
                                         block_size)
        if not self._h:
            raise RuntimeError(lib().oracle_last_error().decode())
        self.block_elems = c.kv_heads * block_size * c.head_dim

    def __del__(self):
        if getattr(self, "_h", None):
            lib().oracle_model_free(self._h)
            self._h = None

    def config(self):
        return self.w.config

    def name(self) -> str:
        return "cpu"

    def forward(self, batch) -> np.ndarray:
        S, nt, tok, sp, tl, tab, want, rows = _flat(batch)
        V = self.w.config.vocab
        out = np.empty((rows, V), np.float32)
        got = lib().oracle_forward(self._h, S, nt, tok, sp, tl, tab, want, int(batch.all_logits), out.ctypes.data,
                                   out.size)
        if got < 0:
            msg = lib().oracle_last_error().decode()
            raise (IndexError if "token id" in msg else ValueError)(msg)
        return out[:got]

    def read_kv_block(self, layer: int, block: int):
        k = np.empty(self.block_elems, np.float32)
        v = np.empty(self.block_elems, np.float32)
        lib().oracle_read_kv_block(self._h, layer, block, k.ctypes.data, v.ctypes.data)
        return k, v

    def write_kv_block(self, layer: int, block: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        lib().oracle_write_kv_block(self._h, layer, block, k.ctypes.data, v.ctypes.data)


class RefBackend:
    """The reference's own CpuBackend (compiled from /root/reference), loaded from a
    Hugging Face model directory with the reference's loader."""

    def __init__(self, model_dir: str, num_blocks: int, block_size: int):
        self._h = ref_lib().ref_model_load(model_dir.encode(), num_blocks, block_size)
        if not self._h:
            raise RuntimeError(ref_lib().ref_last_error().decode())
        self.vocab = ref_lib().ref_model_vocab(self._h)

    def __del__(self):
        if getattr(self, "_h", None):
            ref_lib().ref_model_free(self._h)
            self._h = None

    def forward(self, batch) -> np.ndarray:
        S, nt, tok, sp, tl, tab, want, rows = _flat(batch)
        out = np.empty((rows, self.vocab), np.float32)
        got = ref_lib().ref_forward(self._h, S, nt, tok, sp, tl, tab, want, int(batch.all_logits), out.ctypes.data,
                                    out.size)
        if got < 0:
            raise RuntimeError(ref_lib().ref_last_error().decode())
        return out[:got]

    def generate(self, prompt: list, max_new: int, max_batch_tokens: int = 2048):
        toks = (C.c_int * max_new)()
        logits = np.empty((max_new, self.vocab), np.float32)
        p = (C.c_int * len(prompt))(*prompt)
        n = ref_lib().ref_generate(self._h, p, len(prompt), max_new, max_batch_tokens, toks, logits.ctypes.data)
        if n < 0:
            raise RuntimeError(ref_lib().ref_last_error().decode())
        return list(toks[:n]), logits[:n]

    def write_kv_block(self, layer: int, block: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        if ref_lib().ref_write_kv_block(self._h, layer, block, k.ctypes.data, v.ctypes.data) != 0:
            raise RuntimeError(ref_lib().ref_last_error().decode())

    def rope_inv_freq(self, half: int) -> np.ndarray:
        out = np.empty(half, np.float32)
        ref_lib().ref_rope_inv_freq(self._h, out.ctypes.data)
        return out

    def weight(self, name: str) -> np.ndarray:
        n = ref_lib().ref_weight(self._h, name.encode(), None, 0)
        out = np.empty(max(n, 0), np.float32)
        ref_lib().ref_weight(self._h, name.encode(), out.ctypes.data, out.size)
        return out


# ---- op-level oracles ------------------------------------------------------------------

def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16(x.ctypes.data, out.ctypes.data, x.size)
    return out


def round_f16_inplace(a: np.ndarray) -> np.ndarray:
    """a <- fp16(a) as fp32 values (round to nearest even), in place; a is C-contiguous fp32."""
    assert a.dtype == np.float32 and a.flags.c_contiguous
    lib().oracle_round_f16_inplace(a.ctypes.data, a.size)
    return a


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32(h.ctypes.data, out.ctypes.data, h.size)
    return out


def rope_inv_freq(config) -> np.ndarray:
    out = np.empty(config.head_dim // 2, np.float32)
    cfg = config.to_c()
    lib().oracle_rope_inv_freq(C.byref(cfg), out.ctypes.data)
    return out


def quantize_int8(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    lib().oracle_quantize_int8(w.ctypes.data, N, K, q.ctypes.data, s.ctypes.data)
    return q, s


def _meta_ptrs(meta):
    return [np.ascontiguousarray(meta[k], np.int32) for k in ("pos", "seq", "table_off", "tables")]


def paged_attention(q, q_stride, kpool, vpool, meta, tokens, heads, kv_heads, D, block_size, scale, f64=False):
    """Attention of the listed tokens over a paged cache (fp16 bits as uint16, or fp32): the CPU
    backend's arithmetic (fp32), or a double-precision brute force (f64=True).
    q: float32 rows (fp16 values widened, for comparing with kernels that read fp16 q)."""
    q = np.ascontiguousarray(q, np.float32)
    pos, seq, toff, tabs = _meta_ptrs(meta)
    toks = None if tokens is None else np.ascontiguousarray(tokens, np.int32)
    n = len(toks) if toks is not None else len(pos)
    # fp16 pools (uint16 bits) widen exactly; fp32 pools are used as they are
    widen = lambda a: a.view(np.float16).astype(np.float32) if a.dtype == np.uint16 else np.ascontiguousarray(a, np.float32)
    kp, vp = widen(np.ascontiguousarray(kpool)), widen(np.ascontiguousarray(vpool))
    tp = toks.ctypes.data if toks is not None else None
    if f64:
        out = np.empty((n, heads * D), np.float64)
        lib().oracle_paged_attention_f64(q.ctypes.data, q_stride, kp.ctypes.data, vp.ctypes.data, pos.ctypes.data,
                                         seq.ctypes.data, toff.ctypes.data, tabs.ctypes.data, tp, n, heads,
                                         kv_heads, D, block_size, float(scale), out.ctypes.data)
    else:
        out = np.empty((n, heads * D), np.float32)
        lib().oracle_paged_attention(q.ctypes.data, q_stride, kp.ctypes.data, vp.ctypes.data, pos.ctypes.data,
                                     seq.ctypes.data, toff.ctypes.data, tabs.ctypes.data, tp, n, heads, kv_heads, D,
                                     block_size, float(scale), out.ctypes.data)
    return out


def gemv_int8(w8, scale, x_f16, beta=0.0, y0=None):
    w8 = np.ascontiguousarray(w8, np.int8)
    N, K = w8.shape
    x = np.ascontiguousarray(x_f16, np.uint16)
    T = x.shape[0]
    s = np.ascontiguousarray(scale, np.float32)
    y = np.empty((T, N), np.float64)
    y0p = np.ascontiguousarray(y0, np.float32).ctypes.data if y0 is not None else None
    lib().oracle_gemv_int8(w8.ctypes.data, s.ctypes.data, x.ctypes.data, T, K, N, float(beta), y0p, y.ctypes.data)
    return y
