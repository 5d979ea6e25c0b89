"""relay's backend interface in Python over the HIP backend's C ABI.

SeqChunk / ForwardBatch / the Backend methods mirror relay's C++ boundary
(engine/include/relay/backend.h:22-98): forward(batch) returns float32 logits
[rows, vocab], one row per chunk with want_logits (or per token with all_logits);
KV blocks move as bytes in the cache's dtype (fp16 here); update_weight takes relay's
tensor names. Errors surface as exceptions, the way relay's C++ backends raise them.
"""
from __future__ import annotations

import ctypes as C
import itertools
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .model import HostWeights, ModelConfig


@dataclass
class SeqChunk:
    tokens: list
    start_pos: int = 0
    block_table: list = field(default_factory=list)
    want_logits: bool = True


@dataclass
class ForwardBatch:
    seqs: list = field(default_factory=list)
    all_logits: bool = False


@dataclass
class HipOptions:
    """relay's CudaOptions for the HIP backend (backend.h:85-94)."""
    reference_attention: bool = False
    int8_weights: bool = False

    @classmethod
    def from_env(cls) -> "HipOptions":
        o = _lib.lib().rh_backend_options_from_env()
        return cls(bool(o.reference_attention), bool(o.int8_weights))

    def to_c(self) -> _lib.BackendOptionsC:
        return _lib.BackendOptionsC(int(self.reference_attention), int(self.int8_weights))


def flatten(batch: ForwardBatch):
    """The C ABI's flat batch encoding: per-chunk counts plus concatenated arrays (int32
    numpy arrays, built without intermediate Python lists: a 32-sequence decode batch with
    2048-position block tables flattens in ~0.05 ms)."""
    seqs = batch.seqs
    S = len(seqs)
    n_tokens = np.fromiter((len(s.tokens) for s in seqs), np.int32, S)
    tlen = np.fromiter((len(s.block_table) for s in seqs), np.int32, S)
    tok = np.fromiter(itertools.chain.from_iterable(s.tokens for s in seqs), np.int32, int(n_tokens.sum()))
    tab = np.fromiter(itertools.chain.from_iterable(s.block_table for s in seqs), np.int32, int(tlen.sum()))
    start = np.fromiter((s.start_pos for s in seqs), np.int32, S)
    want = np.fromiter((bool(s.want_logits) for s in seqs), np.int32, S)
    rows = len(tok) if batch.all_logits else sum(1 for s in seqs if s.want_logits and s.tokens)
    return S, n_tokens, tok, start, tlen, tab, want, rows


def _ip(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int))


class HipBackend:
    """make_hip_backend(weights, num_blocks, block_size, device, max_batch_tokens,
    max_context, options): the model's weights are copied to the GPU; the KV cache
    (num_blocks blocks of block_size positions per layer) lives in HBM."""

    def __init__(self, weights: HostWeights | None, num_blocks: int, block_size: int, device: int = 0,
                 max_batch_tokens: int = 2048, max_context: int | None = None, options: HipOptions | None = None,
                 *, config: ModelConfig | None = None, synthetic_seed: int | None = None,
                 synthetic_std: float = 0.02):
        l = _lib.lib()
        _lib.require_device()
        self._config = weights.config if weights is not None else config
        self.num_blocks, self.block_size = num_blocks, block_size
        max_context = num_blocks * block_size if max_context is None else max_context
        opts = (options or HipOptions.from_env()).to_c()
        cfg = self._config.to_c()
        if weights is not None:
            hw, keep = weights.c_views()
            self._h = l.relay_hip_backend_new(C.byref(cfg), C.byref(hw), num_blocks, block_size, device,
                                              max_batch_tokens, max_context, C.byref(opts))
            del keep
        else:
            self._h = l.relay_hip_backend_new_synthetic(C.byref(cfg), synthetic_seed or 0, synthetic_std,
                                                        num_blocks, block_size, device, max_batch_tokens,
                                                        max_context, C.byref(opts))
        if not self._h:
            raise _lib.RelayHipError(f"make_hip_backend: {_lib.last_error()}")

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.lib().relay_hip_backend_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- relay's Backend surface -----------------------------------------------------

    def config(self) -> ModelConfig:
        return self._config

    def name(self) -> str:
        return "hip"

    def kv_block_bytes(self) -> int:
        return _lib.lib().relay_hip_backend_kv_block_bytes(self._h)

    def forward(self, batch: ForwardBatch) -> np.ndarray:
        S, n_tokens, tok, start, tlen, tab, want, rows = flatten(batch)
        V = self._config.vocab
        out = np.empty((rows, V), dtype=np.float32)
        got = _lib.lib().relay_hip_backend_forward(self._h, S, _ip(n_tokens), _ip(tok), _ip(start), _ip(tlen), _ip(tab),
                                                   _ip(want), int(batch.all_logits), out.ctypes.data, out.size)
        if got < 0:
            raise _translate(_lib.last_error())
        return out[:got]

    def read_kv_block(self, layer: int, block: int):
        bb = self.kv_block_bytes()
        k, v = np.empty(bb, np.uint8), np.empty(bb, np.uint8)
        _lib.check(_lib.lib().relay_hip_backend_read_kv_block(self._h, layer, block, k.ctypes.data, v.ctypes.data),
                   "read_kv_block")
        return k, v

    def write_kv_block(self, layer: int, block: int, k: np.ndarray, v: np.ndarray) -> None:
        k, v = np.ascontiguousarray(k), np.ascontiguousarray(v)
        _lib.check(_lib.lib().relay_hip_backend_write_kv_block(self._h, layer, block, k.ctypes.data, v.ctypes.data),
                   "write_kv_block")

    def read_kv_layer(self, layer: int, blocks: list, out: np.ndarray | None = None) -> np.ndarray:
        """All K blocks, then all V blocks (relay's read_kv_layer layout); into `out` (uint8,
        C-contiguous, the right size) when given, else a new array."""
        nbytes = 2 * len(blocks) * self.kv_block_bytes()
        if out is None:
            out = np.empty(nbytes, np.uint8)
        elif out.dtype != np.uint8 or out.nbytes != nbytes or not out.flags["C_CONTIGUOUS"]:
            raise ValueError("read_kv_layer: out must be a C-contiguous uint8 array of 2 * blocks * kv_block_bytes")
        ids = (C.c_int * max(len(blocks), 1))(*blocks)
        _lib.check(_lib.lib().relay_hip_backend_read_kv_layer(self._h, layer, ids, len(blocks), out.ctypes.data),
                   "read_kv_layer")
        return out

    def write_kv_layer(self, layer: int, blocks: list, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        ids = (C.c_int * max(len(blocks), 1))(*blocks)
        _lib.check(_lib.lib().relay_hip_backend_write_kv_layer(self._h, layer, ids, len(blocks), data.ctypes.data),
                   "write_kv_layer")

    def wait_kv_written(self, layer: int) -> None:
        _lib.check(_lib.lib().relay_hip_backend_wait_kv_written(self._h, layer), "wait_kv_written")

    def update_weight(self, name: str, src) -> None:
        """src: a host float32 array, or a torch CUDA tensor (device memory of any GPU)."""
        if hasattr(src, "data_ptr"):
            ptr, n = src.data_ptr(), src.numel()
        else:
            src = np.ascontiguousarray(src, dtype=np.float32)
            ptr, n = src.ctypes.data, src.size
        rc = _lib.lib().relay_hip_backend_update_weight(self._h, name.encode(), ptr, n)
        if rc:
            raise _translate(_lib.last_error())

    # ---- benchmark helpers -------------------------------------------------------------

    def fill_kv_random(self, seed: int = 0, std: float = 1.0) -> None:
        _lib.check(_lib.lib().relay_hip_backend_fill_kv_random(self._h, seed, std), "fill_kv_random")

    def last_forward_ms(self) -> float:
        return _lib.lib().relay_hip_backend_last_forward_ms(self._h)


def _translate(msg: str) -> Exception:
    """The C++ exception classes map onto Python's (relay's error conventions)."""
    if "token id out of range" in msg:
        return IndexError(msg)
    if "update_weight: int8" in msg:
        return RuntimeError(msg)
    if any(s in msg for s in ("block table too short", "max_context", "max_batch_tokens", "block id", "update_weight",
                              "wrong size", "no backend", "logits buffer", "cannot want logits")):
        return ValueError(msg)
    return _lib.RelayHipError(msg)


def make_hip_backend(weights: HostWeights, num_blocks: int, block_size: int, device: int = 0,
                     max_batch_tokens: int = 2048, max_context: int | None = None,
                     options: HipOptions | None = None) -> HipBackend:
    return HipBackend(weights, num_blocks, block_size, device, max_batch_tokens, max_context, options)
