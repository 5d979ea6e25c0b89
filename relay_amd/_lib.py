"""ctypes binding of librelay_hip.so (the C ABI in include/relay_hip.h).

Loading never falls back to anything: if the library is missing, or a call is made on a
machine without a usable HIP device, an error is raised. There is no CPU path in this
package.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# RELAY_HIP_LIB selects another build of the library (A/B measurements); default: the in-tree one.
LIB_PATH = os.environ.get("RELAY_HIP_LIB") or os.path.join(HERE, "librelay_hip.so")


class RelayHipError(RuntimeError):
    pass


class ModelConfigC(C.Structure):
    """rh_model_config (include/relay_hip.h)."""
    _fields_ = [(n, C.c_int) for n in ("hidden", "intermediate", "layers", "heads", "kv_heads", "head_dim", "vocab",
                                       "tie_embeddings", "qkv_bias", "rope_scaling_llama3")] + \
               [(n, C.c_double) for n in ("rms_eps", "rope_theta", "rope_factor", "rope_low_freq_factor",
                                          "rope_high_freq_factor", "rope_original_max_position")]


class HostWeightsC(C.Structure):
    _fields_ = [("embed", C.c_void_p), ("final_norm", C.c_void_p), ("lm_head", C.c_void_p),
                ("attn_norm", C.c_void_p), ("wqkv", C.c_void_p), ("bqkv", C.c_void_p), ("wo", C.c_void_p),
                ("mlp_norm", C.c_void_p), ("w_gate_up", C.c_void_p), ("w_down", C.c_void_p)]


class BackendOptionsC(C.Structure):
    _fields_ = [("reference_attention", C.c_int), ("int8_weights", C.c_int)]


P = C.c_void_p
I = C.c_int
I64 = C.c_int64
F = C.c_float
SZ = C.c_size_t
U64 = C.c_uint64
IP = C.POINTER(C.c_int)

# name -> (restype, argtypes)
SIGNATURES = {
    "rh_last_error": (C.c_char_p, []),
    "rh_device_available": (I, []),
    "rh_paged_decode_attention": (I, [P, I64, P, P, P, P, I, I, I, I, I, I, I, F, P, P, P, P, I64, P]),
    "rh_paged_decode_attention_noalloc": (I, [P, I64, P, P, P, P, I, I, I, I, I, I, I, F, P, I64, P]),
    "rh_decode_noalloc_scratch_bytes": (SZ, []),
    "rh_decode_chunk_keys": (I, [I]),
    "rh_decode_slice_keys": (I, [I, I, I, I, I]),
    "rh_flash_prefill": (I, [P, I64, P, P, P, P, I, I, I, I, I, F, P, I64, P]),
    "rh_prefill_plan": (I, [P, P, P, P, I, I, P, I]),
    "rh_prefill_tile_rows": (I, []),
    "rh_reference_attention": (I, [P, I64, P, P, P, P, P, P, P, I, I, I, I, I, F, P, I64, P]),
    "rh_gemv_int8": (I, [P, I64, P, I, P, P, I, I, I, F, P]),
    "rh_gemv_int8_rmsnorm": (I, [P, I64, P, I, P, P, F, P, I, I, I, F, P]),
    "rh_gemv_int8_silu": (I, [P, I64, P, I, P, P, I, I, I, F, P]),
    "rh_gemv_int8_gate_up_silu": (I, [P, I64, P, I, P, P, I, I, I, P]),
    "rh_gemv_f16_gate_up_silu": (I, [P, I64, P, P, I, I, I, P]),
    "rh_gemv_int8_rmsnorm_gate_up_silu": (I, [P, I64, P, I, P, P, F, P, I, I, I, P]),
    "rh_gemv_int8_qkv": (I, [P, I64, P, I, P, P, I, I, P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "rh_gemv_int8_rmsnorm_qkv": (I, [P, I64, P, I, P, P, F, P, I, I, P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "rh_gemv_int8_row_stride": (I64, [I]),
    "rh_gemv_f16": (I, [P, I64, P, P, I, I, I, F, P]),
    "rh_gemv_f16_splitk": (I, [P, I64, P, P, I, I, I, F, I, P, P, P]),
    "rh_gemv_f16_split_plan": (I, [I, I, I]),
    "rh_gemv_f16_max_tokens": (I, []),
    "rh_gemm_w8": (I, [P, I64, P, P, P, I, I, I, F, P]),
    "rh_gemm_w8_skinny": (I, [P, I64, P, P, P, I, I, I, F, I, P, P]),
    "rh_gemm_w8_split": (I, [P, I64, P, P, P, I, I, I, F, I, P, P]),
    "rh_gemm_w8_partials": (I, [P, I64, P, I, I, I, I, P, P]),
    "rh_w8_merge_silu": (I, [P, I, I, I, P, P, P]),
    "rh_w8_merge_rmsnorm": (I, [P, I, I, I, P, P, P, F, P, P]),
    "rh_w8_merge_rmsnorm_fits": (I, [I]),
    "rh_gemm_w8_plan": (I, [I, I, I]),
    "rh_gemm_w8_partials_plan": (I, [I, I, I]),
    "rh_gemm_w8_kernel": (I, [I, I, I, I]),
    "rh_gemm_w8_gate_up_silu": (I, [P, I64, P, P, P, I, I, I, P]),
    "rh_gemm_w8_split_plan": (I, [I, I, I]),
    "rh_gemv_f16_rmsnorm": (I, [P, I64, P, P, F, P, I, I, I, F, P]),
    "rh_gemv_f16_silu": (I, [P, I64, P, P, I, I, I, F, P]),
    "rh_gemv_f16_fused_fits": (I, [I, I]),
    "rh_gemv_f16_rmsnorm_qkv": (I, [P, I64, P, P, F, P, I, I, P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "rh_gemv_f16_qkv": (I, [P, I64, P, P, I, I, P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "rh_gemv_int8_max_tokens": (I, []),
    "rh_quantize_int8": (I, [P, I, I, P, I64, P, P]),
    "rh_dequant_int8": (I, [P, I64, P, I, I, P, P]),
    "rh_f32_to_f16": (I, [P, P, SZ, P]),
    "rh_embed": (I, [P, I, P, I, P, P]),
    "rh_rmsnorm": (I, [P, P, I, P, I, F, P, P]),
    "rh_qkv_post": (I, [P, I, P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "rh_qkv_post_to_cache": (I, [P, I, P, P, P, P, P, P, P, P, P, F, I, I, I, I, P]),
    "rh_silu_mul": (I, [P, I, I, P, P]),
    "rh_kv_gather": (I, [P, P, P, I, SZ, P, P]),
    "rh_kv_scatter": (I, [P, P, P, I, SZ, P, P]),
    "rh_fill_normal_f16": (I, [P, SZ, U64, U64, F, F, P]),
    "rh_fill_normal_f32": (I, [P, SZ, U64, U64, F, F, P]),
    "rh_synth_normal_f32": (None, [P, SZ, U64, U64, F, F]),
    "rh_backend_options_from_env": (BackendOptionsC, []),
    "relay_hip_backend_new": (P, [C.POINTER(ModelConfigC), C.POINTER(HostWeightsC), I, I, I, I, I,
                                  C.POINTER(BackendOptionsC)]),
    "relay_hip_backend_new_synthetic": (P, [C.POINTER(ModelConfigC), U64, F, I, I, I, I, I,
                                            C.POINTER(BackendOptionsC)]),
    "relay_hip_backend_free": (None, [P]),
    "relay_hip_backend_forward": (I, [P, I, IP, IP, IP, IP, IP, IP, I, P, SZ]),
    "relay_hip_backend_kv_block_bytes": (SZ, [P]),
    "relay_hip_backend_read_kv_block": (I, [P, I, I, P, P]),
    "relay_hip_backend_write_kv_block": (I, [P, I, I, P, P]),
    "relay_hip_backend_read_kv_layer": (I, [P, I, IP, I, P]),
    "relay_hip_backend_write_kv_layer": (I, [P, I, IP, I, P]),
    "relay_hip_backend_wait_kv_written": (I, [P, I]),
    "relay_hip_backend_update_weight": (I, [P, C.c_char_p, P, SZ]),
    "relay_hip_backend_fill_kv_random": (I, [P, U64, F]),
    "relay_hip_backend_last_forward_ms": (C.c_double, [P]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RelayHipError(f"{LIB_PATH} is missing: run `python -m relay_amd.build` (no CPU fallback exists)")
        l = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def last_error() -> str:
    return (lib().rh_last_error() or b"").decode()


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise RelayHipError(f"{what}: {last_error()} (code {rc})")


def require_device() -> None:
    if not lib().rh_device_available():
        raise RelayHipError("no HIP device: relay_amd runs only on the GPU")


def prefill_work(chunks, heads: int):
    """rh_prefill_plan over chunks = [(first row, rows, first position, table offset), ...];
    returns the int32 work records as a numpy array of shape (n_work, 8)."""
    import numpy as np

    cols = [np.ascontiguousarray([c[i] for c in chunks], dtype=np.int32) for i in range(4)]
    cap = len(chunks) + sum(c[1] for c in chunks) // lib().rh_prefill_tile_rows() + 1
    work = np.zeros((cap, 8), dtype=np.int32)
    n = lib().rh_prefill_plan(*[c.ctypes.data for c in cols], len(chunks), heads, work.ctypes.data, cap)
    check(n if n < 0 else 0, "rh_prefill_plan")
    return work[:n].copy()
