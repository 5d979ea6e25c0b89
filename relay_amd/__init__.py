"""relay_amd: relay's attention and int8 GEMV hot path as a native MI355X (gfx950) backend.

The product is librelay_hip.so (hand-written HIP kernels + the C++ HipBackend behind
relay's Backend interface, C ABI in include/relay_hip.h). This package is its Python
host surface: the ctypes binding (_lib), relay's config/weights types (model), the
Backend mirror (backend) and a greedy engine loop (engine). Nothing here computes on the
CPU: without the built library or a GPU, calls raise.
"""
from .backend import ForwardBatch, HipBackend, HipOptions, SeqChunk, make_hip_backend
from .model import HostWeights, ModelConfig, llama3_8b, smollm2_135m, tinyllama_1b

__all__ = ["ForwardBatch", "HipBackend", "HipOptions", "SeqChunk", "make_hip_backend", "HostWeights", "ModelConfig",
           "llama3_8b", "smollm2_135m", "tinyllama_1b"]
