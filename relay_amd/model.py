"""Model configuration and host weights, in relay's terms.

ModelConfig mirrors relay's ModelConfig (engine/include/relay/config.h) and reads a
Hugging Face config.json the way config.cpp:20-77 does. HostWeights mirrors relay's
HostWeights (weights.h:13-31): fp32 arrays with q/k/v fused into wqkv and gate/up into
w_gate_up, loaded from safetensors with the tensor names of weights.cpp:26-61, or drawn
from the seeded synthetic generator.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
from dataclasses import dataclass, field

import numpy as np

from . import _lib


@dataclass
class ModelConfig:
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    tie_embeddings: bool = False
    qkv_bias: bool = False
    rope_llama3: bool = False
    rope_factor: float = 1.0
    rope_low_freq_factor: float = 1.0
    rope_high_freq_factor: float = 4.0
    rope_original_max_position: float = 8192.0
    model_type: str = "llama"
    eos_ids: list = field(default_factory=list)

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @classmethod
    def from_json_text(cls, text: str) -> "ModelConfig":
        """relay's ModelConfig::from_json_text (config.cpp:20-77): llama and qwen2."""
        j = json.loads(text)
        mt = j["model_type"]
        if mt not in ("llama", "qwen2"):
            raise ValueError(f"unsupported model_type {mt} (llama and qwen2 are supported)")
        heads = int(j["num_attention_heads"])
        kvh = j.get("num_key_value_heads")
        kvh = heads if kvh is None else int(kvh)
        hd = j.get("head_dim")
        hd = int(j["hidden_size"]) // heads if hd is None else int(hd)
        c = cls(hidden=int(j["hidden_size"]), intermediate=int(j["intermediate_size"]),
                layers=int(j["num_hidden_layers"]), heads=heads, kv_heads=kvh, head_dim=hd,
                vocab=int(j["vocab_size"]), model_type=mt)
        if "rms_norm_eps" in j:
            c.rms_eps = float(j["rms_norm_eps"])
        if "tie_word_embeddings" in j:
            c.tie_embeddings = bool(j["tie_word_embeddings"])
        c.qkv_bias = mt == "qwen2" or bool(j.get("attention_bias", False))
        if j.get("mlp_bias"):
            raise ValueError("mlp_bias is not supported")
        if j.get("use_sliding_window"):
            raise ValueError("sliding-window attention is not supported")
        rope = j.get("rope_parameters") or j.get("rope_scaling")
        if "rope_theta" in j:
            c.rope_theta = float(j["rope_theta"])
        if rope and "rope_theta" in rope:
            c.rope_theta = float(rope["rope_theta"])
        if rope:
            kind = rope.get("rope_type", rope.get("type"))
            if kind == "llama3":
                c.rope_llama3 = True
                c.rope_factor = float(rope["factor"])
                c.rope_low_freq_factor = float(rope["low_freq_factor"])
                c.rope_high_freq_factor = float(rope["high_freq_factor"])
                c.rope_original_max_position = float(rope["original_max_position_embeddings"])
            elif kind != "default":
                raise ValueError(f"unsupported rope_scaling type {kind}")
        eos = j.get("eos_token_id")
        if eos is not None:
            c.eos_ids = list(eos) if isinstance(eos, list) else [int(eos)]
        if c.heads % c.kv_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        if c.head_dim % 2:
            raise ValueError("head_dim must be even")
        return c

    def to_c(self) -> _lib.ModelConfigC:
        return _lib.ModelConfigC(self.hidden, self.intermediate, self.layers, self.heads, self.kv_heads,
                                 self.head_dim, self.vocab, int(self.tie_embeddings), int(self.qkv_bias),
                                 int(self.rope_llama3), self.rms_eps, self.rope_theta, self.rope_factor,
                                 self.rope_low_freq_factor, self.rope_high_freq_factor,
                                 self.rope_original_max_position)

    def to_hf_json(self) -> dict:
        """A Hugging Face config.json with these hyperparameters (for relay's own loader)."""
        j = {"architectures": ["LlamaForCausalLM" if self.model_type == "llama" else "Qwen2ForCausalLM"],
             "model_type": self.model_type, "hidden_size": self.hidden, "intermediate_size": self.intermediate,
             "num_hidden_layers": self.layers, "num_attention_heads": self.heads,
             "num_key_value_heads": self.kv_heads, "head_dim": self.head_dim, "vocab_size": self.vocab,
             "max_position_embeddings": 131072, "rms_norm_eps": self.rms_eps, "rope_theta": self.rope_theta,
             "tie_word_embeddings": self.tie_embeddings, "attention_bias": self.qkv_bias,
             "eos_token_id": self.eos_ids[0] if self.eos_ids else 0}
        if self.rope_llama3:
            j["rope_scaling"] = {"rope_type": "llama3", "factor": self.rope_factor,
                                 "low_freq_factor": self.rope_low_freq_factor,
                                 "high_freq_factor": self.rope_high_freq_factor,
                                 "original_max_position_embeddings": int(self.rope_original_max_position)}
        return j


# ---- the benchmark shapes -----------------------------------------

def smollm2_135m() -> ModelConfig:
    return ModelConfig(hidden=576, intermediate=1536, layers=30, heads=9, kv_heads=3, head_dim=64, vocab=49152,
                       rms_eps=1e-5, rope_theta=10000.0, tie_embeddings=True)


def tinyllama_1b() -> ModelConfig:
    return ModelConfig(hidden=2048, intermediate=5632, layers=22, heads=32, kv_heads=4, head_dim=64, vocab=32000,
                       rms_eps=1e-5, rope_theta=10000.0)


def llama3_8b() -> ModelConfig:
    # Llama-3.1 rope scaling values (factor 8, low 1, high 4, original 8192).
    return ModelConfig(hidden=4096, intermediate=14336, layers=32, heads=32, kv_heads=8, head_dim=128,
                       vocab=128256, rms_eps=1e-5, rope_theta=500000.0, rope_llama3=True, rope_factor=8.0,
                       rope_low_freq_factor=1.0, rope_high_freq_factor=4.0, rope_original_max_position=8192.0)


@dataclass
class LayerWeights:
    attn_norm: np.ndarray
    wqkv: np.ndarray
    bqkv: np.ndarray | None
    wo: np.ndarray
    mlp_norm: np.ndarray
    w_gate_up: np.ndarray
    w_down: np.ndarray


@dataclass
class HostWeights:
    config: ModelConfig
    embed: np.ndarray
    layers: list
    final_norm: np.ndarray
    lm_head: np.ndarray | None

    def lm_head_or_embed(self) -> np.ndarray:
        return self.embed if self.lm_head is None else self.lm_head

    # ---- loading ------------------------------------------------------------------

    @classmethod
    def load(cls, model_dir: str) -> "HostWeights":
        """relay's HostWeights::load (weights.cpp:26-61) for a single-file model."""
        with open(os.path.join(model_dir, "config.json")) as f:
            c = ModelConfig.from_json_text(f.read())
        t = read_safetensors(os.path.join(model_dir, "model.safetensors"))
        H, Q, KV, I, V = c.hidden, c.q_dim, c.kv_dim, c.intermediate, c.vocab

        def take(name, shape):
            a = t[name]
            if tuple(a.shape) != tuple(shape):
                raise ValueError(f"{name}: expected shape {shape} but the file has {a.shape}")
            return np.ascontiguousarray(a, dtype=np.float32)

        embed = take("model.embed_tokens.weight", (V, H))
        final_norm = take("model.norm.weight", (H,))
        lm_head = None
        if "lm_head.weight" in t and not c.tie_embeddings:
            lm_head = take("lm_head.weight", (V, H))
        elif not c.tie_embeddings:
            raise ValueError("lm_head.weight is missing and the embeddings are not tied")
        layers = []
        for l in range(c.layers):
            p = f"model.layers.{l}."
            wqkv = np.concatenate([take(p + "self_attn.q_proj.weight", (Q, H)),
                                   take(p + "self_attn.k_proj.weight", (KV, H)),
                                   take(p + "self_attn.v_proj.weight", (KV, H))])
            bqkv = None
            if c.qkv_bias:
                bqkv = np.concatenate([take(p + "self_attn.q_proj.bias", (Q,)), take(p + "self_attn.k_proj.bias", (KV,)),
                                       take(p + "self_attn.v_proj.bias", (KV,))])
            gu = np.concatenate([take(p + "mlp.gate_proj.weight", (I, H)), take(p + "mlp.up_proj.weight", (I, H))])
            layers.append(LayerWeights(take(p + "input_layernorm.weight", (H,)), np.ascontiguousarray(wqkv), bqkv,
                                       take(p + "self_attn.o_proj.weight", (H, Q)),
                                       take(p + "post_attention_layernorm.weight", (H,)), np.ascontiguousarray(gu),
                                       take(p + "mlp.down_proj.weight", (H, I))))
        return cls(c, embed, layers, final_norm, lm_head)

    @classmethod
    def synthetic(cls, c: ModelConfig, seed: int = 0, std: float = 0.02, norm_one: bool = True) -> "HostWeights":
        """Every matrix, embedding and bias ~ N(0, std) from the counter-based generator
        (rh_synth_normal_f32); norm weights 1 (the Hugging Face initialisation) unless
        norm_one is False. Stream ids: embed 1, lm_head 2, layer l matrices 100 + 16 l + k."""
        H, Q, KV, I, V = c.hidden, c.q_dim, c.kv_dim, c.intermediate, c.vocab
        QKV = Q + 2 * KV

        def normal(n, stream, s=std):
            out = np.empty(n, dtype=np.float32)
            _lib.lib().rh_synth_normal_f32(out.ctypes.data, n, seed, stream, 0.0, s)
            return out

        def norm(stream):
            return np.ones(H, np.float32) if norm_one else 1.0 + normal(H, stream, 0.1)

        embed = normal(V * H, 1).reshape(V, H)
        lm_head = None if c.tie_embeddings else normal(V * H, 2).reshape(V, H)
        layers = []
        for l in range(c.layers):
            sid = 100 + 16 * l
            layers.append(LayerWeights(norm(sid + 5), normal(QKV * H, sid + 1).reshape(QKV, H),
                                       normal(QKV, sid + 7) if c.qkv_bias else None,
                                       normal(H * Q, sid + 2).reshape(H, Q), norm(sid + 6),
                                       normal(2 * I * H, sid + 3).reshape(2 * I, H),
                                       normal(H * I, sid + 4).reshape(H, I)))
        return cls(c, embed, layers, norm(3), lm_head)

    def named(self) -> dict:
        """Tensors by relay's names (backend.h:74-77)."""
        out = {"embed": self.embed, "final_norm": self.final_norm}
        if self.lm_head is not None:
            out["lm_head"] = self.lm_head
        for i, L in enumerate(self.layers):
            for f in ("attn_norm", "wqkv", "bqkv", "wo", "mlp_norm", "w_gate_up", "w_down"):
                v = getattr(L, f)
                if v is not None:
                    out[f"layers.{i}.{f}"] = v
        return out

    def to_hf_tensors(self) -> dict:
        """Hugging Face tensor names -> arrays (the inverse of load)."""
        c = self.config
        Q, KV, I = c.q_dim, c.kv_dim, c.intermediate
        t = {"model.embed_tokens.weight": self.embed, "model.norm.weight": self.final_norm}
        if self.lm_head is not None:
            t["lm_head.weight"] = self.lm_head
        for l, L in enumerate(self.layers):
            p = f"model.layers.{l}."
            t[p + "input_layernorm.weight"] = L.attn_norm
            t[p + "post_attention_layernorm.weight"] = L.mlp_norm
            t[p + "self_attn.q_proj.weight"] = L.wqkv[:Q]
            t[p + "self_attn.k_proj.weight"] = L.wqkv[Q:Q + KV]
            t[p + "self_attn.v_proj.weight"] = L.wqkv[Q + KV:]
            if L.bqkv is not None:
                t[p + "self_attn.q_proj.bias"] = L.bqkv[:Q]
                t[p + "self_attn.k_proj.bias"] = L.bqkv[Q:Q + KV]
                t[p + "self_attn.v_proj.bias"] = L.bqkv[Q + KV:]
            t[p + "self_attn.o_proj.weight"] = L.wo
            t[p + "mlp.gate_proj.weight"] = L.w_gate_up[:I]
            t[p + "mlp.up_proj.weight"] = L.w_gate_up[I:]
            t[p + "mlp.down_proj.weight"] = L.w_down
        return t

    def c_views(self):
        """(rh_host_weights, keepalive) for the C ABI; arrays are borrowed, not copied."""
        L = self.layers
        n = len(L)
        arr = lambda xs: (C.c_void_p * n)(*[x.ctypes.data if x is not None else None for x in xs])
        an, wq, bq = arr([l.attn_norm for l in L]), arr([l.wqkv for l in L]), arr([l.bqkv for l in L])
        wo, mn, gu, wd = arr([l.wo for l in L]), arr([l.mlp_norm for l in L]), arr([l.w_gate_up for l in L]), \
            arr([l.w_down for l in L])
        hw = _lib.HostWeightsC(self.embed.ctypes.data, self.final_norm.ctypes.data,
                               self.lm_head.ctypes.data if self.lm_head is not None else None,
                               C.addressof(an), C.addressof(wq), C.addressof(bq) if self.config.qkv_bias else None,
                               C.addressof(wo), C.addressof(mn), C.addressof(gu), C.addressof(wd))
        return hw, (an, wq, bq, wo, mn, gu, wd)


def read_safetensors(path: str) -> dict:
    """Tensors of a .safetensors file as fp32 numpy arrays. F16 and BF16 widen exactly
    (relay's f16_to_f32 / bf16_to_f32, safetensors.cpp:31-63)."""
    with open(path, "rb") as f:
        data = f.read()
    (hlen,) = struct.unpack("<Q", data[:8])
    header = json.loads(data[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        b, e = info["data_offsets"]
        raw = data[base + b:base + e]
        dt = info["dtype"]
        if dt == "F32":
            a = np.frombuffer(raw, dtype="<f4").copy()
        elif dt == "F16":
            a = np.frombuffer(raw, dtype="<f2").astype(np.float32)
        elif dt == "BF16":
            a = (np.frombuffer(raw, dtype="<u2").astype(np.uint32) << 16).view(np.float32)
        else:
            raise ValueError(f"{name}: unsupported dtype {dt}")
        out[name] = a.reshape(info["shape"])
    return out


def write_safetensors(path: str, tensors: dict) -> None:
    """fp32 tensors to a .safetensors file (for feeding relay's own loader)."""
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        b = np.ascontiguousarray(a, dtype="<f4").tobytes()
        header[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
