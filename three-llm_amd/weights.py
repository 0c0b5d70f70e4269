"""Canonical host tensors for the decoder and the benchmark configurations.

HostWeights holds, per tensor, exactly the bytes the device receives:
fp16 bits, q4 (packed nibbles + fp16 scales) or fp32 (norms, biases, an fp32
embedding).  Matrices are in the Hugging Face [out][in] orientation; Q|K|V
rows are concatenated as the reference's packProjections does
(load/tensors.ts:224-240, DecoderWeights.ts:305-331).

Synthetic weights (the benchmark configurations) come from a seeded
counter-based generator, one stream per (tensor, layer); norm weights are 1.0.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, Optional, Tuple

import numpy as np

from . import tlm
from .recipe import Recipe, recipe_for

# Tensor kinds (stream ids and upload ids)
EMBED, LM_HEAD, FINAL_NORM, ATTN_NORM, FFN_NORM, WQKV, BQKV, WO, WGATE, WUP, WDOWN = (
    "embed", "lm_head", "final_norm", "attn_norm", "ffn_norm", "wqkv", "bqkv", "wo", "wgate", "wup", "wdown")
LINEARS = (WQKV, WO, WGATE, WUP, WDOWN)
_STREAM = {EMBED: 1, LM_HEAD: 2, FINAL_NORM: 3, ATTN_NORM: 4, FFN_NORM: 5, WQKV: 6, BQKV: 7, WO: 8, WGATE: 9,
           WUP: 10, WDOWN: 11}
_UPLOAD = {EMBED: tlm.T_EMBED, LM_HEAD: tlm.T_LM_HEAD, FINAL_NORM: tlm.T_FINAL_NORM, ATTN_NORM: tlm.T_ATTN_NORM,
           FFN_NORM: tlm.T_FFN_NORM, WQKV: tlm.T_WQKV, BQKV: tlm.T_BQKV, WO: tlm.T_WO, WGATE: tlm.T_WGATE,
           WUP: tlm.T_WUP, WDOWN: tlm.T_WDOWN}
_SCALES = {LM_HEAD: tlm.T_LM_HEAD_SCALES, WQKV: tlm.T_WQKV_SCALES, WO: tlm.T_WO_SCALES, WGATE: tlm.T_WGATE_SCALES,
           WUP: tlm.T_WUP_SCALES, WDOWN: tlm.T_WDOWN_SCALES}


@dataclass
class Storage:
    linear: str = "q4"     # "q4" | "f16"
    head: str = "f16"      # LM head when untied
    embed: str = "f16"     # "f16" | "f32"
    kv: str = "f16"        # "f16" | "f32"


def _fmt(name: str) -> int:
    return {"q4": tlm.FMT_Q4, "f16": tlm.FMT_F16, "f32": tlm.FMT_F32}[name]


class HostWeights:
    """Lazily produced canonical tensors: `tensor(kind, layer)` returns
    (data, scales) with scales None except for q4."""

    def __init__(self, recipe: Recipe, storage: Storage, source: Callable[[str, int], np.ndarray]):
        self.recipe = recipe
        self.storage = storage
        self._source = source  # fp32 [out][in] (or vector) for (kind, layer)
        self.cache: Dict[Tuple[str, int], Tuple[np.ndarray, Optional[np.ndarray]]] = {}
        self.keep = False

    def shape(self, kind: str):
        r = self.recipe
        H, I, V = r.hidden_size, r.inner_size, r.vocab_size
        nqkv = r.q_size + 2 * r.kv_size
        return {EMBED: (V, H), LM_HEAD: (V, H), FINAL_NORM: (H,), ATTN_NORM: (H,), FFN_NORM: (H,), WQKV: (nqkv, H),
                BQKV: (nqkv,), WO: (H, r.q_size), WGATE: (I, H), WUP: (I, H), WDOWN: (H, I)}[kind]

    def fmt(self, kind: str) -> str:
        if kind in LINEARS:
            return self.storage.linear
        if kind == LM_HEAD:
            return self.storage.head
        if kind == EMBED:
            return self.storage.embed
        return "f32"

    def fp32(self, kind: str, layer: int = 0) -> np.ndarray:
        return np.ascontiguousarray(self._source(kind, layer), np.float32).reshape(self.shape(kind))

    def tensor(self, kind: str, layer: int = 0):
        key = (kind, layer)
        if key in self.cache:
            return self.cache[key]
        w = self.fp32(kind, layer)
        fmt = self.fmt(kind)
        if fmt == "q4":
            out = tlm.quantize_q4(w)
        elif fmt == "f16":
            out = (tlm.f32_to_f16(w), None)
        else:
            out = (w, None)
        if self.keep:
            self.cache[key] = out
        return out

    def kinds(self):
        r = self.recipe
        yield EMBED, 0
        if not r.tied_embeddings:
            yield LM_HEAD, 0
        yield FINAL_NORM, 0
        for l in range(r.layer_count):
            for k in (ATTN_NORM, FFN_NORM, WQKV, WO, WGATE, WUP, WDOWN):
                yield k, l
            if r.qkv_bias:
                yield BQKV, l

    def model_desc(self, max_tokens: int) -> Tuple[tlm.ModelDesc, np.ndarray]:
        r = self.recipe
        inv, af = r.rope() if r.rotary_dim > 0 else (np.zeros(1, np.float32), 1.0)
        d = tlm.ModelDesc()
        d.hidden_size, d.intermediate_size, d.num_layers = r.hidden_size, r.inner_size, r.layer_count
        d.num_heads, d.num_kv_heads, d.head_dim, d.vocab_size = r.head_count, r.kv_head_count, r.head_dim, r.vocab_size
        d.max_tokens, d.rotary_dim, d.sliding_window = max_tokens, r.rotary_dim, r.sliding_window
        d.linear_fmt, d.head_fmt = _fmt(self.storage.linear), _fmt(self.storage.head)
        d.embed_fmt, d.kv_fmt = _fmt(self.storage.embed), _fmt(self.storage.kv)
        d.qkv_bias, d.tied = int(r.qkv_bias), int(r.tied_embeddings)
        d.rms_eps, d.attention_factor = r.norm_eps, af
        d.attn_scale = r.attn_scale
        return d, inv

    def upload(self, model: tlm.Model) -> None:
        for kind, layer in self.kinds():
            data, scales = self.tensor(kind, layer)
            model.upload(_UPLOAD[kind], layer, data)
            if scales is not None:
                model.upload(_SCALES[kind], layer, scales)


def from_hf(config: dict, tensors: Dict[str, np.ndarray], storage: Storage) -> HostWeights:
    """HF-named fp32 tensors (e.g. the reference's fixture) -> HostWeights, with
    the reference's Llama mapping (DecoderWeights.ts:305-337)."""
    has_head = "lm_head.weight" in tensors
    has_bias = any(k.endswith("q_proj.bias") for k in tensors)
    rec = recipe_for(config, has_lm_head=has_head, has_qkv_bias=has_bias)

    def T(name):
        return np.asarray(tensors[name], np.float32)

    def source(kind, l):
        p = f"model.layers.{l}."
        if kind == EMBED:
            return T("model.embed_tokens.weight")
        if kind == LM_HEAD:
            return T("lm_head.weight")
        if kind == FINAL_NORM:
            return T("model.norm.weight")
        if kind == ATTN_NORM:
            return T(p + "input_layernorm.weight")
        if kind == FFN_NORM:
            return T(p + "post_attention_layernorm.weight")
        if kind == WQKV:
            return np.concatenate([T(p + "self_attn.q_proj.weight"), T(p + "self_attn.k_proj.weight"),
                                   T(p + "self_attn.v_proj.weight")])
        if kind == BQKV:
            def b(n, size):
                return T(p + f"self_attn.{n}_proj.bias") if p + f"self_attn.{n}_proj.bias" in tensors \
                    else np.zeros(size, np.float32)
            return np.concatenate([b("q", rec.q_size), b("k", rec.kv_size), b("v", rec.kv_size)])
        if kind == WO:
            return T(p + "self_attn.o_proj.weight")
        if kind == WGATE:
            return T(p + "mlp.gate_proj.weight")
        if kind == WUP:
            return T(p + "mlp.up_proj.weight")
        if kind == WDOWN:
            return T(p + "mlp.down_proj.weight")
        raise KeyError(kind)

    hw = HostWeights(rec, storage, source)
    hw.keep = True
    return hw


# -------------------------------------------------------------- synthetic --

@dataclass
class Workload:
    """One benchmark configuration (synthetic weights, N(0, 0.02))."""
    name: str
    config: dict
    storage: Storage
    prompt_len: int
    decode_len: int
    max_tokens: int
    qkv_bias: bool = False
    kv_prefill: int = 0        # positions of N(0,1) cache filled before decoding
    note: str = ""
    extra: dict = field(default_factory=dict)


def _cfg(hidden, inter, layers, heads, kv_heads, head_dim, vocab, theta, eps, tied, maxpos):
    return {"model_type": "llama", "hidden_size": hidden, "intermediate_size": inter, "num_hidden_layers": layers,
            "num_attention_heads": heads, "num_key_value_heads": kv_heads, "head_dim": head_dim,
            "vocab_size": vocab, "rope_theta": theta, "rms_norm_eps": eps, "tie_word_embeddings": tied,
            "max_position_embeddings": maxpos, "eos_token_id": -1}


WORKLOADS = {
    "tiny": Workload("tiny-llama-2x256", _cfg(256, 688, 2, 4, 2, 64, 4096, 1e4, 1e-6, False, 2048),
                     Storage(linear="f16", head="f16", embed="f16"), 16, 32, 2048),
    "qwen2.5-0.5b": Workload("qwen2.5-0.5b-shape-q4", _cfg(896, 4864, 24, 14, 2, 64, 151936, 1e6, 1e-6, True, 32768),
                             Storage(linear="q4", embed="f16"), 128, 256, 32768, qkv_bias=True),
    "llama-3.2-1b": Workload("llama-3.2-1b-shape-q4",
                             _cfg(2048, 8192, 16, 32, 8, 64, 128256, 5e5, 1e-5, True, 131072),
                             Storage(linear="q4", embed="f16"), 4096, 128, 4096 + 128),
    "llama-3.2-3b": Workload("llama-3.2-3b-shape-q4",
                             _cfg(3072, 8192, 28, 24, 8, 128, 128256, 5e5, 1e-5, True, 131072),
                             Storage(linear="q4", embed="f16"), 1, 64, 16384 + 64, kv_prefill=16384),
}


def synthetic(w: Workload, seed: int = 0x5EED, std: float = 0.02) -> HostWeights:
    rec = recipe_for(w.config, has_lm_head=not w.config["tie_word_embeddings"], has_qkv_bias=w.qkv_bias)
    shapes_holder = {}

    def source(kind, layer):
        shape = shapes_holder["hw"].shape(kind)
        if kind in (FINAL_NORM, ATTN_NORM, FFN_NORM):
            return np.ones(shape, np.float32)
        n = int(np.prod(shape))
        return tlm.synth_normal(seed, _STREAM[kind] * 4096 + layer, n, std).reshape(shape)

    hw = HostWeights(rec, w.storage, source)
    shapes_holder["hw"] = hw
    return hw


def prompt_tokens(w: Workload, seed: int = 0x5EED) -> np.ndarray:
    return tlm.synth_tokens(seed, 0xFFFF, max(w.prompt_len, 1), w.config["vocab_size"])
