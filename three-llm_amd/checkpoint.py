"""Local Hugging Face checkpoints -> HostWeights (q4 packed at upload).

Restates, for a local directory instead of URLs (no network here):

* parseSafeTensors (load/SafeTensorsLoader.ts:104-186): the same checks and
  messages; tensors are zero-copy numpy views over a memory map (F16 / BF16
  stay raw uint16 bits, like the reference's Uint16Array views);
* shard discovery (SafeTensorsLoader.ts:228-244): model.safetensors if it
  exists, else the distinct files of model.safetensors.index.json's
  weight_map in first-seen order;
* the Llama alias table, candidate keys and lookup (load/TensorNameMap.ts:
  12-25, 58-73, 133-201) and the language prefix (load/tensors.ts:284-291);
* the recipe from config.json (load/DecoderRecipe.ts:348-420, recipe.py);
* F16 / BF16 -> fp32 (load/tensors.ts:29-68): exact widening.

The q4 pack happens in HostWeights.tensor (tlm_quantize_q4) as the tensors
are uploaded, one at a time, so the fp32 copy of the whole model never exists.
"""
from __future__ import annotations

import json
import mmap
import os
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np

from .recipe import recipe_for
from . import weights as W

DTYPE_BYTES = {"F32": 4, "F16": 2, "BF16": 2, "I32": 4, "I64": 8, "U8": 1, "BOOL": 1}
_NP = {"F32": np.float32, "F16": np.uint16, "BF16": np.uint16, "I32": np.int32, "I64": np.int64, "U8": np.uint8,
       "BOOL": np.uint8}
_MAX_SAFE = 2 ** 53 - 1


class SafeTensorsError(ValueError):
    pass


class Tensor:
    """name, dtype (safetensors spelling), shape and a numpy view of the data."""

    def __init__(self, name: str, dtype: str, shape: List[int], data: np.ndarray):
        self.name, self.dtype, self.shape, self.data = name, dtype, list(shape), data

    def fp32(self) -> np.ndarray:
        """tensorToFloat32 (load/tensors.ts:29-68): fp16 and bf16 widen exactly."""
        if self.dtype == "F32":
            out = self.data
        elif self.dtype == "F16":
            out = self.data.view(np.float16).astype(np.float32)
        elif self.dtype == "BF16":
            out = (self.data.astype(np.uint32) << 16).view(np.float32)
        else:
            raise SafeTensorsError(f'SafeTensorsLoader: Tensor "{self.name}" has non-float dtype "{self.dtype}".')
        return np.asarray(out, np.float32).reshape(self.shape)


def _safe_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) and -_MAX_SAFE <= v <= _MAX_SAFE


def parse_safetensors(buffer, keep_tensor: Optional[Callable[[str], bool]] = None):
    """parseSafeTensors: (metadata, {name: Tensor}) from a bytes-like buffer."""
    mv = memoryview(buffer)
    if mv.nbytes < 8:
        raise SafeTensorsError("SafeTensorsLoader: File is too small to contain a header.")
    low = int.from_bytes(mv[0:4], "little")
    high = int.from_bytes(mv[4:8], "little")
    if high != 0:
        raise SafeTensorsError("SafeTensorsLoader: Header is too large (4 GiB or more).")
    header_end = 8 + low
    if header_end > mv.nbytes:
        raise SafeTensorsError(f"SafeTensorsLoader: Header extends beyond the file ({low} bytes).")
    header = json.loads(bytes(mv[8:header_end]).decode("utf-8"))
    tensors: Dict[str, Tensor] = {}
    for name, desc in header.items():
        if name == "__metadata__":
            continue
        if keep_tensor is not None and keep_tensor(name) is False:
            continue
        if not isinstance(desc, dict):
            raise SafeTensorsError(f'SafeTensorsLoader: Tensor "{name}" has an invalid descriptor.')
        dtype, shape, offsets = desc.get("dtype"), desc.get("shape"), desc.get("data_offsets")
        if dtype not in DTYPE_BYTES:
            raise SafeTensorsError(f'SafeTensorsLoader: Unsupported dtype "{dtype}" for tensor "{name}".')
        if not isinstance(shape, list) or any(not _safe_int(s) or s < 0 for s in shape):
            raise SafeTensorsError(f'SafeTensorsLoader: Tensor "{name}" has an invalid shape.')
        if not isinstance(offsets, list) or len(offsets) != 2:
            raise SafeTensorsError(f'SafeTensorsLoader: Tensor "{name}" has invalid data offsets.')
        begin, end = offsets
        if not _safe_int(begin) or not _safe_int(end) or begin < 0 or end < begin or header_end + end > mv.nbytes:
            raise SafeTensorsError(f'SafeTensorsLoader: Tensor "{name}" data extends beyond the file.')
        count = 1
        for s in shape:
            count *= s
        expected = count * DTYPE_BYTES[dtype]
        if not _safe_int(expected) or end - begin != expected:
            raise SafeTensorsError(
                f'SafeTensorsLoader: Tensor "{name}" has {end - begin} bytes, expected {expected}.')
        data = np.frombuffer(mv, dtype=_NP[dtype], count=count, offset=header_end + begin)
        tensors[name] = Tensor(name, dtype, shape, data)
    meta = header.get("__metadata__") or {}
    return meta, tensors


def resolve_safetensor_files(root: str) -> List[str]:
    """resolveSafetensorFilesFromIndex for a local directory."""
    if os.path.isfile(os.path.join(root, "model.safetensors")):
        return ["model.safetensors"]
    index_path = os.path.join(root, "model.safetensors.index.json")
    if not os.path.isfile(index_path):
        raise SafeTensorsError(f"SafeTensorsLoader: neither model.safetensors nor model.safetensors.index.json "
                               f"in {root}")
    with open(index_path) as f:
        index = json.load(f)
    files: List[str] = []
    for name in index["weight_map"].values():
        if name not in files:
            files.append(name)
    return files


def load_safetensors_model(root: str, keep_tensor: Optional[Callable[[str], bool]] = None,
                           on_progress: Optional[Callable[[str], None]] = None) -> Dict[str, Tensor]:
    """loadSafetensorsModel: every shard parsed (memory-mapped) and merged."""
    tensors: Dict[str, Tensor] = {}
    files = resolve_safetensor_files(root)
    for i, name in enumerate(files):
        with open(os.path.join(root, name), "rb") as f:
            size = os.fstat(f.fileno()).st_size
            buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else b""
        _, part = parse_safetensors(buf, keep_tensor)
        tensors.update(part)
        if on_progress:
            on_progress(f"Loading tensor model data, {i + 1} of {len(files)} parts")
    return tensors


# ------------------------------------------------------------- name mapping --

LLAMA_GLOBAL = {  # TensorNameMap.ts:20-24
    "token_embd": ["embed_tokens.weight"],
    "output": ["lm_head.weight", "embed_tokens.weight"],
    "output_norm": ["norm.weight"],
}
LLAMA_BLOCK = {  # TensorNameMap.ts:58-73
    "attn_norm": ["layers.{bid}.input_layernorm.weight"],
    "ffn_norm": ["layers.{bid}.post_attention_layernorm.weight"],
    "attn_q": ["layers.{bid}.self_attn.q_proj.weight"],
    "attn_k": ["layers.{bid}.self_attn.k_proj.weight"],
    "attn_v": ["layers.{bid}.self_attn.v_proj.weight"],
    "attn_q_bias": ["layers.{bid}.self_attn.q_proj.bias"],
    "attn_k_bias": ["layers.{bid}.self_attn.k_proj.bias"],
    "attn_v_bias": ["layers.{bid}.self_attn.v_proj.bias"],
    "attn_q_norm": ["layers.{bid}.self_attn.q_norm.weight"],
    "attn_k_norm": ["layers.{bid}.self_attn.k_norm.weight"],
    "attn_out": ["layers.{bid}.self_attn.o_proj.weight"],
    "ffn_gate": ["layers.{bid}.mlp.gate_proj.weight"],
    "ffn_up": ["layers.{bid}.mlp.up_proj.weight"],
    "ffn_down": ["layers.{bid}.mlp.down_proj.weight"],
}


class TensorNameError(KeyError):
    pass


def detect_language_prefix(tensors) -> str:
    """detectLanguagePrefix, load/tensors.ts:284-291."""
    for p in ("model.language_model.", "language_model.", "model."):
        if p + "embed_tokens.weight" in tensors:
            return p
    if "embed_tokens.weight" in tensors:
        return ""
    return "model."


def _aliases(key: str, bid: Optional[int]) -> Optional[List[str]]:
    table = LLAMA_GLOBAL if bid is None else LLAMA_BLOCK
    if key not in table:
        return None
    return table[key] if bid is None else [a.replace("{bid}", str(bid)) for a in table[key]]


def _find(tensors, prefix: str, aliases: List[str]):
    tried = []
    for a in aliases:
        for k in ([prefix + a, a] if prefix else [a]):  # candidateKeys
            tried.append(k)
            if k in tensors:
                return tensors[k], tried
    return None, tried


def has_mapped_tensor(tensors, prefix: str, key: str, bid: Optional[int] = None) -> bool:
    aliases = _aliases(key, bid)
    return aliases is not None and _find(tensors, prefix, aliases)[0] is not None


def resolve_tensor(tensors, prefix: str, key: str, bid: Optional[int] = None):
    """resolveTensor (TensorNameMap.ts:180-201) for the llama architecture."""
    aliases = _aliases(key, bid)
    if aliases is None:
        raise TensorNameError(f'TensorNameMap: Unknown tensor "{key}" for architecture "llama".')
    t, tried = _find(tensors, prefix, aliases)
    if t is None:
        raise TensorNameError(f'TensorNameMap: Missing "{key}" (llama). Tried: {", ".join(tried)}.')
    return t


# ------------------------------------------------------------------ loading --

def load_config(root: str) -> dict:
    with open(os.path.join(root, "config.json")) as f:
        return json.load(f)


def host_weights(config: dict, tensors, storage: "W.Storage") -> "W.HostWeights":
    """HostWeights over named checkpoint tensors (Tensor objects or arrays):
    the reference's Llama mapping (DecoderWeights.ts:305-337) through the
    alias table; QKV rows packed Q|K|V (tensors.ts:224-240)."""
    def f32(t):
        return t.fp32() if isinstance(t, Tensor) else np.asarray(t, np.float32)

    prefix = detect_language_prefix(tensors)
    # untied only with a separate lm_head.weight (the recipe also honours tie_word_embeddings)
    has_head = _find(tensors, prefix, ["lm_head.weight"])[0] is not None
    has_bias = has_mapped_tensor(tensors, prefix, "attn_q_bias", 0)
    rec = recipe_for(config, has_lm_head=has_head, has_qkv_bias=has_bias)

    def R(key, bid=None):
        return f32(resolve_tensor(tensors, prefix, key, bid))

    def bias(key, l, size):
        return R(key, l) if has_mapped_tensor(tensors, prefix, key, l) else np.zeros(size, np.float32)

    def source(kind, l):
        if kind == W.EMBED:
            return R("token_embd")
        if kind == W.LM_HEAD:
            return R("output")
        if kind == W.FINAL_NORM:
            return R("output_norm")
        if kind == W.ATTN_NORM:
            return R("attn_norm", l)
        if kind == W.FFN_NORM:
            return R("ffn_norm", l)
        if kind == W.WQKV:
            return np.concatenate([R("attn_q", l), R("attn_k", l), R("attn_v", l)])
        if kind == W.BQKV:
            return np.concatenate([bias("attn_q_bias", l, rec.q_size), bias("attn_k_bias", l, rec.kv_size),
                                   bias("attn_v_bias", l, rec.kv_size)])
        if kind == W.WO:
            return R("attn_out", l)
        if kind == W.WGATE:
            return R("ffn_gate", l)
        if kind == W.WUP:
            return R("ffn_up", l)
        if kind == W.WDOWN:
            return R("ffn_down", l)
        raise KeyError(kind)

    return W.HostWeights(rec, storage, source)


def load_checkpoint(root: str, storage: Optional["W.Storage"] = None,
                    on_progress: Optional[Callable[[str], None]] = None) -> Tuple["W.HostWeights", dict]:
    """loadHFModelBundle for a local directory (config + safetensors shards),
    without the tokenizer: (HostWeights, config).  Linears default to q4 g32,
    the embedding / tied head to fp16, the cache to fp16."""
    config = load_config(root)
    tensors = load_safetensors_model(root, on_progress=on_progress)
    hw = host_weights(config, tensors, storage or W.Storage(linear="q4", head="f16", embed="f16", kv="f16"))
    hw.tensors = tensors  # keeps the memory maps alive
    return hw, config
