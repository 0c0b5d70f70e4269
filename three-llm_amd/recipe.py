"""Decoder recipe and RoPE tables for the Llama/Qwen2 family.

Restates the parts of the reference's loader that fix the per-token path's
numerics (paths relative to packages/three-llm/src/):
  * load/DecoderRecipe.ts:103-174 ``scalingConfig``  (rope_scaling -> RopeScalingConfig)
  * load/DecoderRecipe.ts:348-420 ``buildRecipe`` Llama/Qwen2 branch + ``recipeFor`` checks
  * runtime/rope.ts:4-52          ``ropeParameters`` (inv_freq table, attention factor)
Other architectures (GPT-2, Phi, Gemma, Qwen3.5) are outside this path and are
rejected with the reference's own error text.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np


class RecipeError(ValueError):
    pass


def scaling_config(text: dict) -> Optional[dict]:
    """scalingConfig, load/DecoderRecipe.ts:103-174 (llama architecture)."""
    if text.get("rope_parameters"):
        raise RecipeError("Unsupported rope_parameters configuration; use rope_scaling for this architecture.")
    scaling = text.get("rope_scaling")
    if not scaling:
        return None
    if scaling.get("rope_type") and scaling.get("type") and scaling["rope_type"] != scaling["type"]:
        raise RecipeError("Conflicting RoPE scaling types.")
    kind = scaling.get("rope_type") or scaling.get("type")
    if kind == "default":
        if any(k not in ("rope_type", "type") for k in scaling):
            raise RecipeError("Default RoPE cannot include scaling parameters.")
        return None
    if kind not in ("yarn", "linear", "llama3"):
        raise RecipeError(f'Unsupported RoPE scaling type "{kind}".')
    allowed = {"type", "rope_type", "factor"}
    if kind == "yarn":
        allowed |= {"original_max_position_embeddings", "beta_fast", "beta_slow", "attention_factor", "mscale",
                    "mscale_all_dim"}
    elif kind == "llama3":
        allowed |= {"original_max_position_embeddings", "low_freq_factor", "high_freq_factor"}
    for key in scaling:
        if key not in allowed:
            raise RecipeError(f'Unsupported {kind} RoPE parameter "{key}".')
    factor = scaling.get("factor")
    if factor is None or not math.isfinite(factor) or factor < 1:
        raise RecipeError("Invalid RoPE scaling factor.")
    if kind == "linear":
        return {"type": "linear", "factor": float(factor)}
    original = scaling.get("original_max_position_embeddings", text.get("max_position_embeddings"))
    if kind == "llama3":
        return {"type": "llama3", "factor": float(factor), "originalContextLength": original,
                "lowFreqFactor": scaling.get("low_freq_factor"), "highFreqFactor": scaling.get("high_freq_factor")}
    # Transformers 4.51.3 derives the effective factor from the context ratio
    # when original_max_position_embeddings is given explicitly.
    if scaling.get("original_max_position_embeddings") is not None:
        factor = text["max_position_embeddings"] / original

    def mscale(value):
        return 1.0 if factor <= 1 else 1 + 0.1 * value * math.log(factor)

    if scaling.get("attention_factor") is not None:
        attention_factor = scaling["attention_factor"]
    elif scaling.get("mscale") and scaling.get("mscale_all_dim"):
        attention_factor = mscale(scaling["mscale"]) / mscale(scaling["mscale_all_dim"])
    else:
        attention_factor = mscale(1)
    return {"type": "yarn", "factor": float(factor), "originalContextLength": original,
            "betaFast": scaling.get("beta_fast", 32), "betaSlow": scaling.get("beta_slow", 1),
            "attentionFactor": attention_factor}


def rope_parameters(dim: int, theta: float, scaling: Optional[dict] = None):
    """ropeParameters, runtime/rope.ts:4-52 -> (inv_freq float32[dim/2], attention_factor)."""
    if not isinstance(dim, int) or dim < 0 or dim % 2 != 0:
        raise RecipeError("RoPE dimension must be a non-negative even integer.")
    if not math.isfinite(theta) or theta <= 1:
        raise RecipeError("RoPE theta must be finite and greater than one.")
    kind = scaling.get("type") if scaling else None
    inv_freq = np.zeros(dim // 2, np.float32)
    attention_factor = 1.0
    low = high = 0.0
    if scaling and (not math.isfinite(scaling["factor"]) or scaling["factor"] < 1):
        raise RecipeError("RoPE scaling factor must be finite and at least one.")
    if kind == "yarn":
        orig, bf, bs = scaling["originalContextLength"], scaling["betaFast"], scaling["betaSlow"]
        if not all(math.isfinite(v) for v in (orig, bf, bs)) or not (orig > 0 and bf > 0 and bs > 0 and bf >= bs):
            raise RecipeError("Invalid YaRN context or beta range.")
        af = scaling.get("attentionFactor")
        attention_factor = af if af is not None else 1 + 0.1 * math.log(scaling["factor"])
        if not math.isfinite(attention_factor) or attention_factor <= 0:
            raise RecipeError("Invalid YaRN attention factor.")

        def correction(rotations):
            return (dim * math.log(orig / (rotations * 2 * math.pi))) / (2 * math.log(theta))

        low = max(0.0, math.floor(correction(bf)))
        high = min(dim - 1.0, math.ceil(correction(bs)))
        if low == high:
            high += 0.001
    if kind == "llama3":
        orig, lo, hi = scaling["originalContextLength"], scaling["lowFreqFactor"], scaling["highFreqFactor"]
        if lo is None or hi is None or not all(math.isfinite(v) for v in (orig, lo, hi)) or \
                not (orig > 0 and lo > 0 and hi > lo):
            raise RecipeError("Invalid Llama 3 RoPE frequency range.")
    for i in range(dim // 2):
        frequency = 1.0 / math.pow(theta, (2 * i) / dim)
        if kind == "linear":
            frequency /= scaling["factor"]
        if kind == "yarn":
            ramp = min(1.0, max(0.0, (i - low) / (high - low)))
            frequency *= 1 - ramp + ramp / scaling["factor"]
        if kind == "llama3":
            wavelength = (2 * math.pi) / frequency
            if wavelength > orig / lo:
                frequency /= scaling["factor"]
            elif wavelength >= orig / hi:
                smooth = (orig / wavelength - lo) / (hi - lo)
                frequency *= (1 - smooth) / scaling["factor"] + smooth
        inv_freq[i] = frequency
    return inv_freq, attention_factor


@dataclass
class Recipe:
    """The DecoderRecipe fields the per-token path reads (types.ts:201-243)."""
    hidden_size: int
    inner_size: int
    layer_count: int
    head_count: int
    kv_head_count: int
    head_dim: int
    vocab_size: int
    context_limit: int
    norm_eps: float
    rope_theta: float
    rotary_dim: int
    qkv_bias: bool = False
    tied_embeddings: bool = False
    sliding_window: int = 0
    # config layer_types (None: absent); an empty list still counts as present,
    # as the reference's `this.layerTypes ? 0 : ...` test of an array does
    layer_types: Optional[list] = None
    attn_scale: float = 0.0  # attnScale: undefined (0 selects 1/sqrt(head_dim)) for this recipe
    rope_scaling: Optional[dict] = None
    end_of_text_token_id: int = 0
    stop_token_ids: list = field(default_factory=list)
    model_type: str = "llama"

    @property
    def q_size(self) -> int:
        return self.head_count * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.kv_head_count * self.head_dim

    def rope(self):
        return rope_parameters(self.rotary_dim, self.rope_theta, self.rope_scaling)

    def layer_window(self, index: int) -> int:
        """The block's slidingWindow (DecoderWeights.ts:307-311): with layer types,
        sliding_attention layers take the recipe's window and the others 0;
        without them every layer takes the recipe's window."""
        types = self.layer_types
        layer_type = (types[index] if types is not None and index < len(types) else None) or "full_attention"
        if layer_type == "sliding_attention":
            return self.sliding_window or 0
        return 0 if types is not None else (self.sliding_window or 0)

    @property
    def layer_windows(self) -> list:
        return [self.layer_window(i) for i in range(self.layer_count)]


def recipe_for(config: dict, has_lm_head: bool = True, has_qkv_bias: bool = False) -> Recipe:
    """buildRecipe Llama/Qwen2 branch + recipeFor (load/DecoderRecipe.ts:348-420)."""
    text = config.get("text_config") if isinstance(config.get("text_config"), dict) else config
    model_type = text.get("model_type", "llama")
    if model_type not in ("llama", "qwen2", "mistral"):
        raise RecipeError(f'Unsupported model_type "{model_type}".')
    hidden = text["hidden_size"]
    heads = text["num_attention_heads"]
    head_dim = text.get("head_dim") or hidden // heads
    if text.get("rotary_dim") is not None:
        rotary_dim = text["rotary_dim"]
    elif text.get("partial_rotary_factor") is not None:
        rotary_dim = int(math.floor(text["partial_rotary_factor"] * head_dim))
    else:
        rotary_dim = head_dim
    if not isinstance(rotary_dim, int) or rotary_dim < 0 or rotary_dim > head_dim or rotary_dim % 2 != 0:
        raise RecipeError("Invalid rotary dimension: expected an even integer within the head dimension.")
    eos = text.get("eos_token_id", 0)
    eos_ids = eos if isinstance(eos, list) else [eos]
    sliding = 0 if text.get("use_sliding_window") is False else (text.get("sliding_window") or 0)
    layer_types = text.get("layer_types")
    if layer_types is not None and "sliding_attention" in layer_types:
        # sliding layers take localRopeTheta (DecoderWeights.ts:310), which
        # differs from rope_theta only with rope_local_base_freq; one RoPE
        # table per model here
        local = text.get("rope_local_base_freq")
        if local and local != (text.get("rope_theta") or 10000):
            raise RecipeError("Per-layer RoPE bases (rope_local_base_freq) are not supported.")
    recipe = Recipe(
        hidden_size=hidden,
        inner_size=text["intermediate_size"],
        layer_count=text["num_hidden_layers"],
        head_count=heads,
        kv_head_count=text.get("num_key_value_heads") or heads,
        head_dim=head_dim,
        vocab_size=text["vocab_size"],
        context_limit=text.get("max_position_embeddings") or 2048,
        norm_eps=text.get("rms_norm_eps") or 1e-5,
        rope_theta=text.get("rope_theta") or 10000,
        rotary_dim=rotary_dim,
        qkv_bias=bool(has_qkv_bias or text.get("attention_bias")),
        # DecoderWeights.loadOutputWeight (DecoderWeights.ts:243-251): the head is
        # untied only if lm_head.weight exists and tie_word_embeddings is not true.
        tied_embeddings=not (has_lm_head and text.get("tie_word_embeddings") is not True),
        sliding_window=sliding,
        layer_types=list(layer_types) if layer_types is not None else None,
        rope_scaling=scaling_config(text),
        end_of_text_token_id=eos_ids[0] if eos_ids else 0,
        stop_token_ids=list(eos_ids),
        model_type=model_type,
    )
    if recipe.rotary_dim > 0:
        recipe.rope()  # raises on the configurations ropeParameters rejects
    return recipe
