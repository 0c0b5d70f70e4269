"""Per-layer attention options on the CPU: the recipe's per-layer sliding
windows (DecoderWeights.ts:307-311 from the config's layer_types,
DecoderRecipe.ts:355-362) and the oracle's model loop with those windows and
an attention scale (DecoderCPURunner.attention, DecoderCPURunner.ts:140-160).

The oracle's model with per-layer options is pinned against the same layer
loop composed in Python from the oracle's op-level functions, which the
oracle's own tests pin (brute-force attention, closed-form linear and norm);
positions run past the window so a window applied to the wrong layer, or not
at all, changes the result (checked too)."""
import numpy as np
import pytest

from oracle import oracle as orc
from three_llm_amd.recipe import RecipeError, recipe_for


def _cfg(**extra):
    cfg = {"model_type": "qwen2", "hidden_size": 64, "intermediate_size": 96, "num_hidden_layers": 4,
           "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 16, "vocab_size": 50,
           "rope_theta": 1e4, "rms_norm_eps": 1e-6, "max_position_embeddings": 64}
    cfg.update(extra)
    return cfg


# ------------------------------------------------------------------ recipe --

def test_layer_windows_follow_layer_types():
    r = recipe_for(_cfg(sliding_window=8, layer_types=["sliding_attention", "full_attention"] * 2))
    assert r.layer_windows == [8, 0, 8, 0]


def test_without_layer_types_every_layer_takes_the_recipe_window():
    assert recipe_for(_cfg(sliding_window=8)).layer_windows == [8] * 4
    assert recipe_for(_cfg()).layer_windows == [0] * 4
    # use_sliding_window false turns the recipe window off (DecoderRecipe.ts:362)
    r = recipe_for(_cfg(sliding_window=8, use_sliding_window=False,
                        layer_types=["sliding_attention"] * 4))
    assert r.layer_windows == [0] * 4


def test_an_empty_layer_type_list_still_counts_as_present():
    # `this.layerTypes ? 0 : recipe.slidingWindow` with [] (truthy in JS):
    # every layer is full_attention and takes window 0
    assert recipe_for(_cfg(sliding_window=8, layer_types=[])).layer_windows == [0] * 4


def test_missing_entries_default_to_full_attention():
    r = recipe_for(_cfg(sliding_window=8, layer_types=["sliding_attention"]))
    assert r.layer_windows == [8, 0, 0, 0]


def test_per_layer_rope_bases_are_refused():
    with pytest.raises(RecipeError):
        recipe_for(_cfg(sliding_window=8, layer_types=["sliding_attention", "full_attention"] * 2,
                        rope_local_base_freq=1e3))
    # the same base as rope_theta is the single table
    r = recipe_for(_cfg(sliding_window=8, layer_types=["sliding_attention"] * 4, rope_local_base_freq=1e4))
    assert r.layer_windows == [8] * 4


def test_attn_scale_is_undefined_for_this_recipe():
    # DecoderRecipe.ts:391 (attnScale: undefined): 0 selects 1/sqrt(head_dim)
    assert recipe_for(_cfg()).attn_scale == 0.0


# ------------------------------------------------------------------ oracle --

def _weights(rng, H, I, L, Hq, Hkv, D, V):
    s = 0.2
    w = {"embed": rng.standard_normal((V, H)).astype(np.float32), "head": (rng.standard_normal((V, H)) * s),
         "final": 1 + 0.1 * rng.standard_normal(H)}
    for l in range(L):
        w[l] = {"an": 1 + 0.1 * rng.standard_normal(H), "fn": 1 + 0.1 * rng.standard_normal(H),
                "qkv": rng.standard_normal(((Hq + 2 * Hkv) * D, H)) * s, "bqkv": rng.standard_normal((Hq + 2 * Hkv) * D) * s,
                "o": rng.standard_normal((H, Hq * D)) * s, "g": rng.standard_normal((I, H)) * s,
                "u": rng.standard_normal((I, H)) * s, "d": rng.standard_normal((H, I)) * s}
    return w


def _oracle_model(w, dims, windows, scale, inv):
    H, I, L, Hq, Hkv, D, V, T = dims
    m = orc.Model(H, I, L, Hq, Hkv, D, V, T, 1e-6, inv, 1.0, kv_f16=False, attn_scale=scale, layer_windows=windows)
    m.set(orc.EMBED, 0, w["embed"])
    m.set(orc.LM_HEAD, 0, w["head"])
    m.set(orc.FINAL_NORM, 0, w["final"])
    for l in range(L):
        for k, t in (("an", orc.ATTN_NORM), ("fn", orc.FFN_NORM), ("qkv", orc.WQKV), ("bqkv", orc.BQKV),
                     ("o", orc.WO), ("g", orc.WGATE), ("u", orc.WUP), ("d", orc.WDOWN)):
            m.set(t, l, w[l][k])
    return m


def _composed(w, dims, windows, scale, inv, tokens):
    """DecoderCPURunner.forwardToken's Llama branch (:102-132) from the oracle's ops."""
    H, I, L, Hq, Hkv, D, V, T = dims
    kc = [np.zeros((T, Hkv * D), np.float32) for _ in range(L)]
    vc = [np.zeros((T, Hkv * D), np.float32) for _ in range(L)]
    out = []
    for pos, tok in enumerate(tokens):
        x = w["embed"][tok].astype(np.float32)
        for l in range(L):
            qkv = orc.linear_t(orc.rmsnorm(x, w[l]["an"], 1e-6), w[l]["qkv"], w[l]["bqkv"])
            att = orc.attention(qkv, Hq, Hkv, D, pos, kc[l], vc[l], inv, sliding_window=windows[l],
                                attn_scale=scale)
            x = (x.astype(np.float64) + orc.linear_t(att, w[l]["o"]).astype(np.float64)).astype(np.float32)
            n = orc.rmsnorm(x, w[l]["fn"], 1e-6)
            g, u = orc.linear_t(n, w[l]["g"]), orc.linear_t(n, w[l]["u"])
            h = np.array([orc.silu(float(a)) * float(b) for a, b in zip(g, u)], np.float32)
            x = (x.astype(np.float64) + orc.linear_t(h, w[l]["d"]).astype(np.float64)).astype(np.float32)
        out.append(orc.linear_t(orc.rmsnorm(x, w["final"], 1e-6), w["head"]))
    return np.array(out)


def test_oracle_model_applies_each_layers_window_and_the_scale():
    rng = np.random.default_rng(7)
    dims = (32, 48, 3, 4, 2, 8, 40, 24)
    H, I, L, Hq, Hkv, D, V, T = dims
    w = _weights(rng, H, I, L, Hq, Hkv, D, V)
    inv, _ = orc.rope_parameters(D, 1e4)
    tokens = rng.integers(0, V, 14)
    windows, scale = [0, 3, 5], 0.2
    m = _oracle_model(w, dims, windows, scale, inv)
    got = np.array([m.forward(int(t), i) for i, t in enumerate(tokens)])
    m.close()
    want = _composed(w, dims, windows, scale, inv, tokens)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    # the options matter at these positions: other windows or the default
    # scale change the logits past position 3
    for other_w, other_s in (([3, 0, 5], scale), ([0, 3, 0], scale), (windows, 0.0)):
        m2 = _oracle_model(w, dims, other_w, other_s, inv)
        alt = np.array([m2.forward(int(t), i) for i, t in enumerate(tokens)])
        m2.close()
        if other_s == scale:  # windows of 3 and 5 cut nothing before position 3
            np.testing.assert_allclose(alt[:3], got[:3], rtol=1e-6, atol=1e-6)
        assert np.abs(alt[6:] - got[6:]).max() > 1e-4


def test_oracle_model_windows_equal_the_model_window_when_uniform():
    rng = np.random.default_rng(8)
    dims = (32, 48, 2, 4, 2, 8, 40, 16)
    H, I, L, Hq, Hkv, D, V, T = dims
    w = _weights(rng, H, I, L, Hq, Hkv, D, V)
    inv, _ = orc.rope_parameters(D, 1e4)
    a = _oracle_model(w, dims, [4, 4], 0.0, inv)
    b = orc.Model(H, I, L, Hq, Hkv, D, V, T, 1e-6, inv, 1.0, sliding_window=4, kv_f16=False)
    b.set(orc.EMBED, 0, w["embed"])
    b.set(orc.LM_HEAD, 0, w["head"])
    b.set(orc.FINAL_NORM, 0, w["final"])
    for l in range(L):
        for k, t in (("an", orc.ATTN_NORM), ("fn", orc.FFN_NORM), ("qkv", orc.WQKV), ("bqkv", orc.BQKV),
                     ("o", orc.WO), ("g", orc.WGATE), ("u", orc.WUP), ("d", orc.WDOWN)):
            b.set(t, l, w[l][k])
    for i, t in enumerate(rng.integers(0, V, 10)):
        np.testing.assert_array_equal(a.forward(int(t), i), b.forward(int(t), i))
    a.close()
    b.close()


def test_oracle_model_rejects_bad_windows():
    inv, _ = orc.rope_parameters(8, 1e4)
    with pytest.raises(ValueError):
        orc.Model(32, 48, 2, 4, 2, 8, 40, 16, 1e-6, inv, 1.0, layer_windows=[1])
    with pytest.raises(ValueError):
        orc.Model(32, 48, 2, 4, 2, 8, 40, 16, 1e-6, inv, 1.0, layer_windows=[1, -2])
