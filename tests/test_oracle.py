"""Pins the CPU oracle before anything is compared against it.

Every check here is independent of the oracle's own formulas: the Hugging Face
fixture the reference commits (src/test/fixtures/transformers-llama.json), the
reference's closed-form known answers (src/engine.test.ts:489-612), IEEE
conversions done by numpy, and invariants (exhaustive round trips, shift
invariance, brute force on tiny shapes).
"""
import hashlib
import math

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import oracle as orc
import three_llm_amd.recipe as recipe

ATOL, RTOL = 2e-5, 2e-4  # src/test/reference.ts:39 expectClose defaults


def close(actual, expected, atol=ATOL, rtol=RTOL):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape
    assert np.all(np.isfinite(actual))
    err = np.abs(actual - expected) - (atol + rtol * np.abs(expected))
    assert err.max() <= 0, f"max excess {err.max()} at {np.argmax(err)}"


def test_fixture_hash_pinned():
    digest = hashlib.sha256((GOLDEN / "transformers-llama.json").read_bytes()).hexdigest()
    assert digest == (GOLDEN / "transformers-llama.sha256").read_text().strip()


# ------------------------------------------------------------------ dtypes --

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))  # signed zeros too
    # known answers, engine.test.ts:599-601
    assert orc.f16_to_f32(0x3C00) == 1.0


def test_bf16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32)
    expected = (bits << 16).astype(np.uint32).view(np.float32)
    got = np.array([orc.bf16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))
    assert orc.bf16_to_f32(0x3F80) == 1.0 and orc.bf16_to_f32(0x4000) == 2.0  # engine.test.ts:600-609


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(7)
    mant = rng.integers(0, 1 << 23, 200000, dtype=np.uint32)
    exp = rng.integers(95, 145, 200000, dtype=np.uint32)  # spans fp16 zero/subnormal/normal/overflow
    sign = rng.integers(0, 2, 200000, dtype=np.uint32) << 31
    vals = (sign | (exp << 23) | mant).view(np.float32)
    # exact ties and halfway subnormals
    ties = (np.arange(1, 2048, dtype=np.float64) * 2.0 ** -25).astype(np.float32)
    vals = np.concatenate([vals, ties, -ties, np.float32([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0, np.inf])])
    with np.errstate(over="ignore"):
        expected = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, expected)


# -------------------------------------------------------------- closed forms --

def test_reference_closed_forms():
    # engine.test.ts:491-505
    close(orc.linear([1, 2], [3, 4, 5, 6], [7, 8], 2, 2), [20, 24], 1e-6, 0)
    close(orc.linear([1, 2], [3, 4, 5, 6], None, 2, 2), [13, 16], 1e-6, 0)
    close(orc.linear([1, 2], [1, 0, 0, 1], [0, 0], 2, 2), [1, 2], 1e-6, 0)
    # tsl.browser.test.ts:70-79 (non-square, no bias)
    close(orc.linear([1, -1, 0.5], [1, 2, 3, 4, 5, 6], None, 3, 2), [0.5, 1], 1e-6, 0)
    # [out][in] storage gives the same bits as the reference [in][out] order
    rng = np.random.default_rng(1)
    w = rng.standard_normal((37, 23)).astype(np.float32)
    x = rng.standard_normal(37).astype(np.float32)
    b = rng.standard_normal(23).astype(np.float32)
    assert np.array_equal(orc.linear(x, w.reshape(-1), b, 37, 23), orc.linear_t(x, w.T.copy(), b))
    # softmax, engine.test.ts:507-513
    close(orc.softmax([1, 2, 3]), [0.09003057, 0.24472848, 0.66524094], 1e-6, 0)
    close(orc.softmax([1, 1, 1]), [1 / 3] * 3, 1e-6, 0)
    close(orc.softmax([100, 101, 102]), orc.softmax([0, 1, 2]), 1e-6, 0)
    assert abs(orc.softmax([-5, 0, 2.5]).astype(np.float64).sum() - 1) < 1e-6
    # rmsNorm, engine.test.ts:535-545
    inv = 1 / math.sqrt(14 / 3 + 1e-5)
    close(orc.rmsnorm([1, 2, 3], [1, 1, 1]), [inv, 2 * inv, 3 * inv], 1e-5, 0)
    close(orc.rmsnorm([1, 2, 3], [0.5, 0, -0.25], 1e-5, True), [inv * 1.5, 2 * inv, 3 * inv * 0.75], 1e-5, 0)
    # silu, engine.test.ts:547-548
    assert abs(orc.silu(0)) < 1e-6 and abs(orc.silu(1) - 0.731058578) < 1e-6
    # RoPE cos(1), engine.test.ts:550-551
    inv_freq, af = orc.rope_parameters(4, 10000)
    assert abs(orc.apply_rope([1, 0, 0, 1], 4, 1, inv_freq, af)[0] - math.cos(1)) < 1e-5


def test_rmsnorm_against_float64_closed_form_large_offset():
    # normalization.browser.test.ts:1-53: sizes 1..4096 with a 1e4 offset, tol 2e-5
    for n in (1, 7, 64, 896, 4096):
        x = (np.sin(np.arange(n) * 0.37) + 1e4).astype(np.float32)
        w = (1 + 0.1 * np.cos(np.arange(n))).astype(np.float32)
        xd = x.astype(np.float64)
        expected = xd / np.sqrt((xd * xd).mean() + 1e-6) * w
        close(orc.rmsnorm(x, w, 1e-6), expected, 2e-5, 0)


def test_argmax_first_max_and_ties():
    # tsl.browser.test.ts:82-103: [1,7,7,-2] ++ [8,3,6] -> 4
    assert orc.argmax([1, 7, 7, -2, 8, 3, 6]) == 4
    assert orc.argmax([1, 7, 7, -2]) == 1  # first maximum wins (math.ts:585 strict >)
    assert orc.argmax([-np.inf, -np.inf]) == 0
    # engine.test.ts:515-516
    assert orc.argmax([1, 2, 3]) == 2 and orc.argmax([1, 4, 3]) == 1


LOWEST = float(np.float32(-3.4028234663852886e38))


def _brute_topk(logits, k, softcap=0.0):
    """Sort by (score desc, id asc) over the entries above LOWEST_FLOAT; pad
    with (0, LOWEST_FLOAT)."""
    x = np.asarray(logits, np.float32)
    if softcap:
        x = (np.float32(softcap) * np.tanh(x / np.float32(softcap), dtype=np.float32)).astype(np.float32)
    ids = np.arange(len(x))
    valid = x > np.float32(LOWEST)  # NaN compares false
    order = sorted(ids[valid], key=lambda i: (-float(x[i]), int(i)))[:k]
    out = [(int(i), float(x[i])) for i in order]
    return out + [(0, LOWEST)] * (k - len(out))


def test_topk_candidates_known_answers():
    # tsl.browser.test.ts:82-103: chunks [1,7,7,-2] ++ [8,3,6], candidateCount 3
    assert orc.topk_candidates([1, 7, 7, -2, 8, 3, 6], 3, chunk=4) == [(4, 8.0), (1, 7.0), (2, 7.0)]
    assert orc.topk_candidates([1, 7, 7, -2, 8, 3, 6], 1, chunk=4) == [(4, 8.0)]
    # tsl.browser.test.ts:105-120: softcap 1 applied before ranking
    c = orc.topk_candidates([10, 2, -1], 2, softcap=1.0)
    assert c[0][0] == 0 and c[0][1] <= 1 and c[1][0] == 1


@pytest.mark.parametrize("seed", range(6))
def test_topk_candidates_brute_force_and_chunk_invariance(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000))
    x = rng.integers(-20, 20, size=n).astype(np.float32)  # many ties
    for special in (np.inf, -np.inf, np.nan, LOWEST, -LOWEST):
        x[rng.integers(0, n, size=max(1, n // 50))] = special
    for k in (1, 3, 8, 16):
        ref = _brute_topk(x, k)
        for chunk in (1, 7, 64, 8192):
            got = orc.topk_candidates(x, k, chunk=chunk)
            assert [t for t, _ in got] == [t for t, _ in ref], (k, chunk)
            assert np.array_equal(np.float32([v for _, v in got]), np.float32([v for _, v in ref]))
    # fewer valid entries than k: the remaining slots are (0, LOWEST_FLOAT)
    assert orc.topk_candidates([np.nan, -np.inf, 2.0], 3) == [(2, 2.0), (0, LOWEST), (0, LOWEST)]


# --------------------------------------------------------------------- RoPE --

def _scaling(case):
    return recipe.scaling_config(case["config"])


def test_rope_parameters_match_fixture_and_product(hf_fixture):
    for case in hf_fixture["cases"]:
        scaling = _scaling(case)
        inv, af = orc.rope_parameters(8, 10000, scaling)
        close(inv, case["rope"]["inv_freq"], 1e-8, 1e-6)  # rope.test.ts:13
        assert abs(af - case["rope"]["attention_factor"]) < 1e-6
        inv_p, af_p = recipe.rope_parameters(8, 10000.0, scaling)
        assert np.array_equal(inv.view(np.uint32), inv_p.view(np.uint32)) and af == af_p


def test_rope_rotations_match_fixture(hf_fixture):
    for case in hf_fixture["cases"]:
        inv, af = orc.rope_parameters(8, 10000, _scaling(case))
        r = case["rope"]
        for i, pos in enumerate(r["positions"]):
            close(orc.apply_rope(r["query"][i], 8, pos, inv, af), r["rotated_query"][i])
            close(orc.apply_rope(r["key"][i], 8, pos, inv, af), r["rotated_key"][i])


def test_rope_zero_rotation_is_identity():
    v = np.float32([1, 2, 3, 4])
    assert np.array_equal(orc.apply_rope(v, 0, 8, np.zeros(1, np.float32)), v)  # rope.test.ts:43


def test_rope_rejects_invalid():
    with pytest.raises(ValueError):
        orc.rope_parameters(3, 10000)
    with pytest.raises(ValueError):
        orc.rope_parameters(8, 1.0)
    with pytest.raises(recipe.RecipeError):
        recipe.scaling_config({"max_position_embeddings": 64, "rope_scaling": {"rope_type": "dynamic", "factor": 4}})
    with pytest.raises(recipe.RecipeError):
        recipe.recipe_for({"model_type": "llama", "hidden_size": 32, "num_attention_heads": 4, "intermediate_size": 8,
                           "num_hidden_layers": 1, "vocab_size": 8, "rotary_dim": 3})


# ---------------------------------------------------------------- attention --

def _brute_attention(qkv, heads, kv_heads, D, kc, vc, first, pos):
    """float64 attention over an already-filled cache: a different formula path
    (matrix products, scipy-style stable softmax) than the oracle's loops."""
    q = np.asarray(qkv[: heads * D], np.float64).reshape(heads, D)
    out = np.zeros((heads, D))
    for h in range(heads):
        kvh = h * kv_heads // heads
        K = kc[first:pos + 1, kvh * D:(kvh + 1) * D].astype(np.float64)
        V = vc[first:pos + 1, kvh * D:(kvh + 1) * D].astype(np.float64)
        s = K @ q[h] / math.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V
    return out.reshape(-1)


@pytest.mark.parametrize("heads,kv_heads,D,window", [(4, 2, 2, 0), (2, 2, 4, 0), (4, 2, 2, 2), (14, 2, 64, 0),
                                                     (3, 1, 128, 5)])
def test_attention_brute_force_no_rope(heads, kv_heads, D, window):
    rng = np.random.default_rng(heads * 100 + D)
    T = 9
    kv = kv_heads * D
    kc = np.zeros((T, kv), np.float32)
    vc = np.zeros((T, kv), np.float32)
    inv = np.zeros(1, np.float32)
    for pos in range(T):
        qkv = rng.standard_normal(heads * D + 2 * kv).astype(np.float32)
        out = orc.attention(qkv, heads, kv_heads, D, pos, kc, vc, inv, rotary_dim=0, sliding_window=window)
        first = max(0, pos - window + 1) if window > 0 else 0
        close(out, _brute_attention(qkv, heads, kv_heads, D, kc, vc, first, pos), 1e-5, 1e-5)
        if pos == 0:  # a single visible token: the output is that token's V row
            for h in range(heads):
                kvh = h * kv_heads // heads
                assert np.array_equal(out[h * D:(h + 1) * D], vc[0, kvh * D:(kvh + 1) * D])


def test_softmax_shift_invariance_and_kv_f16_rounding():
    s = np.float32([0.5, -1.25, 3.0, 2.0])
    close(orc.softmax(s + 1000), orc.softmax(s), 1e-6, 0)
    heads, kv_heads, D = 2, 1, 8
    kc = np.zeros((2, D), np.float32)
    vc = np.zeros((2, D), np.float32)
    qkv = np.float32(np.sin(np.arange(heads * D + 2 * D)) * 3.1)
    orc.attention(qkv, heads, kv_heads, D, 0, kc, vc, np.zeros(1, np.float32), rotary_dim=0, kv_f16=True)
    assert np.array_equal(vc[0], qkv[heads * D + D:].astype(np.float16).astype(np.float32))


# ------------------------------------------------------------ whole forward --

def oracle_from_hf(fixture, case, fp16_storage=False):
    """Build the oracle model from the fixture tensors the way DecoderWeights
    does for the Llama recipe (DecoderWeights.ts:257-353); fp16_storage rounds
    every weight except the embedding once to fp16 (generate.py:77-84)."""
    cfg = case["config"]
    rec = recipe.recipe_for(cfg, has_lm_head=True)
    T = {k: np.asarray(v["values"], np.float32).reshape(v["shape"]) for k, v in fixture["tensors"].items()}

    def w(name):
        a = T[name]
        return a.astype(np.float16).astype(np.float32) if fp16_storage and name != "model.embed_tokens.weight" else a

    inv, af = rec.rope()
    m = orc.Model(rec.hidden_size, rec.inner_size, rec.layer_count, rec.head_count, rec.kv_head_count, rec.head_dim,
                  rec.vocab_size, 64, rec.norm_eps, inv, af)
    m.set(orc.EMBED, 0, w("model.embed_tokens.weight"))
    m.set(orc.LM_HEAD, 0, w("lm_head.weight") if not rec.tied_embeddings else w("model.embed_tokens.weight"))
    m.set(orc.FINAL_NORM, 0, w("model.norm.weight"))
    for l in range(rec.layer_count):
        p = f"model.layers.{l}."
        m.set(orc.ATTN_NORM, l, w(p + "input_layernorm.weight"))
        m.set(orc.FFN_NORM, l, w(p + "post_attention_layernorm.weight"))
        m.set(orc.WQKV, l, np.concatenate([w(p + "self_attn.q_proj.weight"), w(p + "self_attn.k_proj.weight"),
                                           w(p + "self_attn.v_proj.weight")]))
        m.set(orc.WO, l, w(p + "self_attn.o_proj.weight"))
        m.set(orc.WGATE, l, w(p + "mlp.gate_proj.weight"))
        m.set(orc.WUP, l, w(p + "mlp.up_proj.weight"))
        m.set(orc.WDOWN, l, w(p + "mlp.down_proj.weight"))
    return m


@pytest.mark.parametrize("fp16_storage", [False, True])
def test_forward_matches_hf_fixture(hf_fixture, fp16_storage):
    key_logits = "fp16_storage_logits" if fp16_storage else "logits"
    key_hidden = "fp16_storage_final_hidden" if fp16_storage else "final_hidden"
    for case in hf_fixture["cases"]:
        m = oracle_from_hf(hf_fixture, case, fp16_storage)
        for i, tok in enumerate(hf_fixture["input_ids"]):
            logits, hidden = m.forward(tok, i, want_hidden=True)
            close(logits, case[key_logits][i])
            close(hidden, case[key_hidden][i])
        m.close()


# ----------------------------------------------------------------------- q4 --

def test_q4_dequant_closed_form_exhaustive():
    # every byte value against every scale in a set covering zero, subnormal,
    # normal and the largest finite fp16
    scale_bits = np.uint16([0x0000, 0x0001, 0x03FF, 0x0400, 0x1C00, 0x2E66, 0x3C00, 0x4B00, 0x7BFF])
    N = len(scale_bits)
    packed = np.tile(np.arange(256, dtype=np.uint8)[:16], (N, 1))  # K = 32 -> 16 bytes per row
    packed = np.concatenate([packed] + [np.tile(np.arange(256, dtype=np.uint8)[16 * j:16 * j + 16], (N, 1))
                                        for j in range(1, 16)], axis=1)  # K = 512 covers all 256 bytes
    K = packed.shape[1] * 2
    scales = np.repeat(scale_bits[:, None], K // 32, axis=1)
    out = orc.q4_dequant(packed, scales)
    nib = np.stack([packed & 15, packed >> 4], axis=2).reshape(N, K).astype(np.int32)
    expected = scales.view(np.float16).astype(np.float32).repeat(32, axis=1) * (nib - 8).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))


def test_q4_quantize_round_trip_bound():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[3, :32] = 0  # an all-zero group
    w[5, 40] = 1.5  # an outlier group
    packed, scales = orc.q4_quantize(w)
    deq = orc.q4_dequant(packed, scales)
    s = scales.view(np.float16).astype(np.float32).repeat(32, axis=1)
    assert np.all(np.abs(deq - w) <= s / 2 * (1 + 1e-3) + 1e-12)
    assert scales[3, 0] == 0 and np.all(packed[3, :16] == 0x88)
    nib = np.stack([packed & 15, packed >> 4], axis=2).reshape(64, 256)
    assert nib.max() <= 15
    # the largest magnitude of each group maps to code +-7 (or -8 after clamp)
    g = np.abs(w).reshape(64, 8, 32).argmax(axis=2)
    codes = nib.reshape(64, 8, 32).astype(np.int32) - 8
    top = np.take_along_axis(codes, g[..., None], axis=2)[..., 0]
    assert np.all((np.abs(top) == 7) | (scales == 0))
