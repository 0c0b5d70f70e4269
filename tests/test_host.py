"""CPU-side checks of the host layer: the C ABI library loads and exports every
symbol of include/tlm.h, the host helpers agree with the oracle, and the
restated generate loop matches the reference's own tests."""
import ctypes
import re

import numpy as np
import pytest

from conftest import ROOT
from oracle import oracle as orc
import three_llm_amd.generate as gen
import three_llm_amd.tlm as tlm
import three_llm_amd.weights as W


def header_functions():
    text = (ROOT / "include" / "tlm.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tlm_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(str(tlm.LIB_PATH))
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(tlm.EXPORTS) == names
    assert tlm.lib().tlm_abi_version() == 3


def header_struct_fields(name):
    """Field names of `typedef struct name {...} name;` in include/tlm.h."""
    text = (ROOT / "include" / "tlm.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if decl:
            fields += [n.strip().lstrip("*") for n in re.sub(r"^[\w\s\*]*?(?=\**\w+\s*(,|$))", "", decl,
                                                              count=1).split(",")]
    return fields


@pytest.mark.parametrize("cname,pytype", [("tlm_model_desc", tlm.ModelDesc), ("tlm_attn_desc", tlm.AttnDesc),
                                          ("tlm_model_counts", tlm.ModelCounts)])
def test_ctypes_structs_match_the_header(cname, pytype):
    """The ctypes mirrors name the header's fields in the header's order (a
    missing or extra field shifts every later one)."""
    assert [f for f, _ in pytype._fields_] == header_struct_fields(cname)


def test_open_reports_errors_through_last_error():
    # here there is no GPU: tlm_open must fail with a message, never fall back
    p = ctypes.c_void_p()
    rc = tlm.lib().tlm_open(0, ctypes.byref(p))
    if rc != 0:
        assert tlm.lib().tlm_last_error().startswith(b"HIP") or b"TLMContext" in tlm.lib().tlm_last_error()
        with pytest.raises(tlm.TlmError):
            tlm.Context(0)
    else:
        tlm.lib().tlm_close(p)
    assert tlm.lib().tlm_open(-1, ctypes.byref(p)) != 0


def test_product_quantizer_matches_oracle_bytes():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((96, 320)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    w[1, 5] = 3.0
    w[2, :32] = np.float32(7 * 6.0e-8)  # subnormal-range scale
    p1, s1 = tlm.quantize_q4(w)
    p2, s2 = orc.q4_quantize(w)
    assert np.array_equal(p1, p2) and np.array_equal(s1, s2)


def test_product_f16_rounding_matches_numpy():
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(200000) * np.exp(rng.uniform(-20, 12, 200000))).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = a.astype(np.float16).view(np.uint16)
    assert np.array_equal(tlm.f32_to_f16(a), ref)


def test_synthetic_generator_is_deterministic_and_normal():
    a = tlm.synth_normal(1, 7, 1 << 20, 0.02)
    b = tlm.synth_normal(1, 7, 1 << 20, 0.02)
    c = tlm.synth_normal(1, 8, 1 << 20, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 2e-4
    # prefix property: stream contents do not depend on n (odd n too)
    assert np.array_equal(tlm.synth_normal(1, 7, 1001, 0.02)[:1000], a[:1000])
    t = tlm.synth_tokens(3, 9, 10000, 151936)
    assert t.min() >= 0 and t.max() < 151936 and len(np.unique(t)) > 9000


def test_workload_shapes_match_configs():
    hw = W.synthetic(W.WORKLOADS["qwen2.5-0.5b"])
    r = hw.recipe
    assert (r.hidden_size, r.layer_count, r.head_count, r.kv_head_count, r.head_dim) == (896, 24, 14, 2, 64)
    assert r.tied_embeddings and r.qkv_bias and r.vocab_size == 151936 and r.rope_theta == 1e6
    assert hw.shape(W.WQKV) == (1152, 896) and hw.shape(W.WDOWN) == (896, 4864)
    q = hw.fp32(W.WO, 3)
    assert q.shape == (896, 896) and abs(q.std() - 0.02) < 1e-3
    tiny = W.synthetic(W.WORKLOADS["tiny"])
    assert not tiny.recipe.tied_embeddings and tiny.fmt(W.WQKV) == "f16"


# -------------------------------------------- generate loop (engine.test.ts) --

def test_sample_top_k_known_answers():
    # engine.test.ts:514-525
    assert gen.sample_top_k(np.float32([1, 2, 3]), topK=1) == 2
    assert gen.sample_top_k(np.float32([1, 4, 3]), temperature=0, topK=40) == 1
    assert gen.sample_top_k(np.float32([1, 2, 3, 4]), topK=2, temperature=1, random=lambda: 0) == 3
    assert gen.sample_top_k(np.float32([1, 2, 3, 4]), temperature=1e-8, topK=40, random=lambda: 0.5) == 3
    assert gen.sample_top_k(np.float32([5, 4]), temperature=0, tokens=[0], repetitionPenalty=2) == 1
    assert gen.sample_top_k(np.float32([3, 2, 1]), temperature=0, tokens=[0, 0], frequencyPenalty=1) == 1
    assert gen.sample_top_k(np.float32([0, 0, 10, 1]), temperature=0, tokens=[0, 1, 2, 0, 1],
                            noRepeatNgramSize=3) == 3
    assert gen.sample_top_k(np.float32([5, 4]), temperature=0, tokens=[0], repetitionPenalty=1) == 0


@pytest.mark.parametrize("top_k", [0, -1, 1.9])
def test_topk_normalisation(top_k):
    # runtime/sampling.test.ts:5-9
    opts = {"topK": top_k, "temperature": 1, "random": lambda: 0.99}
    assert gen.gpu_candidate_count(opts, 8) == 1
    assert gen.sample_top_k(np.float32([1, 3, 2]), topK=top_k, temperature=1, random=lambda: 0.99) == 1


def test_prompt_cache_plan():
    # engine.test.ts:793-808
    assert gen.shared_prefix_length([1, 2, 3], [1, 2, 9]) == 2
    assert gen.shared_prefix_length([1, 2], [1, 2, 3]) == 2
    a = gen.plan_prompt_cache([1, 2, 3], np.float32([0]), [1, 2, 3, 4], True)
    assert a.start == 3 and not a.reset and a.logits is not None
    r = gen.plan_prompt_cache([1, 2, 3, 9], np.float32([0]), [1, 2, 4], True)
    assert r.start == 2 and not r.reset
    assert gen.plan_prompt_cache([1, 2, 3, 9], np.float32([0]), [1, 2, 4], False).reset
    assert gen.prepare_generation_from_tokens([1, 2], 8, 0, 0) == ([1, 2], 0)


class _FakeWeights:
    endOfTextTokenId = 0
    stopTokenIds = []

    class tokenizer:
        @staticmethod
        def decode(t):
            return ",".join(map(str, t))

    @staticmethod
    def prepareGeneration(prompt, max_tokens, max_new):
        return [1, 2, 3, 4], 1


class _FakeRunner:
    maxTokens = 8
    weights = _FakeWeights()
    _cacheTokens = None
    _cacheLogits = None


def test_generate_reports_prefill_progress():
    # engine.test.ts:840-889
    progress, computed = [], []

    def prefill(tokens, start, end, on_progress):
        assert list(tokens) == [1, 2, 3, 4] and (start, end) == (0, 3)
        on_progress(2)
        on_progress(3)

    res = gen.generate(_FakeRunner(), "prompt",
                       {"temperature": 0, "topK": 1, "onPrefillProgress": lambda e: progress.append(
                           e["completedPromptTokens"]), "gpuSampling": False},
                       gen.GenerateControls(rewindable=True, resetCache=lambda: None,
                                            computeToken=lambda t, p, c, k: computed.append([t, p]),
                                            readLogits=lambda: np.float32([0, 1]), prefillTokens=prefill))
    assert progress == [2, 3, 4]
    assert computed == [[4, 3], [1, 4]]
    assert res["generatedTokens"] == [1]
