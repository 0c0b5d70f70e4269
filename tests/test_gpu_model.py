"""Whole-model parity on the GPU: the runner (C ABI + HIP graphs) against the
pinned Hugging Face fixture and against the CPU oracle fed the same bytes.

Tolerances: the north-star contract for logits is max-abs 2e-2 / rel 1e-2
with fp16 weights/cache; greedy streams must be identical except after a step
where the oracle's top-2 logit gap is under that tolerance.
"""
import numpy as np
import pytest

from bridge import close, oracle_model, top2_gap
from oracle import oracle as orc
import three_llm_amd.runner as R
import three_llm_amd.tlm as tlm
import three_llm_amd.weights as W

pytestmark = pytest.mark.gpu
LOGIT_ATOL, LOGIT_RTOL = 2e-2, 1e-2


@pytest.fixture(scope="module")
def ctx():
    c = tlm.Context(0)
    yield c
    c.close()


def fixture_tensors(hf):
    return {k: np.asarray(v["values"], np.float32).reshape(v["shape"]) for k, v in hf["tensors"].items()}


@pytest.mark.parametrize("case_index", range(5))
def test_hf_fixture_fp16_storage_on_gpu(ctx, hf_fixture, case_index):
    """reference.browser.test.ts:7-40 on the device: fp16 weights (embedding
    fp32, like the fixture's fp16-storage contract), fp32 KV cache."""
    case = hf_fixture["cases"][case_index]
    # the fixture rounds every parameter except the embedding to fp16 once
    # (scripts/reference/generate.py:77-84), norm weights included
    tensors = {k: (v if k == "model.embed_tokens.weight" else v.astype(np.float16).astype(np.float32))
               for k, v in fixture_tensors(hf_fixture).items()}
    hw = W.from_hf(case["config"], tensors, W.Storage(linear="f16", head="f16", embed="f32", kv="f32"))
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 64}, ctx=ctx)
    om = oracle_model(hw, 64, kv_f16=False)
    ids = hf_fixture["input_ids"]
    for i, tok in enumerate(ids):
        runner.computeToken(tok, i, True)
        logits = runner.readLogits()
        close(logits, case["fp16_storage_logits"][i], 3e-5, 2e-4)  # reference.browser.test.ts:16 hardware atol
        close(runner.model.read_hidden(), case["fp16_storage_final_hidden"][i], 3e-5, 2e-4)
        close(logits, om.forward(tok, i), 1e-5, 1e-4)
    # chunked prefill equals the token-by-token result (reference.browser.test.ts:35-39)
    runner.resetCache()
    runner.prefillChunkSize = 7
    runner.prefillTokens(ids, 0, 18)
    runner.computeToken(ids[18], 18, True)
    close(runner.readLogits(), case["fp16_storage_logits"][18], 3e-5, 2e-4)
    runner.close()
    om.close()


def greedy_against_oracle(runner, om, prompt, n_decode, check_every=1):
    """Host-driven prompt + device greedy decode; returns (device stream, oracle stream)."""
    for i, t in enumerate(prompt[:-1]):
        runner.computeToken(int(t), i, False)
        om.forward(int(t), i)
    pos = len(prompt) - 1
    runner.computeToken(int(prompt[-1]), pos, True)
    dev_logits = runner.readLogits()
    ref_logits = om.forward(int(prompt[-1]), pos)
    close(dev_logits, ref_logits, LOGIT_ATOL, LOGIT_RTOL)
    first = runner.sampleToken(1, {"temperature": 0})
    assert first == int(np.argmax(dev_logits))
    device_stream = [first] + list(runner.decodeGreedy(first, pos + 1, n_decode - 1))
    oracle_stream = []
    tok = int(np.argmax(ref_logits))
    gaps = [top2_gap(ref_logits)]
    for step in range(n_decode):
        oracle_stream.append(tok)
        if step == n_decode - 1:
            break
        if device_stream[step] != tok:
            break
        ref_logits = om.forward(tok, pos + 1 + step)
        gaps.append(top2_gap(ref_logits))
        tok = int(np.argmax(ref_logits))
    return device_stream, oracle_stream, gaps


def assert_streams_match(device_stream, oracle_stream, gaps):
    for i, (a, b) in enumerate(zip(device_stream, oracle_stream)):
        if a != b:
            assert gaps[i] < LOGIT_ATOL, f"stream diverged at step {i} with top-2 gap {gaps[i]}"
            return
    assert len(oracle_stream) == len(device_stream)


def test_tiny_config_greedy_stream(ctx):
    """Tiny Llama-style config (2 x 256, fp16 weights): prompt 16, decode 32."""
    wl = W.WORKLOADS["tiny"]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens}, ctx=ctx)
    om = oracle_model(hw, wl.max_tokens, kv_f16=True)
    prompt = W.prompt_tokens(wl)
    dev, ref, gaps = greedy_against_oracle(runner, om, prompt, wl.decode_len)
    print("device:", dev)
    assert_streams_match(dev, ref, gaps)
    runner.close()
    om.close()


def test_decode_reaches_the_last_cache_position(ctx):
    """Tiny config with a 40-position cache: prompt 16, then greedy decode
    through position 39 (the last row of the cache) equal to the oracle's
    stream; position 40 is refused."""
    wl = W.WORKLOADS["tiny"]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 40}, ctx=ctx)
    om = oracle_model(hw, 40, kv_f16=True)
    prompt = W.prompt_tokens(wl)[:16]
    dev, ref, gaps = greedy_against_oracle(runner, om, prompt, 25)
    assert_streams_match(dev, ref, gaps)
    with pytest.raises(tlm.TlmError):
        runner.computeToken(int(dev[-1]), 40, True)
    runner.close()
    om.close()


@pytest.mark.parametrize("gqa,prompt_len,max_tokens,plan", [
    ("0", 1100, 2200, "nsplit=69/18 G=4]"), ("1", 4400, 4500, "nsplit=141/32 G=4 long=mfma]")],
    ids=["one-head-blocks", "matrix-core"])
def test_long_window_decode_with_more_than_16_chunks(ctx, monkeypatch, gqa, prompt_len, max_tokens, plan):
    """One kv head and four query heads, past the 1024-position window where
    the long-window kernels take over, with more long-window chunks per query
    head than the 16 the O projection's prologue folds per round trip (its
    32-slot form): the one-head-per-block kernel (TLM_GQA=0) has 18 chunks of
    at least 32 positions at 1100 positions; the matrix-core kernel, one block
    per kv head and chunk, has 32 chunks of 138 positions at 4400.  The
    prompt runs as a batched prefill, then the logits at the next four
    positions are checked against the oracle."""
    monkeypatch.setenv("TLM_GQA", gqa)
    cfg = {"model_type": "llama", "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
           "num_attention_heads": 4, "num_key_value_heads": 1, "head_dim": 64, "vocab_size": 2048,
           "rope_theta": 1e4, "rms_norm_eps": 1e-6, "tie_word_embeddings": True,
           "max_position_embeddings": 8192, "eos_token_id": -1}
    wl = W.Workload("long-window-1kv", cfg, W.Storage(linear="q4", head="f16", embed="f16"), prompt_len + 4, 1,
                    max_tokens)
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens}, ctx=ctx)
    assert plan in runner.model.describe()
    om = oracle_model(hw, wl.max_tokens, kv_f16=True, threads=16)
    prompt = W.prompt_tokens(wl)
    runner.prefillTokens([int(x) for x in prompt[:prompt_len]], 0, prompt_len)
    for i in range(prompt_len):
        om.prefill(int(prompt[i]), i)
    for i in range(prompt_len, prompt_len + 4):
        runner.computeToken(int(prompt[i]), i, True)
        close(runner.readLogits(), om.forward(int(prompt[i]), i), LOGIT_ATOL, LOGIT_RTOL)
    runner.close()
    om.close()


def test_qwen_shape_with_bias_past_1024_positions(ctx):
    """Two layers of the Qwen2.5-0.5B shape (QKV bias, 7 query heads per kv
    head, head_dim 64) over a 1100-id prompt (batched prefill), then three
    decode steps in the long-window mode, where the matrix-core attention adds
    the bias to the QKV partials: logits against the oracle at 2e-2 / 1e-2."""
    wl = W.WORKLOADS["qwen2.5-0.5b"]
    cfg = dict(wl.config, num_hidden_layers=2)
    wl = W.Workload(wl.name + "-2l-long", cfg, wl.storage, 1103, 1, 1200, qkv_bias=True)
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens}, ctx=ctx)
    assert "long=mfma" in runner.model.describe()
    om = oracle_model(hw, wl.max_tokens, kv_f16=True, threads=16)
    prompt = [int(x) for x in W.prompt_tokens(wl)]
    runner.prefillTokens(prompt[:1100], 0, 1100)
    for i in range(1100):
        om.prefill(prompt[i], i)
    for i in range(1100, 1103):
        runner.computeToken(prompt[i], i, True)
        close(runner.readLogits(), om.forward(prompt[i], i), LOGIT_ATOL, LOGIT_RTOL)
    runner.close()
    om.close()


def _reduced_qwen(layers):
    wl = W.WORKLOADS["qwen2.5-0.5b"]
    cfg = dict(wl.config, num_hidden_layers=layers)
    return W.Workload(wl.name + f"-{layers}l", cfg, wl.storage, 8, 8, 1024, qkv_bias=True)


@pytest.mark.parametrize("layers", [2, 24])
def test_qwen_shape_q4_against_oracle(ctx, layers):
    """Qwen2.5-0.5B shape (q4 linears, fp16 tied head, QKV bias): logits within
    2e-2/1e-2 and the greedy stream equal, with 2 layers and with all 24."""
    wl = _reduced_qwen(layers)
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens}, ctx=ctx)
    om = oracle_model(hw, wl.max_tokens, kv_f16=True, threads=16)
    prompt = W.prompt_tokens(wl)
    dev, ref, gaps = greedy_against_oracle(runner, om, prompt, 6)
    print("device:", dev, "oracle:", ref)
    assert_streams_match(dev, ref, gaps)
    runner.close()
    om.close()


def _reduced(name, layers, prompt_len=8):
    wl = W.WORKLOADS[name]
    cfg = dict(wl.config, num_hidden_layers=layers)
    return W.Workload(wl.name + f"-{layers}l", cfg, wl.storage, prompt_len, 6, 512, qkv_bias=wl.qkv_bias)


@pytest.mark.parametrize("name", ["llama-3.2-1b", "llama-3.2-3b"])
def test_llama_shapes_q4_against_oracle(ctx, name):
    """Llama-3.2-1B (hidden 2048, 32/8 heads, head_dim 64) and 3B (hidden 3072,
    24/8 heads, head_dim 128) shapes with 2 layers: q4 linears, fp16 tied head,
    fp16 cache; logits within 2e-2/1e-2 and the greedy stream equal."""
    wl = _reduced(name, 2)
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens}, ctx=ctx)
    om = oracle_model(hw, wl.max_tokens, kv_f16=True, threads=16)
    prompt = W.prompt_tokens(wl)
    dev, ref, gaps = greedy_against_oracle(runner, om, prompt, 6)
    print(name, "device:", dev, "oracle:", ref)
    assert_streams_match(dev, ref, gaps)
    runner.close()
    om.close()


def test_device_loop_equals_host_loop(ctx):
    wl = W.WORKLOADS["tiny"]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 256}, ctx=ctx)
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    runner.prefillTokens(prompt, 0, len(prompt) - 1)
    runner.computeToken(prompt[-1], len(prompt) - 1, True)
    first = runner.sampleToken(1, {"temperature": 0})
    device = list(runner.decodeGreedy(first, len(prompt), 10))
    runner.resetCache()
    for i, t in enumerate(prompt):
        runner.computeToken(t, i, i == len(prompt) - 1)
    host = []
    tok = runner.sampleToken(1, {"temperature": 0})
    assert tok == first
    for step in range(10):
        runner.computeToken(tok, len(prompt) + step, True)
        tok = runner.sampleToken(1, {"temperature": 0})
        host.append(tok)
    assert device == host
    # generate() drives the same controls (generate.ts:210-305)
    runner.resetCache()
    res = runner.generate("", {"inputTokens": prompt, "temperature": 0, "maxNewTokens": 11})
    assert res["generatedTokens"] == [first] + device
    runner.close()


def test_kv_cache_round_trip_and_reset(ctx):
    wl = W.WORKLOADS["tiny"]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 64}, ctx=ctx)
    m = runner.model
    k = np.arange(5 * 2 * 64, dtype=np.uint16).reshape(5, 2, 64)
    v = (k + 7).astype(np.uint16)
    m.kv_write(1, 3, k, v)
    k2, v2 = m.kv_read(1, 3, 5)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)
    m.reset_cache()
    k3, _ = m.kv_read(1, 3, 5)
    assert not k3.any()
    # the reset clears only the rows that can hold values (every path that
    # writes rows extends that range): a prefill, a device-fed decode and a
    # filled cache, then a reset, leave every row of every layer zero
    for fill in (False, True):
        if fill:
            m.kv_fill_normal(3, 40)
        runner.prefillTokens(list(range(1, 21)), 0, 20)
        runner.decodeGreedy(5, 20, 10)
        rows = np.concatenate([np.concatenate(m.kv_read(l, 0, 64)).ravel() for l in range(hw.recipe.layer_count)])
        assert rows.any()
        m.reset_cache()
        rows = np.concatenate([np.concatenate(m.kv_read(l, 0, 64)).ravel() for l in range(hw.recipe.layer_count)])
        assert not rows.any(), f"rows left after a reset (fill {fill})"
    with pytest.raises(tlm.TlmError):
        runner.computeToken(10 ** 6, 0, True)
    with pytest.raises(tlm.TlmError):
        runner.computeToken(1, 64, True)
    # host buffers the library would read past, or of the wrong element type
    with pytest.raises(tlm.TlmError):
        m.kv_write(1, 3, k.astype(np.float32), v)
    with pytest.raises(tlm.TlmError):
        m.kv_write(1, 3, k[:, :1], v[:, :1])
    with pytest.raises(tlm.TlmError):
        m.kv_write(1, 3, k, v[:4])
    with pytest.raises(tlm.TlmError):
        m.prefill([1, 2, 3], 0, 4)
    runner.close()


def test_device_top_k_sampling_matches_full_logit_sampling(ctx):
    """readCandidates equals the oracle's candidate levels over the device
    logits, and generate() with device top-k sampling (TSLLogitSampler) gives
    the same tokens as sampling from the full logits on the host
    (sampleTopK, math.ts:549-593) with the same random draws."""
    import random as _random
    wl = W.WORKLOADS["tiny"]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 128}, ctx=ctx)
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    for i, t in enumerate(prompt):
        runner.computeToken(t, i, i == len(prompt) - 1)
    logits = runner.readLogits()
    for k in (1, 5, 8):
        assert runner.readCandidates(k) == orc.topk_candidates(logits, k)
    streams = []
    for gpu in (True, False):
        runner.resetCache()
        rnd = _random.Random(1234)
        res = runner.generate("", {"inputTokens": prompt, "temperature": 0.9, "topK": 5, "maxNewTokens": 24,
                                   "gpuSampling": gpu, "random": rnd.random})
        streams.append(res["generatedTokens"])
    print("sampled:", streams[0])
    assert streams[0] == streams[1] and len(streams[0]) == 24
    runner.close()
