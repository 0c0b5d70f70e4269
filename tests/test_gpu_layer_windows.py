"""Per-layer sliding windows and the attention scale of the model ABI on the
GPU (DecoderCPURunner.attention passes block.slidingWindow and
recipe.attnScale per layer, DecoderCPURunner.ts:140-160; the windows come from
the config's layer_types, DecoderWeights.ts:307-311): the persistent schedule,
the graph of per-stage kernels, the batched prefill and, at positions past
1024, the long-window graph with one layer still on the short-window kernels,
each against the oracle run with the same per-layer options.

Tolerances: logits max-abs 2e-2 / rel 1e-2 against the oracle; persistent vs
per-stage kernels 2e-3 / 1e-3 (the same math, other summation orders).
"""
import os
import re

import pytest

from bridge import close, oracle_model
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


def _weights(window, types, attn_scale, prompt_len, max_tokens):
    wl = W.WORKLOADS["tiny"]
    # intermediate 768 (the tiny config's 688 is no multiple of 32, which the
    # batched prefill's GEMMs need)
    cfg = dict(wl.config, sliding_window=window, layer_types=types, max_position_embeddings=max_tokens,
               intermediate_size=768)
    wl = W.Workload(wl.name + "-layer-windows", cfg, wl.storage, prompt_len, 8, max_tokens)
    hw = W.synthetic(wl)
    hw.keep = True
    hw.recipe.attn_scale = attn_scale
    return wl, hw


def _runner(hw, ctx, max_tokens, persistent, batch_rows=0, chunk=None):
    old = os.environ.get("TLM_PERSISTENT")
    os.environ["TLM_PERSISTENT"] = "1" if persistent else "0"
    try:
        opts = {"maxTokens": max_tokens, "prefillBatchRows": batch_rows}
        if chunk:
            opts["prefillChunkSize"] = chunk
        return R.DecoderHIPRunner(hw, opts, ctx=ctx)
    finally:
        if old is None:
            del os.environ["TLM_PERSISTENT"]
        else:
            os.environ["TLM_PERSISTENT"] = old


def test_layer_windows_and_scale_in_both_decode_schedules(ctx):
    """Layer 0 slides over 8 positions, layer 1 attends to all; softmax scale
    0.1: 40 positions token by token, persistent against per-stage kernels
    every step and against the oracle every 4th."""
    wl, hw = _weights(8, ["sliding_attention", "full_attention"], 0.1, 40, 64)
    assert hw.recipe.layer_windows == [8, 0]
    ps = _runner(hw, ctx, 64, True)
    ref = _runner(hw, ctx, 64, False)
    assert "windows[8,0]" in ps.model.describe()
    assert re.search(r"persistent\[\d+ blocks", ps.model.describe())
    assert "persistent[off]" in ref.model.describe()
    om = oracle_model(hw, 64, kv_f16=True, threads=16)
    toks = [int(t) for t in W.prompt_tokens(wl)][:40]
    for i, t in enumerate(toks):
        ps.computeToken(t, i, True)
        ref.computeToken(t, i, True)
        got = ps.readLogits()
        close(got, ref.readLogits(), 2e-3, 1e-3)
        want = om.forward(t, i)
        if i % 4 == 3:
            close(got, want, LOGIT_ATOL, LOGIT_RTOL)
    ps.close()
    ref.close()
    om.close()


def test_layer_windows_in_the_batched_prefill(ctx):
    """The same model's 40-id prompt as batched row chunks of 16 (each layer's
    flash attention with its own window), then the logits at position 40."""
    wl, hw = _weights(8, ["sliding_attention", "full_attention"], 0.1, 41, 64)
    runner = _runner(hw, ctx, 64, True, batch_rows=8, chunk=16)
    assert runner.batchedPrefill
    om = oracle_model(hw, 64, kv_f16=True, threads=16)
    toks = [int(t) for t in W.prompt_tokens(wl)][:41]
    runner.prefillTokens(toks, 0, 40)
    assert runner.model.counts()["prefill_chunks"] == 3
    for i in range(40):
        om.prefill(toks[i], i)
    runner.computeToken(toks[40], 40, True)
    close(runner.readLogits(), om.forward(toks[40], 40), LOGIT_ATOL, LOGIT_RTOL)
    runner.close()
    om.close()


def test_long_window_graph_with_a_short_window_layer(ctx):
    """Layer 0 slides over 512 positions, layer 1 attends to all 1100+: past
    position 1023 the long-window graph runs, with layer 0 still on the
    short-window kernels.  1100 positions batched, then 3 decode steps."""
    wl, hw = _weights(512, ["sliding_attention", "full_attention"], 0.0, 1103, 1200)
    runner = _runner(hw, ctx, 1200, True, batch_rows=64)
    om = oracle_model(hw, 1200, kv_f16=True, threads=16)
    toks = [int(t) for t in W.prompt_tokens(wl)][:1103]
    runner.prefillTokens(toks, 0, 1100)
    for i in range(1100):
        om.prefill(toks[i], i)
    for i in range(1100, 1103):
        runner.computeToken(toks[i], i, True)
        close(runner.readLogits(), om.forward(toks[i], i), LOGIT_ATOL, LOGIT_RTOL)
    runner.close()
    om.close()


def test_negative_windows_are_refused(ctx):
    wl, hw = _weights(8, None, 0.0, 8, 64)
    desc, inv = hw.model_desc(64)
    with pytest.raises(tlm.TlmError) as e:
        tlm.Model(ctx, desc, inv, layer_windows=[4, -1])
    assert "sliding window" in str(e.value)
    with pytest.raises(ValueError):
        tlm.Model(ctx, desc, inv, layer_windows=[4])

