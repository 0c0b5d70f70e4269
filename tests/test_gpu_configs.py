"""Whole-model parity at the depth, context and prompt length of the benchmark
configurations (the reference's GPU == CPU greedy contract,
src/test/tsl.browser.test.ts:397-449, and chunked prefill == token-by-token,
src/test/reference.browser.test.ts:35-39):

* Qwen2.5-0.5B shape, 24 layers: the 128-id prompt through the batched
  prefill, then 256 greedy tokens against the oracle.
* Llama-3.2-1B shape, 16 layers: a 4095-id prompt (two chunks, the second
  attending over 2048 earlier rows), batched against the replayed decode
  graph; the oracle continues from the device cache and checks the last
  prompt rows and 32 decode steps (every greedy token, the logits every 8th).
* Llama-3.2-3B shape, 28 layers, 8 decode steps over a 16384-position
  N(0, 1) cache that the oracle is given too.
* The 2048-position prefill chunk of the Llama-3.2-1B shape at 16 layers,
  against the replayed decode graph, and the oracle from the chunk's cache
  rows at its last positions.

Tolerances: logits max-abs 2e-2 / rel 1e-2 (fp16 storage); the greedy stream
is identical except after a step whose oracle top-2 gap is under 2e-2.
"""
import numpy as np
import pytest

from bridge import close, oracle_model, top2_gap
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


def _kv_f32(model, layer, pos0, count):
    k, v = model.kv_read(layer, pos0, count)
    return k.view(np.float16).astype(np.float32), v.view(np.float16).astype(np.float32)


def _say(msg):
    print(msg, flush=True)


@pytest.mark.timeout(300)
def test_qwen_full_prompt_and_256_greedy_tokens(ctx):
    """24 layers; prompt positions 0..126 batched (one chunk of 127 rows), then
    256 greedy steps driven from the host with the oracle fed the device's
    tokens, so every step is compared: the device token is the oracle's argmax
    unless the oracle's top-2 gap is under the tolerance (then either may win),
    and the logits are within tolerance at position 127 and every 32nd step.
    The device loop (decodeGreedy) gives the same 256 tokens as the host loop."""
    wl = W.WORKLOADS["qwen2.5-0.5b"]
    hw = W.synthetic(wl)
    hw.keep = True
    max_tokens = wl.prompt_len + wl.decode_len + 8
    runner = R.DecoderHIPRunner(hw, {"maxTokens": max_tokens}, ctx=ctx)
    assert runner.batchedPrefill
    om = oracle_model(hw, max_tokens, kv_f16=True, threads=16)
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    n = len(prompt) - 1
    runner.prefillTokens(prompt, 0, n)
    for i in range(n):
        om.prefill(prompt[i], i)
    _say("prompt done")
    tok, pos = prompt[-1], n
    device, near_ties, worst = [], [], 0.0
    for step in range(wl.decode_len):
        runner.computeToken(tok, pos + step, True)
        ref = om.forward(tok, pos + step)
        if step % 32 == 0 or step == wl.decode_len - 1:
            got = runner.readLogits()
            close(got, ref, LOGIT_ATOL, LOGIT_RTOL)
            worst = max(worst, float(np.abs(got.astype(np.float64) - ref).max()))
        dev_tok = runner.sampleToken(1, {"temperature": 0})
        if dev_tok != int(np.argmax(ref)):
            assert top2_gap(ref) < LOGIT_ATOL, f"step {step}: token {dev_tok}, oracle {int(np.argmax(ref))}, " \
                                               f"top-2 gap {top2_gap(ref)}"
            near_ties.append(step)
        device.append(dev_tok)
        tok = dev_tok
    _say(f"{len(device)} tokens; near-tie steps where the device took the runner-up: {near_ties}; "
         f"worst |logits - oracle| {worst:.3g}")
    # the device-driven loop (one graph per token, token fed back on the device)
    runner.resetCache()
    runner.prefillTokens(prompt, 0, n)
    runner.computeToken(prompt[-1], n, True)
    first = runner.sampleToken(1, {"temperature": 0})
    loop = [first] + list(runner.decodeGreedy(first, n + 1, len(device) - 1))
    assert loop == device
    runner.close()
    om.close()


@pytest.mark.timeout(300)
def test_llama1b_4095_id_prompt_and_decode(ctx):
    """16 layers, prompt positions 0..4094 batched as chunks of 2048 + 2047
    rows against the replayed decode graph (KV rows of every layer and the
    logits at 4095).  The oracle is then given the batched cache rows
    0..4089 and computes positions 4090..4094 itself (its K/V rows must match
    the device's) and 32 decode steps from 4095: every greedy token (the
    oracle fed the device's tokens) and the logits every 8th step; the device
    loop gives the same tokens."""
    wl = W.WORKLOADS["llama-3.2-1b"]
    L = wl.config["num_hidden_layers"]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens, "prefillChunkSize": 2048}, ctx=ctx)
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    n = len(prompt) - 1
    assert n == 4095
    m = runner.model
    m.set_prefill(0, 2048)  # the reference's semantics: the decode graph once per position
    m.prefill(prompt, 0, n)
    m.compute_token(prompt[-1], n, True)
    replay_logits = m.read_logits()
    replay_kv = [_kv_f32(m, l, 0, n) for l in range(L)]
    _say("replay done")
    m.reset_cache()
    m.set_prefill(runner.prefillBatchRows, 2048)
    runner.prefillTokens(prompt, 0, n)
    runner.computeToken(prompt[-1], n, True)
    logits = runner.readLogits()
    kv = [_kv_f32(m, l, 0, n) for l in range(L)]
    for l in range(L):
        for got, ref in zip(kv[l], replay_kv[l]):
            close(got, ref, 2e-2, 1e-2)
    close(logits, replay_logits, LOGIT_ATOL, LOGIT_RTOL)
    del replay_kv
    _say(f"batched == replay; max |logits - replay| {float(np.abs(logits - replay_logits).max()):.3g}")
    om = oracle_model(hw, wl.max_tokens, kv_f16=True, threads=16)
    p0 = n - 5
    for l in range(L):
        om.write_cache(l, 0, kv[l][0][:p0], kv[l][1][:p0])
    for i in range(p0, n):
        om.prefill(prompt[i], i)
    for l in range(L):
        k_ref, v_ref = om.read_cache(l, n)
        close(kv[l][0][p0:n].reshape(n - p0, -1), k_ref[p0:n], 2e-2, 1e-2)
        close(kv[l][1][p0:n].reshape(n - p0, -1), v_ref[p0:n], 2e-2, 1e-2)
    del kv
    ref = om.forward(prompt[-1], n)
    close(logits, ref, LOGIT_ATOL, LOGIT_RTOL)
    tok = runner.sampleToken(1, {"temperature": 0})
    host = [tok]
    for step in range(1, 32):
        pos = n + step
        if tok != int(np.argmax(ref)):
            assert top2_gap(ref) < LOGIT_ATOL
            break
        runner.computeToken(tok, pos, True)
        ref = om.forward(tok, pos)
        if step % 8 == 0:
            close(runner.readLogits(), ref, LOGIT_ATOL, LOGIT_RTOL)
        tok = runner.sampleToken(1, {"temperature": 0})
        host.append(tok)
    _say(f"oracle checks done ({len(host)} decode steps)")
    # the device-fed loop from the same cache state gives the host loop's tokens
    dev = list(runner.decodeGreedy(host[0], n + 1, len(host) - 1))
    assert dev == host[1:]
    runner.close()
    om.close()


@pytest.mark.timeout(300)
def test_llama3b_decode_over_16384_cached_positions(ctx):
    """28 layers, head_dim 128, the fp16 cache filled with N(0, 1) to 16384
    positions (the matrix-core long-window attention and its 32-slot combine in the O
    projection).  The oracle gets the same cache rows; 8 decode steps at
    16384..16391 (the oracle takes seconds per step at this context): every
    greedy token equal (the oracle fed the device's tokens), the logits
    within tolerance at every 4th step."""
    wl = W.WORKLOADS["llama-3.2-3b"]
    L, fill = wl.config["num_hidden_layers"], wl.kv_prefill
    hw = W.synthetic(wl)
    hw.keep = True
    max_tokens = fill + 24
    runner = R.DecoderHIPRunner(hw, {"maxTokens": max_tokens}, ctx=ctx)
    m = runner.model
    m.kv_fill_normal(0xC0FFEE, fill)
    om = oracle_model(hw, max_tokens, kv_f16=True, threads=16)
    for l in range(L):
        k, v = _kv_f32(m, l, 0, fill)
        om.write_cache(l, 0, k, v)
    _say("caches filled")
    tok = int(W.prompt_tokens(wl)[0])
    for pos in range(fill, fill + 8):
        runner.computeToken(tok, pos, True)
        ref = om.forward(tok, pos)
        if (pos - fill) % 4 == 0:
            close(runner.readLogits(), ref, LOGIT_ATOL, LOGIT_RTOL)
        _say(f"step {pos} checked")
        dev_tok = runner.sampleToken(1, {"temperature": 0})
        if dev_tok != int(np.argmax(ref)):
            assert top2_gap(ref) < LOGIT_ATOL
            break
        tok = dev_tok
    # the rows appended at the first step (every layer) match the oracle's
    for l in range(L):
        k_dev, v_dev = _kv_f32(m, l, fill, 1)
        k_ref, v_ref = om.read_cache(l, fill + 1)
        close(k_dev.reshape(1, -1), k_ref[fill:fill + 1], 2e-2, 1e-2)
        close(v_dev.reshape(1, -1), v_ref[fill:fill + 1], 2e-2, 1e-2)
    runner.close()
    om.close()


@pytest.mark.timeout(300)
def test_llama1b_2048_row_chunk_at_full_depth(ctx):
    """The prefill-chunk workload (Llama-3.2-1B shape, 16 layers, 2048 random
    ids): the batched chunk against the replayed decode graph, KV rows of
    every layer and the logits at position 2048; then the oracle, given the
    batched chunk's cache rows 0..2043, computes positions 2044..2047 itself
    (its K/V rows must match the chunk's) and the logits at 2048."""
    wl = W.WORKLOADS["llama-3.2-1b"]
    L, n = wl.config["num_hidden_layers"], 2048
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": n + 8, "prefillChunkSize": 2048}, ctx=ctx)
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, wl.config["vocab_size"], n + 1)]
    m = runner.model
    m.set_prefill(0, 2048)
    m.prefill(prompt, 0, n)
    m.compute_token(prompt[-1], n, True)
    replay_logits = m.read_logits()
    replay_kv = [_kv_f32(m, l, 0, n) for l in range(L)]
    m.reset_cache()
    m.set_prefill(runner.prefillBatchRows, 2048)
    runner.prefillTokens(prompt, 0, n)
    runner.computeToken(prompt[-1], n, True)
    logits = runner.readLogits()
    for l in range(L):
        for got, ref in zip(_kv_f32(m, l, 0, n), replay_kv[l]):
            close(got, ref, 2e-2, 1e-2)
    close(logits, replay_logits, LOGIT_ATOL, LOGIT_RTOL)
    _say(f"max |logits - replay| {float(np.abs(logits - replay_logits).max()):.3g}")
    del replay_kv
    om = oracle_model(hw, n + 8, kv_f16=True, threads=16)
    p0 = n - 4
    kv = [_kv_f32(m, l, 0, n) for l in range(L)]
    for l in range(L):
        om.write_cache(l, 0, kv[l][0][:p0], kv[l][1][:p0])
    for i in range(p0, n):
        om.prefill(prompt[i], i)
    for l in range(L):
        k_ref, v_ref = om.read_cache(l, n)
        close(kv[l][0][p0:n].reshape(n - p0, -1), k_ref[p0:n], 2e-2, 1e-2)
        close(kv[l][1][p0:n].reshape(n - p0, -1), v_ref[p0:n], 2e-2, 1e-2)
    close(logits, om.forward(prompt[-1], n), LOGIT_ATOL, LOGIT_RTOL)
    _say("oracle from the chunk's cache done")
    om.close()
    runner.close()
