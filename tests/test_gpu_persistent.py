"""The persistent per-token schedule (one kernel per decode token: every CU
runs fixed stage items of every layer and hands sequence-tagged partial sums
to the next stage through device memory) against the graph of per-stage
kernels and against the oracle.  The reference runs one submission per token
(DecoderTSLRunner.ts:487-502); both schedules give the same logits.

Tolerances: persistent vs per-stage kernels max-abs 1e-2 / rel 5e-3 (the
persistent q4 linears dot fp16 copies of their inputs, two weights per
v_dot2_f32_f16 with fp32 sums, where the per-stage kernels keep fp32 inputs;
the fp16 rounding, 2^-11 relative per input, is the difference), and 2e-3 /
1e-3 for fp16 weights (the same math with other fp32 summation orders); both
against the oracle max-abs 2e-2 / rel 1e-2, greedy tokens equal unless the
oracle's top-2 gap is under 2e-2.
"""
import os
import re
import threading
import time

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


def _workload(name, layers, max_tokens):
    wl = W.WORKLOADS[name]
    cfg = dict(wl.config, num_hidden_layers=layers)
    return W.Workload(wl.name, cfg, wl.storage, wl.prompt_len, 8, max_tokens, qkv_bias=wl.qkv_bias)


def _runner(hw, ctx, max_tokens, persistent):
    old = os.environ.get("TLM_PERSISTENT")
    os.environ["TLM_PERSISTENT"] = "1" if persistent else "0"
    try:
        return R.DecoderHIPRunner(hw, {"maxTokens": max_tokens, "prefillBatchRows": 0}, ctx=ctx)
    finally:
        if old is None:
            del os.environ["TLM_PERSISTENT"]
        else:
            os.environ["TLM_PERSISTENT"] = old


@pytest.mark.parametrize("name,layers", [("tiny", 2), ("qwen2.5-0.5b", 4), ("llama-3.2-1b", 2)])
def test_persistent_equals_stage_kernels_and_oracle(ctx, name, layers):
    wl = _workload(name, layers, 256)
    hw = W.synthetic(wl)
    hw.keep = True
    ps = _runner(hw, ctx, 256, True)
    ref = _runner(hw, ctx, 256, False)
    assert "persistent[off]" in ref.model.describe()
    desc = ps.model.describe()
    assert re.search(r"persistent\[\d+ blocks", desc), desc
    om = oracle_model(hw, 256, kv_f16=True, threads=16)
    prompt = [int(t) for t in W.prompt_tokens(wl)][:10]
    atol, rtol = (1e-2, 5e-3) if hw.storage.linear == "q4" else (2e-3, 1e-3)
    for i, t in enumerate(prompt):
        ps.computeToken(t, i, True)
        ref.computeToken(t, i, True)
        got = ps.readLogits()
        close(got, ref.readLogits(), atol, rtol)
        close(got, om.forward(t, i), LOGIT_ATOL, LOGIT_RTOL)
    L = wl.config["num_hidden_layers"]
    for l in range(L):  # the appended cache rows agree too
        for a, b in zip(ps.model.kv_read(l, 0, len(prompt)), ref.model.kv_read(l, 0, len(prompt))):
            close(a.view(np.float16).astype(np.float32), b.view(np.float16).astype(np.float32), atol, rtol)
    assert ps.model.counts()["recomputed_positions"] == 0  # no token was flagged
    # the device-driven greedy loop (one persistent kernel + head per token)
    tok = ps.sampleToken(1, {"temperature": 0})
    assert tok == ref.sampleToken(1, {"temperature": 0})
    dev = list(ps.decodeGreedy(tok, len(prompt), 6))
    t = tok
    for step, d in enumerate(dev):
        r = om.forward(t, len(prompt) + step)
        if d != int(np.argmax(r)):
            assert top2_gap(r) < LOGIT_ATOL
            break
        t = d
    ps.close()
    ref.close()
    om.close()


def test_trace_orders_every_stage(ctx):
    """tlm_trace_decode: per block and layer, each item's stamps run issue <=
    ready <= computed <= published, and a stage is ready only after every
    item of the stage it reads has published (the handoff is a dependency):
    the k|v and attention items read the previous layer's down partials (the
    attention items compute q themselves), O the attention outputs, gate|up
    O's partials, down gate|up's."""
    wl = _workload("qwen2.5-0.5b", 3, 256)
    hw = W.synthetic(wl)
    ps = _runner(hw, ctx, 256, True)
    nb = int(re.search(r"persistent\[(\d+) blocks", ps.model.describe()).group(1))
    tr = ps.model.trace_decode(5, 20, 3, nb).astype(np.int64)[:, 0]  # wave 0: [block][layer][stage][event]
    L = 3
    used = [np.where(tr[:, 0, st, 0] > 0)[0] for st in range(5)]
    assert all(len(u) > 0 for u in used)
    for st in range(5):
        ev = tr[used[st], :L, st, :]
        assert (ev > 0).all()
        assert (np.diff(ev, axis=-1) >= 0).all()
    for l in range(L):
        for st in range(2, 5):
            prev_pub = tr[used[st - 1], l, st - 1, 3].min()
            assert tr[used[st], l, st, 1].min() >= prev_pub
        if l > 0:
            for st in (0, 1):
                assert tr[used[st], l, st, 1].min() >= tr[used[4], l - 1, 4, 3].min()
    with pytest.raises(tlm.TlmError):
        ps.model.trace_decode(5, 20, 3, nb + 1)
    ps.close()


def test_l2_handoffs_give_the_bits_of_device_scope_handoffs(ctx):
    """At the Qwen2.5-0.5B shape the k|v, attention and O items of each O
    split (one kv head's group: 4 k|v, 7 attention and 14 O items) share one
    class of blocks (equal b % 8), which the hardware runs on one XCD, and the
    k|v and attention items publish with plain stores into that XCD's L2.  The
    arithmetic is the same as with every handoff device-scope (TLM_PS_L2=0),
    so the logits, the appended cache rows and the greedy tokens are equal
    bit for bit."""
    wl = _workload("qwen2.5-0.5b", 4, 256)
    hw = W.synthetic(wl)
    hw.keep = True
    l2 = _runner(hw, ctx, 256, True)
    old = os.environ.get("TLM_PS_L2")
    os.environ["TLM_PS_L2"] = "0"
    try:
        dev = _runner(hw, ctx, 256, True)
    finally:
        if old is None:
            del os.environ["TLM_PS_L2"]
        else:
            os.environ["TLM_PS_L2"] = old
    n = int(re.search(r"(\d+) publish through their XCD's L2", l2.model.describe()).group(1))
    assert n == 8 + 14  # every k|v and attention item
    assert "; 0 publish through their XCD's L2" in dev.model.describe()
    prompt = [int(t) for t in W.prompt_tokens(wl)][:12]
    for i, t in enumerate(prompt):
        l2.computeToken(t, i, True)
        dev.computeToken(t, i, True)
        np.testing.assert_array_equal(l2.readLogits(), dev.readLogits())
    for l in range(wl.config["num_hidden_layers"]):
        for a, b in zip(l2.model.kv_read(l, 0, len(prompt)), dev.model.kv_read(l, 0, len(prompt))):
            np.testing.assert_array_equal(a, b)
    tok = l2.sampleToken(1, {"temperature": 0})
    assert tok == dev.sampleToken(1, {"temperature": 0})
    assert list(l2.decodeGreedy(tok, len(prompt), 16)) == list(dev.decodeGreedy(tok, len(prompt), 16))
    assert l2.model.counts()["recomputed_positions"] == 0
    assert dev.model.counts()["recomputed_positions"] == 0
    l2.close()
    dev.close()


def test_persistent_attention_across_the_wave_ranges(ctx):
    """Every window length the persistent attention item splits differently,
    up to its last one (1024 positions): its 16 waves take 32-position ranges
    of the cached rows up to 512 positions and 64-position ranges after that,
    and the last wave also takes the row at pos (alone while its range is
    empty, after its range from 481 cached rows on).  The tiny decoder runs
    1024 positions token by token through the persistent schedule and the
    per-stage graph; logits are compared at the boundaries of those splits
    (and against the oracle, which runs every position), and the appended
    cache rows at the end."""
    wl = _workload("tiny", 2, 1024)
    hw = W.synthetic(wl)
    hw.keep = True
    ps = _runner(hw, ctx, 1024, True)
    ref = _runner(hw, ctx, 1024, False)
    assert re.search(r"persistent\[\d+ blocks", ps.model.describe())
    om = oracle_model(hw, 1024, kv_f16=True, threads=16)
    rng = np.random.default_rng(7)
    toks = [int(t) for t in rng.integers(0, wl.config["vocab_size"], 1024)]
    check = {0, 1, 31, 32, 33, 479, 480, 481, 482, 496, 511, 512, 513, 514, 700, 993, 1022, 1023}
    for i, t in enumerate(toks):
        ps.computeToken(t, i, i in check)
        ref.computeToken(t, i, i in check)
        if i in check:
            got = ps.readLogits()
            close(got, ref.readLogits(), 2e-3, 1e-3)
            close(got, om.forward(t, i), LOGIT_ATOL, LOGIT_RTOL)
        else:
            om.prefill(t, i)
    for l in range(wl.config["num_hidden_layers"]):
        for a, b in zip(ps.model.kv_read(l, 0, 1024), ref.model.kv_read(l, 0, 1024)):
            close(a.view(np.float16).astype(np.float32), b.view(np.float16).astype(np.float32), 2e-3, 1e-3)
    ps.close()
    ref.close()
    om.close()


@pytest.mark.parametrize("window,rotary", [(32, 64), (48, 32)])
def test_persistent_sliding_window_and_partial_rotary(ctx, window, rotary):
    """The tiny decoder with a sliding window (positions past it leave the
    attention range, TSLAttention.ts:306-428) and, in the second case, RoPE on
    the first 32 of 64 dims: 80 positions through the persistent schedule
    against the per-stage graph and, every 8th, the oracle."""
    wl = W.WORKLOADS["tiny"]
    cfg = dict(wl.config, sliding_window=window)
    if rotary != cfg["head_dim"]:
        cfg["partial_rotary_factor"] = rotary / cfg["head_dim"]
    wl = W.Workload(wl.name + "-window", cfg, wl.storage, 80, 8, 128)
    hw = W.synthetic(wl)
    hw.keep = True
    assert hw.recipe.sliding_window == window and hw.recipe.rotary_dim == rotary
    ps = _runner(hw, ctx, 128, True)
    ref = _runner(hw, ctx, 128, False)
    assert re.search(r"persistent\[\d+ blocks", ps.model.describe())
    om = oracle_model(hw, 128, kv_f16=True, threads=16)
    toks = [int(t) for t in W.prompt_tokens(wl)][:80]
    for i, t in enumerate(toks):
        ps.computeToken(t, i, True)
        ref.computeToken(t, i, True)
        got = ps.readLogits()
        close(got, ref.readLogits(), 2e-3, 1e-3)
        want = om.forward(t, i)
        if i % 8 == 7:
            close(got, want, LOGIT_ATOL, LOGIT_RTOL)
    ps.close()
    ref.close()
    om.close()


def test_a_wait_that_runs_out_is_recomputed_and_every_block_leaves(ctx):
    """The failure path of the bounded waits, forced from the host: layer 1's
    QKV items report a time-out without waiting (TLM_PS_FAIL_LAYER), so every
    item that depends on them runs out its own wait (TLM_PS_TIMEOUT_US: 2 ms
    instead of 100) and its block leaves.  The kernel ends, and the read that
    follows finds the flag and recomputes the tokens enqueued since the last
    read on the per-stage graph: it returns the oracle's logits (and a greedy
    run the oracle's tokens), and the model keeps its persistent schedule,
    with every handoff device-scope from then on."""
    wl = _workload("tiny", 2, 64)
    hw = W.synthetic(wl)
    hw.keep = True
    knobs = {"TLM_PS_FAIL_LAYER": "1", "TLM_PS_TIMEOUT_US": "2000"}
    saved = {k: os.environ.get(k) for k in knobs}
    os.environ.update(knobs)
    try:
        bad = _runner(hw, ctx, 64, True)
    finally:
        for k, v in saved.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    assert re.search(r"persistent\[\d+ blocks", bad.model.describe())
    l2_before = int(re.search(r"(\d+) publish through their XCD's L2", bad.model.describe()).group(1))
    om = oracle_model(hw, 64, kv_f16=True, threads=16)
    toks = [5, 9, 11]
    for step, t in enumerate(toks):
        t0 = time.perf_counter()
        bad.computeToken(t, step, True)
        close(bad.readLogits(), om.forward(t, step), LOGIT_ATOL, LOGIT_RTOL)
        assert time.perf_counter() - t0 < 5.0  # bounded: a few 2 ms waits in a row
    assert bad.model.counts()["recomputed_positions"] == 3
    # two unread tokens, then a greedy run: all of them recomputed in order
    bad.computeToken(3, 3, False)
    bad.computeToken(4, 4, False)
    om.prefill(3, 3)
    om.prefill(4, 4)
    out = list(bad.decodeGreedy(7, 5, 4))
    t = 7
    for i, d in enumerate(out):
        r = om.forward(t, 5 + i)
        if d != int(np.argmax(r)):
            assert top2_gap(r) < LOGIT_ATOL
            break
        t = d
    assert bad.model.counts()["recomputed_positions"] == 3 + 2 + 4
    assert re.search(r"persistent\[\d+ blocks", bad.model.describe())
    # a time-out also turns the handoffs through an XCD's L2 off (a block may have
    # run on another XCD than its roles were placed for)
    assert l2_before > 0
    assert "; 0 publish through their XCD's L2" in bad.model.describe()
    bad.close()
    om.close()


def _big_mlp_norm(wl, scale):
    """Synthetic weights with layer 0's MLP norm weights set to `scale`."""
    hw = W.synthetic(wl)
    hw.keep = True
    src = hw._source
    hw._source = lambda k, l: np.full(hw.shape(k), scale, np.float32) if (k, l) == (W.FFN_NORM, 0) else src(k, l)
    return hw


def test_fp16_input_overflow_recomputes_on_the_stage_kernels(ctx):
    """Inputs of the persistent q4 linears past the fp16 range: layer 0's
    MLP norm weights of 2^12 put silu(g) * u near 1e8 and the residual near
    1e7, past 65504 (and inside the per-stage kernels' fixed-point range).
    The fp16 copy overflows, its dot products turn NaN, the last layer's rows
    flag the token, and the read recomputes it on the per-stage kernels (fp32
    inputs) and turns the schedule off for the model: every logit equals the
    per-stage model's, within the oracle's tolerance of the oracle."""
    wl = _workload("qwen2.5-0.5b", 4, 64)
    hw = _big_mlp_norm(wl, 2.0 ** 12)
    ps = _runner(hw, ctx, 64, True)
    ref = _runner(hw, ctx, 64, False)
    assert re.search(r"persistent\[\d+ blocks", ps.model.describe())
    om = oracle_model(hw, 64, kv_f16=True, threads=16)
    for i, t in enumerate([int(t) for t in W.prompt_tokens(wl)][:5]):
        ps.computeToken(t, i, True)
        ref.computeToken(t, i, True)
        got = ps.readLogits()
        assert np.array_equal(got, ref.readLogits())
        close(got, om.forward(t, i), LOGIT_ATOL, LOGIT_RTOL)
    assert "persistent[off after an fp16 range overflow]" in ps.model.describe()
    assert ps.model.counts()["recomputed_positions"] == 1
    ps.close()
    ref.close()
    om.close()


def test_two_contexts_decode_at_once_on_one_device(ctx):
    """Two models on two contexts (two streams) of one GPU, each with the
    persistent schedule, which needs every CU at once: their launches are
    ordered per device (each waits for the other's previous one), so greedy
    runs enqueued from two threads at the same time both finish with no
    wait running out (nothing recomputed) and with identical tokens, and
    token-by-token decodes enqueued back to back give identical logits."""
    wl = _workload("qwen2.5-0.5b", 4, 128)
    hw = W.synthetic(wl)
    hw.keep = True
    ctx_b = tlm.Context(0)
    a = _runner(hw, ctx, 128, True)
    b = _runner(hw, ctx_b, 128, True)
    for r in (a, b):
        assert re.search(r"persistent\[\d+ blocks", r.model.describe())
    prompt = [int(t) for t in W.prompt_tokens(wl)][:8]
    for i, t in enumerate(prompt):
        a.computeToken(t, i, True)
        b.computeToken(t, i, True)
    assert np.array_equal(a.readLogits(), b.readLogits())
    out = {}

    def run(name, r):
        out[name] = list(r.decodeGreedy(prompt[-1], len(prompt), 48))

    th = [threading.Thread(target=run, args=(n, r)) for n, r in (("a", a), ("b", b))]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    assert out["a"] == out["b"] and len(out["a"]) == 48
    for r in (a, b):
        assert r.model.counts()["recomputed_positions"] == 0
    a.close()
    b.close()
    ctx_b.close()


def test_a_residual_past_the_fixed_point_range_is_reported(ctx):
    """The per-stage kernels sum the residual stream in 64-bit fixed point
    (x * 2^32, exact while |x| < 2^31).  Layer 0's MLP norm weights of 2^17
    put the residual near 1e10: the kernels flag the values of 2^30 or more,
    the read raises the library's range error instead of returning wrapped
    values, and after a cache reset the flag is gone."""
    wl = _workload("qwen2.5-0.5b", 2, 64)
    hw = _big_mlp_norm(wl, 2.0 ** 17)
    ref = _runner(hw, ctx, 64, False)
    ref.computeToken(5, 0, True)
    with pytest.raises(tlm.TlmError) as err:
        ref.readLogits()
    assert "fixed-point range" in str(err.value)
    ref.resetCache()
    ref.readLogits()  # nothing enqueued since: no flag
    ref.close()
