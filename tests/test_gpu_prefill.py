"""Batched prefill on the GPU: the MFMA GEMM, the MFMA flash attention and the
whole-model pass, against the CPU oracle and against the replayed decode graph
(the reference's prefill, DecoderTSLRunner.ts:472-480, 504-530).

Precision contract of the batched path: activations enter the GEMMs and the
attention as fp16, q4 weights are dequantised to fp16 ((code - 8) * s rounded
once), products accumulate in fp32.  The GEMM is therefore checked tightly
against a float64 product of the same fp16 operands; model-level results use
the north-star tolerance (logits max-abs 2e-2 / rel 1e-2, greedy stream equal
except under a top-2 gap below it).
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


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def f16_bits(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16).view(np.uint16))


def make_linear(ctx, fmt, w):
    if fmt == tlm.FMT_Q4:
        packed, scales = orc.q4_quantize(w)
        return tlm.Linear(ctx, fmt, packed, scales), orc.q4_dequant(packed, scales)
    bits = f16_bits(w)
    return tlm.Linear(ctx, fmt, bits), bits.view(np.float16).astype(np.float32)


# ------------------------------------------------------------------- GEMM --

@pytest.mark.parametrize("fmt,M,N,K", [
    (tlm.FMT_Q4, 1, 1152, 896), (tlm.FMT_Q4, 37, 1152, 896), (tlm.FMT_Q4, 64, 896, 896),
    (tlm.FMT_Q4, 127, 1152, 896), (tlm.FMT_Q4, 200, 896, 4864), (tlm.FMT_Q4, 65, 200, 96),
    (tlm.FMT_Q4, 300, 2048, 2048), (tlm.FMT_Q4, 33, 64, 32),
    (tlm.FMT_Q4, 300, 44032, 64),  # 172 x 3 blocks of 256 columns, ragged last block
    (tlm.FMT_Q4, 1100, 4096, 128),  # 9 x 16 blocks of 128 rows x 256 columns, the last 76 rows
    (tlm.FMT_Q4, 127, 9664, 896),   # 151 x 4 K-wave blocks (more than the CUs), an odd tile count
    (tlm.FMT_F16, 70, 256, 64), (tlm.FMT_F16, 5, 37, 32), (tlm.FMT_F16, 130, 512, 256)])
def test_linear_rows_matches_fp16_operand_product(ctx, fmt, M, N, K):
    """Each row equals bias + W x with x and W rounded to fp16 (the device's
    operands) and an fp32-accumulated sum: checked against float64."""
    rng = np.random.default_rng(M * 31 + N + K)
    w = f32(rng.standard_normal((N, K)) * 0.02)
    x = f32(rng.standard_normal((M, K)))
    b = f32(rng.standard_normal(N) * 0.1)
    L, wd = make_linear(ctx, fmt, w)
    xb = f16_bits(x)
    y = L.rows(ctx.array(xb), M, ctx.buffer(4 * M * N), ctx.array(b)).read().reshape(M, N)
    xh = xb.view(np.float16).astype(np.float64)
    wh = wd.astype(np.float16).astype(np.float64)  # (code - 8) * s rounded once to fp16
    ref = xh @ wh.T + b
    mag = np.abs(xh) @ np.abs(wh).T + np.abs(b)
    err = np.abs(y - ref) - (2e-6 * mag + 1e-7)
    assert err.max() <= 0, f"max excess {err.max()}"
    # and within fp16-operand rounding of the oracle's fp32 linear
    ref32 = np.stack([orc.linear_t(x[i], wd, b) for i in range(min(M, 4))])
    close(y[:len(ref32)], ref32, 2e-3, 2e-3)
    L.close()


def test_linear_rows_rejects_unsupported(ctx):
    rng = np.random.default_rng(3)
    L, _ = make_linear(ctx, tlm.FMT_F16, f32(rng.standard_normal((8, 24))))  # K % 32 != 0
    with pytest.raises(tlm.TlmError):
        L.rows(ctx.array(f16_bits(np.zeros((2, 24)))), 2, ctx.buffer(64))
    L.close()
    w = f32(rng.standard_normal((64, 32)))
    w[0, 0] = 60000.0  # scale 60000 / 7 > 8188: (code - 8) * s would overflow fp16
    L, _ = make_linear(ctx, tlm.FMT_Q4, w)
    with pytest.raises(tlm.TlmError):
        L.rows(ctx.array(f16_bits(np.zeros((2, 32)))), 2, ctx.buffer(4 * 2 * 64))
    L.close()


# -------------------------------------------------------------- attention --

@pytest.mark.parametrize("heads,kv,D,theta,before,rows,window,rd", [
    (14, 2, 64, 1e6, 0, 127, 0, 64),      # Qwen2.5-0.5B heads, one prompt chunk
    (32, 8, 64, 5e5, 0, 300, 0, 64),      # Llama-3.2-1B heads
    (24, 8, 128, 5e5, 0, 100, 0, 128),    # Llama-3.2-3B heads (head_dim 128)
    (14, 2, 64, 1e6, 45, 90, 0, 64),      # continuation after 45 decoded positions
    (4, 2, 64, 1e4, 20, 200, 50, 64),     # sliding window
    (8, 1, 128, 1e4, 3, 1, 0, 128),       # one row
    (8, 2, 64, 1e4, 10, 71, 0, 32),       # partial rotary: dims 32..63 pass through
])
def test_attention_rows_match_oracle(ctx, heads, kv, D, theta, before, rows, window, rd):
    """Positions [before, before + rows) as one batched call after `before`
    decode-op positions; every row against the oracle's attention with the same
    fp16 cache rounding, and the cache rows it appended."""
    rng = np.random.default_rng(heads * D + rows)
    inv, af = orc.rope_parameters(rd, theta)
    T = before + rows + 8
    A = tlm.Attention(ctx, heads, kv, D, T, inv, rotary_dim=rd, attention_factor=af, sliding_window=window,
                      kv_fmt=tlm.FMT_F16)
    kc = np.zeros((T, kv * D), np.float32)
    vc = np.zeros_like(kc)
    width = (heads + 2 * kv) * D
    out1 = ctx.buffer(4 * heads * D)
    for pos in range(before):
        qkv = f32(rng.standard_normal(width))
        A(ctx.array(qkv), pos, out1)
        orc.attention(qkv, heads, kv, D, pos, kc, vc, inv, rotary_dim=rd, attention_factor=af,
                      sliding_window=window, kv_f16=True)
    qkv = f32(rng.standard_normal((rows, width)))
    got = A.rows(ctx.array(qkv), rows, before, ctx.buffer(2 * rows * heads * D)).read(np.uint16)
    got = got.view(np.float16).astype(np.float32).reshape(rows, heads * D)
    ref = np.stack([orc.attention(qkv[i], heads, kv, D, before + i, kc, vc, inv, rotary_dim=rd, attention_factor=af,
                                  sliding_window=window, kv_f16=True) for i in range(rows)])
    # fp16 q, probabilities and output on top of the cache rounding
    close(got, ref, 4e-3, 4e-3)
    k, v = A.read_cache(before + rows)
    close(v, vc[:before + rows], 0, 0)
    close(k, kc[:before + rows], 1e-3, 1e-3)
    print(f"max |attn rows - oracle| = {np.abs(got - ref).max():.3g}")
    A.close()


# ------------------------------------------------------------------ model --

def _workload(name, layers, prompt_len, max_tokens=512):
    wl = W.WORKLOADS[name]
    cfg = dict(wl.config, num_hidden_layers=layers)
    return W.Workload(wl.name + f"-{layers}l", cfg, wl.storage, prompt_len, 6, max_tokens, qkv_bias=wl.qkv_bias)


def _kv(model, layers, count):
    return [tuple(a.view(np.float16).astype(np.float32) for a in model.kv_read(l, 0, count)) for l in range(layers)]


@pytest.mark.parametrize("name,layers,prompt_len,chunk", [
    ("qwen2.5-0.5b", 2, 128, 2048),   # the benchmark prompt: one batched chunk of 127 rows
    ("qwen2.5-0.5b", 2, 151, 64),     # chunks 64 + 64 batched, 22 replayed
    ("qwen2.5-0.5b", 2, 701, 2048),   # 700 rows: 22 row tiles of the K-wave kernels, RoPE epilogue
    ("llama-3.2-1b", 2, 200, 2048),
    ("llama-3.2-1b", 2, 100, 2048),   # 99 rows: K-wave O and gate|up GEMMs, the O GEMM's fold over 32 tiles
    ("llama-3.2-3b", 2, 100, 2048),   # head_dim 128
])
def test_batched_prefill_matches_replay_and_oracle(ctx, name, layers, prompt_len, chunk):
    wl = _workload(name, layers, prompt_len, max_tokens=max(512, prompt_len + 16))
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens, "prefillChunkSize": chunk}, ctx=ctx)
    assert runner.batchedPrefill
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    n = len(prompt) - 1
    m = runner.model
    # replayed decode graph (the reference's semantics)
    m.set_prefill(0, chunk)
    m.prefill(prompt, 0, n)
    m.compute_token(prompt[-1], n, True)
    replay_logits = m.read_logits()
    replay_kv = _kv(m, layers, n)
    # batched
    m.reset_cache()
    m.set_prefill(64, chunk)
    runner.prefillTokens(prompt, 0, n)
    runner.computeToken(prompt[-1], n, True)
    logits = runner.readLogits()
    kv = _kv(m, layers, n)
    for l in range(layers):
        for got, ref in zip(kv[l], replay_kv[l]):
            close(got, ref, 2e-2, 1e-2)
    close(logits, replay_logits, LOGIT_ATOL, LOGIT_RTOL)
    # against the oracle: logits after the prompt and the greedy stream
    om = oracle_model(hw, wl.max_tokens, kv_f16=True, threads=16)
    for i, t in enumerate(prompt[:-1]):
        om.prefill(t, i)
    ref = om.forward(prompt[-1], n)
    close(logits, ref, LOGIT_ATOL, LOGIT_RTOL)
    first = runner.sampleToken(1, {"temperature": 0})
    stream = [first] + list(runner.decodeGreedy(first, n + 1, 3))
    tok, pos = int(np.argmax(ref)), n + 1
    for step, got in enumerate(stream):
        if got != tok:
            assert top2_gap(ref) < LOGIT_ATOL, f"stream diverged at step {step}"
            break
        if step == len(stream) - 1:
            break
        ref = om.forward(tok, pos)
        tok, pos = int(np.argmax(ref)), pos + 1
    print(name, "stream", stream, "max |logits - replay|", float(np.abs(logits - replay_logits).max()))
    om.close()
    runner.close()


def test_batched_prefill_2048_rows_matches_replay(ctx):
    """One chunk of 2048 positions through two Llama-3.2-1B layers: the
    large-batch shapes of the q4 GEMM (16 row tiles of 128 x 8..64 column
    blocks of 256, split K for the partial sums) and 64 query tiles of the
    flash attention.  Checked against the replayed decode graph, an
    independent path (the oracle would need ~250 GMAC on the host here)."""
    layers, n = 2, 2048
    wl = _workload("llama-3.2-1b", layers, n + 1, max_tokens=n + 8)
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": wl.max_tokens, "prefillChunkSize": 2048}, ctx=ctx)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, wl.config["vocab_size"], n + 1)]
    m = runner.model
    m.set_prefill(0, 2048)
    m.prefill(prompt, 0, n)
    m.compute_token(prompt[-1], n, True)
    replay_logits = m.read_logits()
    replay_kv = _kv(m, layers, n)
    m.reset_cache()
    m.set_prefill(64, 2048)
    runner.prefillTokens(prompt, 0, n)
    runner.computeToken(prompt[-1], n, True)
    logits = runner.readLogits()
    kv = _kv(m, layers, n)
    for l in range(layers):
        for got, ref in zip(kv[l], replay_kv[l]):
            close(got, ref, 2e-2, 1e-2)
    close(logits, replay_logits, LOGIT_ATOL, LOGIT_RTOL)
    print("max |logits - replay|", float(np.abs(logits - replay_logits).max()))
    runner.close()


@pytest.mark.parametrize("name,layers,prompt_len", [
    ("qwen2.5-0.5b", 24, 128),   # 127 rows: the K-wave GEMMs (each wave streams its K range through an LDS ring)
    ("llama-3.2-1b", 16, 301),   # 300 rows
])
def test_batched_prefill_is_repeatable(ctx, name, layers, prompt_len):
    """The same chunk prefilled five times on one model gives bit-identical
    cache rows in every layer.  (A refill of a GEMM's LDS ring stage that did
    not wait for the wave's last reads of that stage once made rows of random
    layers differ between runs.)"""
    wl = _workload(name, layers, prompt_len)
    hw = W.synthetic(wl)
    runner = R.DecoderHIPRunner(hw, {"maxTokens": prompt_len + 8}, ctx=ctx)
    assert runner.batchedPrefill
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    n = len(prompt) - 1
    first = None
    for rep in range(5):
        runner.resetCache()
        runner.prefillTokens(prompt, 0, n)
        rows = [np.concatenate([a.reshape(n, -1) for a in runner.model.kv_read(l, 0, n)], axis=1)
                for l in range(layers)]
        if first is None:
            first = rows
            continue
        for l in range(layers):
            diff = np.where((rows[l] != first[l]).reshape(n, -1).any(axis=1))[0]
            assert len(diff) == 0, f"run {rep}: layer {l} rows {diff[:8]} differ from run 0"
    runner.close()


def test_fp16_overflow_in_a_batched_chunk_replays_it_on_the_decode_path(ctx):
    """Layer 0's gate and up weights scaled to N(0, 10): the SwiGLU output of
    the batched chunk passes 65504, the row kernels' overflow flag trips and
    tlm_prefill replays the chunk on the fp32 decode graph, so the cache rows
    and the next logits equal the pure replay's bit for bit and stay finite.
    Unscaled weights never trip it."""
    wl = _workload("qwen2.5-0.5b", 2, 100)
    hw = W.synthetic(wl)
    src = hw._source
    hw._source = lambda kind, layer: src(kind, layer) * (500.0 if kind in (W.WGATE, W.WUP) and layer == 0 else 1.0)
    hw.keep = True
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    n = len(prompt) - 1
    runs = []
    for min_rows in (64, 0):  # batched (falls back), then the reference's replay only
        runner = R.DecoderHIPRunner(hw, {"maxTokens": n + 8}, ctx=ctx)
        m = runner.model
        m.set_prefill(min_rows, 2048)
        runner.prefillTokens(prompt, 0, n)
        runner.computeToken(prompt[-1], n, True)
        logits = runner.readLogits()
        kv = [np.concatenate([a.reshape(n, -1) for a in m.kv_read(l, 0, n)], axis=1) for l in range(2)]
        runs.append((logits, kv, m.describe()))
        runner.close()
    (lb, kvb, db), (lr, kvr, dr) = runs
    assert "1 replayed after fp16 overflow" in db, db
    assert "0 replayed after fp16 overflow" in dr
    assert np.isfinite(lb).all()
    assert np.array_equal(lb, lr)
    for a, b in zip(kvb, kvr):
        assert np.array_equal(a, b)
    # the same model with unscaled weights: the batched chunk stands
    plain = W.synthetic(wl)
    runner = R.DecoderHIPRunner(plain, {"maxTokens": n + 8}, ctx=ctx)
    runner.prefillTokens(prompt, 0, n)
    assert "0 replayed after fp16 overflow" in runner.model.describe()
    runner.close()
