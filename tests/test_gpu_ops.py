"""Op-level parity of the HIP kernels against the CPU oracle, through the C ABI.

Cases follow the reference's own op tests (src/test/tsl.browser.test.ts) plus
the shapes of the benchmark configurations.  Tolerances are written per test;
integer/byte work (dequant, token ids) is compared bit for bit.
"""
import math

import numpy as np
import pytest

from bridge import close
from oracle import oracle as orc
import three_llm_amd.tlm as tlm

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = tlm.Context(0)
    name, cus = c.info()
    print(f"device: {name}, {cus} CUs", flush=True)
    yield c
    c.close()


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def fill_sin(n, seed):
    """fillSin, src/test/helpers.ts:13-16."""
    return f32(np.sin(seed + np.arange(n) * 0.17) * 0.35)


def make_linear(ctx, fmt, w):
    if fmt == tlm.FMT_Q4:
        packed, scales = orc.q4_quantize(w)
        return tlm.Linear(ctx, fmt, packed, scales), orc.q4_dequant(packed, scales)
    bits = f32(w).astype(np.float16).view(np.uint16)
    return tlm.Linear(ctx, fmt, bits), bits.view(np.float16).astype(np.float32)


# ------------------------------------------------------------------ linear --

def test_linear_closed_forms(ctx):
    # tsl.browser.test.ts:58-80; the reference's W [in][out] = [3,4,5,6] is [[3,5],[4,6]] as [out][in]
    L, _ = make_linear(ctx, tlm.FMT_F16, np.float32([[3, 5], [4, 6]]))
    x, y, b = ctx.array(f32([1, 2])), ctx.buffer(8), ctx.array(f32([7, 8]))
    assert np.array_equal(L(x, y, b).read(), [20, 24])
    assert np.array_equal(L(x, y).read(), [13, 16])
    L2, _ = make_linear(ctx, tlm.FMT_F16, np.float32([[1, 3, 5], [2, 4, 6]]))
    assert np.array_equal(L2(ctx.array(f32([1, -1, 0.5])), ctx.buffer(8)).read(), [0.5, 1])
    L.close()
    L2.close()


@pytest.mark.parametrize("fmt,N,K", [(tlm.FMT_Q4, 1152, 896), (tlm.FMT_Q4, 896, 4864), (tlm.FMT_Q4, 100, 96),
                                     (tlm.FMT_Q4, 64, 32), (tlm.FMT_F16, 37, 23), (tlm.FMT_F16, 2048, 896)])
def test_dequant_is_bit_exact(ctx, fmt, N, K):
    rng = np.random.default_rng(N * 7 + K)
    w = f32(rng.standard_normal((N, K)) * 0.02)
    L, ref = make_linear(ctx, fmt, w)
    got = L.dequant()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    L.close()


@pytest.mark.parametrize("fmt,N,K", [(tlm.FMT_Q4, 1152, 896), (tlm.FMT_Q4, 896, 896), (tlm.FMT_Q4, 9728, 896),
                                     (tlm.FMT_Q4, 896, 4864), (tlm.FMT_Q4, 2048, 8192), (tlm.FMT_Q4, 100, 96),
                                     (tlm.FMT_F16, 512, 256), (tlm.FMT_F16, 256, 688), (tlm.FMT_F16, 37, 23)])
def test_linear_matches_oracle(ctx, fmt, N, K):
    rng = np.random.default_rng(N + K)
    w = f32(rng.standard_normal((N, K)) * 0.02)
    x = f32(rng.standard_normal(K))
    b = f32(rng.standard_normal(N) * 0.1)
    L, wd = make_linear(ctx, fmt, w)
    y = L(ctx.array(x), ctx.buffer(4 * N), ctx.array(b)).read()
    ref = orc.linear_t(x, wd, b)
    mag = orc.linear_t(np.abs(x), np.abs(wd)) + np.abs(b)
    # fp32 accumulation (q4 path: 8*sum(x) offset) against the oracle's double sum
    err = np.abs(y.astype(np.float64) - ref) - (4e-5 * mag + 1e-7)
    assert err.max() <= 0, f"max excess {err.max()}"
    L.close()


# ------------------------------------------------------------ element ops --

def test_rmsnorm_matches_oracle(ctx):
    for n, offset in ((3, False), (896, False), (4096, True), (1, False)):
        x = f32(np.sin(np.arange(n) * 0.37) * 3 + 0.5)
        w = f32(1 + 0.1 * np.cos(np.arange(n)))
        y = tlm.rmsnorm(ctx, ctx.array(x), ctx.array(w), n, 1e-6, offset, ctx.buffer(4 * n)).read()
        close(y, orc.rmsnorm(x, w, 1e-6, offset), 1e-6, 2e-6)


def test_silu_mul_and_gated_mlp(ctx):
    # tsl.browser.test.ts:275-294 (reference weights [in][out] = 2x3 / 3x2)
    x = f32([1, -0.5])
    g_ref, u_ref, d_ref = f32([0.5, -0.25, 1, 0.75, 0.5, -1]), f32([1, 0, 0, 1, 0.5, -0.5]), f32([1, 0, 0, 0.25, -0.5,
                                                                                                  0.5])
    gate = orc.linear(x, g_ref, None, 2, 3)
    up = orc.linear(x, u_ref, None, 2, 3)
    hidden = f32([orc.silu(float(gate[i])) * float(up[i]) for i in range(3)])
    expected = orc.linear(hidden, d_ref, None, 3, 2)
    h = tlm.silu_mul(ctx, ctx.array(gate), ctx.array(up), 3, ctx.buffer(12)).read()
    close(h, hidden, 1e-7, 1e-6)
    gu = np.concatenate([g_ref.reshape(2, 3).T, u_ref.reshape(2, 3).T])  # [2I][H] rows gate then up
    GU, _ = make_linear(ctx, tlm.FMT_F16, gu)
    DN, _ = make_linear(ctx, tlm.FMT_F16, d_ref.reshape(3, 2).T)
    y = tlm.gated_mlp(GU, DN, ctx.array(x), ctx.buffer(8)).read()
    close(y, expected, 1e-6, 1e-5)  # tsl.browser.test.ts:291 uses 1e-4


@pytest.mark.parametrize("fmt,H,I", [(tlm.FMT_Q4, 896, 4864), (tlm.FMT_F16, 256, 688)])
def test_gated_mlp_matches_oracle(ctx, fmt, H, I):
    rng = np.random.default_rng(H)
    g = f32(rng.standard_normal((I, H)) * 0.02)
    u = f32(rng.standard_normal((I, H)) * 0.02)
    d = f32(rng.standard_normal((H, I)) * 0.02)
    x = f32(rng.standard_normal(H))
    GU, gud = make_linear(ctx, fmt, np.concatenate([g, u]))
    DN, dd = make_linear(ctx, fmt, d)
    y = tlm.gated_mlp(GU, DN, ctx.array(x), ctx.buffer(4 * H)).read()
    gate = orc.linear_t(x, gud[:I])
    up = orc.linear_t(x, gud[I:])
    act = f32([orc.silu(float(a)) * float(b) for a, b in zip(gate, up)])
    ref = orc.linear_t(act, dd)
    close(y, ref, 2e-5, 2e-4)


# --------------------------------------------------------------- attention --

ATTN_CASES = [  # tsl.browser.test.ts:318-380 (QK-norm is outside the Llama/Qwen2 recipe)
    dict(name="gqa_no_rope", heads=4, kv=2, D=2, max_tokens=4, seqs=[(16, 0.3), (16, 1.1)]),
    dict(name="rope_mha", heads=2, kv=2, D=2, max_tokens=8, theta=10000, seqs=[(12, 0.2), (12, 0.8), (12, 1.4)]),
    dict(name="gqa_rope", heads=4, kv=2, D=2, max_tokens=4, theta=10000, rd=2, seqs=[(16, 0.5), (16, 1.5)]),
    dict(name="partial_rope_scale", heads=2, kv=2, D=4, max_tokens=4, theta=10000, rd=2, scale=0.25,
         seqs=[(24, 0.6), (24, 1.6)]),
    dict(name="sliding_gqa", heads=4, kv=2, D=2, max_tokens=8, window=2, seqs=[(16, 0.4), (16, 1.4), (16, 2.4)]),
]


@pytest.mark.parametrize("case", ATTN_CASES, ids=[c["name"] for c in ATTN_CASES])
def test_attention_reference_cases(ctx, case):
    heads, kv, D = case["heads"], case["kv"], case["D"]
    rd = case.get("rd", D) if case.get("theta") else 0
    inv = orc.rope_parameters(rd, case["theta"])[0] if rd else np.zeros(1, np.float32)
    A = tlm.Attention(ctx, heads, kv, D, case["max_tokens"], inv if rd else None, rotary_dim=rd,
                      sliding_window=case.get("window", 0), kv_fmt=tlm.FMT_F32, attn_scale=case.get("scale", 0.0))
    kc = np.zeros((case["max_tokens"], kv * D), np.float32)
    vc = np.zeros_like(kc)
    out = ctx.buffer(4 * heads * D)
    for pos, (n, seed) in enumerate(case["seqs"]):
        qkv = fill_sin(n, seed)
        got = A(ctx.array(qkv), pos, out).read()
        ref = orc.attention(qkv, heads, kv, D, pos, kc, vc, inv, rotary_dim=rd, sliding_window=case.get("window", 0),
                            attn_scale=case.get("scale", 0.0))
        close(got, ref, 1e-6, 1e-5)
    k, v = A.read_cache(len(case["seqs"]))
    close(k, kc[:len(case["seqs"])], 1e-7, 1e-6)
    close(v, vc[:len(case["seqs"])], 0, 0)
    A.close()


@pytest.mark.parametrize("kv_fmt", [tlm.FMT_F16, tlm.FMT_F32], ids=["f16", "f32"])
def test_attention_window_of_one_returns_the_current_value_row(ctx, kv_fmt):
    """A sliding window of 1 leaves only the current position: the softmax over
    one score is 1, so every query head's output is its kv head's new V row
    (rounded like the cache), whatever q and the cached past hold."""
    heads, kv, D, T = 4, 2, 64, 48
    inv = orc.rope_parameters(D, 1e4)[0]
    A = tlm.Attention(ctx, heads, kv, D, T, inv, sliding_window=1, kv_fmt=kv_fmt)
    out = ctx.buffer(4 * heads * D)
    rng = np.random.default_rng(11)
    for pos in range(T):
        qkv = rng.standard_normal((heads + 2 * kv) * D).astype(np.float32)
        got = A(ctx.array(qkv), pos, out).read().reshape(heads, D)
        v = qkv[(heads + kv) * D:].reshape(kv, D)
        if kv_fmt == tlm.FMT_F16:
            v = v.astype(np.float16).astype(np.float32)
        want = np.repeat(v, heads // kv, axis=0)
        close(got, want, 1e-7, 1e-6)
    A.close()


@pytest.mark.parametrize("heads,kv,D,theta,steps,window,kv_fmt", [
    (14, 2, 64, 1e6, 700, 0, tlm.FMT_F16), (24, 8, 128, 5e5, 300, 0, tlm.FMT_F16),
    (32, 8, 64, 5e5, 1100, 0, tlm.FMT_F16), (4, 2, 64, 1e4, 300, 100, tlm.FMT_F16),
    (24, 8, 128, 5e5, 300, 0, tlm.FMT_F32), (4, 2, 128, 5e5, 1100, 0, tlm.FMT_F32),
    # long windows of the grouped kernel: 7 query heads per kv head (8-head
    # variant), one (multi-head attention), and head_dim 128 with a window
    (14, 2, 64, 1e6, 1100, 0, tlm.FMT_F16), (8, 8, 128, 5e5, 1100, 0, tlm.FMT_F16),
    (6, 2, 128, 1e4, 1300, 1100, tlm.FMT_F16),
    # the matrix-core kernel's edges: 16 query heads on one kv head (every
    # padded head column used), (G + 2) head_dim = 1536 exactly (three q|k|v
    # elements per thread), and one group past that (the per-head kernel)
    (16, 1, 64, 1e4, 1060, 0, tlm.FMT_F16), (20, 2, 128, 5e5, 1060, 0, tlm.FMT_F16),
    (22, 2, 128, 5e5, 1040, 0, tlm.FMT_F16)])
def test_attention_long_fp16_cache(ctx, heads, kv, D, theta, steps, window, kv_fmt):
    """fp16 (and fp32) cache, split-K over many chunks: every output against
    the oracle run with the same cache rounding.  The 1100-step cases cross the
    1024-position window where the long-window kernels take over."""
    rng = np.random.default_rng(heads * D)
    inv, af = orc.rope_parameters(D, theta)
    M = steps + 8
    A = tlm.Attention(ctx, heads, kv, D, M, inv, attention_factor=af, sliding_window=window, kv_fmt=kv_fmt)
    kc = np.zeros((M, kv * D), np.float32)
    vc = np.zeros_like(kc)
    out = ctx.buffer(4 * heads * D)
    worst = 0.0
    for pos in range(steps):
        qkv = f32(rng.standard_normal((heads + 2 * kv) * D))
        got = A(ctx.array(qkv), pos, out).read()
        ref = orc.attention(qkv, heads, kv, D, pos, kc, vc, inv, attention_factor=af, sliding_window=window,
                            kv_f16=kv_fmt == tlm.FMT_F16)
        # K/V are rounded to fp16 from RoPE values computed in fp32 (device) or
        # double (oracle); an occasional 1-ulp fp16 difference bounds this.
        close(got, ref, 2e-3, 2e-3)
        worst = max(worst, float(np.abs(got - ref).max()))
    k, v = A.read_cache(steps)
    close(v, vc[:steps], 0, 0)
    close(k, kc[:steps], 1e-3, 1e-3)
    print(f"max |attn - oracle| = {worst:.3g}")
    A.close()


def test_attention_long_window_partial_rotary(ctx):
    """Partial rotary (32 of 64 dims rotated) past the 1024-position window,
    where the matrix-core kernel rotates q and the new k in its prologue and
    passes the other 32 dims through: every output against the oracle with the
    same fp16 cache rounding, and the appended rows read back."""
    heads, kv, D, rd, steps = 8, 2, 64, 32, 1060
    rng = np.random.default_rng(3207)
    inv, af = orc.rope_parameters(rd, 1e4)
    M = steps + 8
    A = tlm.Attention(ctx, heads, kv, D, M, inv, rotary_dim=rd, attention_factor=af, kv_fmt=tlm.FMT_F16)
    kc = np.zeros((M, kv * D), np.float32)
    vc = np.zeros_like(kc)
    out = ctx.buffer(4 * heads * D)
    for pos in range(steps):
        qkv = f32(rng.standard_normal((heads + 2 * kv) * D))
        got = A(ctx.array(qkv), pos, out).read()
        ref = orc.attention(qkv, heads, kv, D, pos, kc, vc, inv, rotary_dim=rd, attention_factor=af, kv_f16=True)
        if pos >= 1024 or pos % 128 == 0:
            close(got, ref, 2e-3, 2e-3)
    k, v = A.read_cache(steps)
    close(v, vc[:steps], 0, 0)
    close(k, kc[:steps], 1e-3, 1e-3)
    A.close()


def test_attention_decode_after_16384_positions(ctx):
    """The Llama-3.2-3B decode case (24/8 heads, head_dim 128, theta 5e5, fp16
    cache) at its real window: positions 0..16383 are appended by the batched
    rows path (8 calls), the cache is read back, and three decode steps at
    16384.. are checked against the oracle over that same cache.  At this
    window the matrix-core kernel takes one block per kv head and chunk (32
    chunks of ~513 positions, 8 waves each) for the group's 3 query heads, and
    the combine folds 32 partials per head."""
    heads, kv, D, theta, n0 = 24, 8, 128, 5e5, 16384
    rng = np.random.default_rng(16384)
    inv, af = orc.rope_parameters(D, theta)
    M = n0 + 8
    A = tlm.Attention(ctx, heads, kv, D, M, inv, attention_factor=af, kv_fmt=tlm.FMT_F16)
    width = (heads + 2 * kv) * D
    rows_out = ctx.buffer(2 * 2048 * heads * D)
    for p0 in range(0, n0, 2048):
        A.rows(ctx.array(f32(rng.standard_normal((2048, width)))), 2048, p0, rows_out)
    k, v = A.read_cache(n0)
    kc = np.zeros((M, kv * D), np.float32)
    vc = np.zeros_like(kc)
    kc[:n0], vc[:n0] = k, v
    out = ctx.buffer(4 * heads * D)
    worst = 0.0
    for pos in range(n0, n0 + 3):
        qkv = f32(rng.standard_normal(width))
        qkv[:heads * D] *= 6.0  # peaked softmax: a few positions carry each head, so a lost chunk shows
        got = A(ctx.array(qkv), pos, out).read()
        ref = orc.attention(qkv, heads, kv, D, pos, kc, vc, inv, attention_factor=af, kv_f16=True)
        assert np.abs(ref).max() > 0.5
        close(got, ref, 2e-3, 2e-3)
        worst = max(worst, float(np.abs(got - ref).max() / np.abs(ref).max()))
    k2, v2 = A.read_cache(n0 + 3)
    close(v2, vc[:n0 + 3], 0, 0)
    close(k2[n0:], kc[n0:n0 + 3], 1e-3, 1e-3)
    assert worst < 1e-4, worst
    print(f"max |attn - oracle| / max |oracle| over 16384+ positions = {worst:.3g}")
    A.close()


def test_device_copy_is_exact(ctx):
    """tlm_copy: byte-exact device-to-device copy; sizes not a multiple of 16 are rejected."""
    rng = np.random.default_rng(7)
    a = rng.integers(0, 256, size=(1 << 20) + 48, dtype=np.uint8)
    src, dst = ctx.buffer(a.nbytes), ctx.buffer(a.nbytes)
    src.write(a)
    dst.copy_from(src)
    assert np.array_equal(dst.read(np.uint8), a)
    with pytest.raises(tlm.TlmError):
        dst.copy_from(src, 8)
    src.free()
    dst.free()


# ------------------------------------------------------------------ logits --

def test_argmax_known_answers(ctx):
    tok = ctx.buffer(4)
    for logits, expected in (([1, 7, 7, -2, 8, 3, 6], 4), ([1, 7, 7, -2], 1), ([-np.inf, -np.inf], 0),
                             ([np.nan, 2, 2], 1), ([5], 0)):
        lg = f32(logits)
        assert tlm.argmax(ctx, ctx.array(lg), len(lg), tok).read(np.int32)[0] == expected
    rng = np.random.default_rng(2)
    big = f32(rng.standard_normal(151936))
    big[[777, 150000, 90000]] = 9.0  # planted tie: the lowest id wins
    assert tlm.argmax(ctx, ctx.array(big), len(big), tok).read(np.int32)[0] == 777


def test_topk_known_answers(ctx):
    # tsl.browser.test.ts:82-120
    lg = f32([1, 7, 7, -2, 8, 3, 6])
    assert tlm.topk(ctx, ctx.array(lg), 7, 3) == [(4, 8.0), (1, 7.0), (2, 7.0)]
    assert tlm.topk(ctx, ctx.array(lg), 7, 1) == [(4, 8.0)]
    c = tlm.topk(ctx, ctx.array(f32([10, 2, -1])), 3, 2, softcap=1.0)
    assert c[0][0] == 0 and c[0][1] <= 1 and c[1][0] == 1
    lowest = float(np.float32(-3.4028234663852886e38))
    assert tlm.topk(ctx, ctx.array(f32([np.nan, -np.inf, 2.0])), 3, 3) == [(2, 2.0), (0, lowest), (0, lowest)]


@pytest.mark.parametrize("n,k", [(151936, 8), (128256, 16), (4096, 1), (300000, 16), (2049, 5), (10, 16)])
def test_topk_matches_oracle(ctx, n, k):
    """GPU candidates (one or two block levels) equal the oracle's restatement
    of the reference's chunked candidate levels, ids and scores exactly, with
    ties, -inf, NaN and LOWEST_FLOAT planted; softcap scores within 2 ulp."""
    rng = np.random.default_rng(n + k)
    x = f32(np.round(rng.standard_normal(n) * 4, 1))  # rounded: many ties
    hot = rng.integers(0, n, size=min(n, 40))
    x[hot] = 9.5  # a tie at the top across the whole vector
    x[rng.integers(0, n, size=max(1, n // 1000))] = np.nan
    x[rng.integers(0, n, size=max(1, n // 1000))] = -np.inf
    buf = ctx.array(x)
    got = tlm.topk(ctx, buf, n, k)
    ref = orc.topk_candidates(x, k)
    assert got == ref
    got = tlm.topk(ctx, buf, n, k, softcap=30.0)
    ref = orc.topk_candidates(x, k, softcap=30.0)
    assert [t for t, _ in got] == [t for t, _ in ref]
    close([v for _, v in got], [v for _, v in ref], 0, 2.5e-7)


@pytest.mark.parametrize("V,H", [(151936, 896), (4096, 256), (1000, 64), (7, 8)])
def test_logits_head_matches_oracle(ctx, V, H):
    rng = np.random.default_rng(V)
    w = f32(rng.standard_normal((V, H)) * 0.02)
    x = f32(rng.standard_normal(H))
    L, wd = make_linear(ctx, tlm.FMT_F16, w)
    out = ctx.buffer(4 * V)
    tok = ctx.buffer(4)
    tlm.logits(L, ctx.array(x), out, tok)
    got = out.read()
    ref = orc.linear_t(x, wd)
    mag = orc.linear_t(np.abs(x), np.abs(wd))
    assert (np.abs(got - ref) - (2e-5 * mag + 1e-7)).max() <= 0
    t = int(tok.read(np.int32)[0])
    # the fused argmax is exact on the device logits
    assert t == int(np.argmax(got))
    L.close()
