"""tlm_op_attention_rows_noalloc (the allocation-free variant of the batched
attention; its query staging is the library's fixed device array) against
tlm_op_attention_rows on the same inputs: the same kernels, so the outputs
and the appended cache rows are bit-identical.  Two calls in a row, the
second with fewer rows, so that the second reads only what it wrote into the
shared array; the free device memory is the same before and after each
call (nothing allocated, nothing left behind); then a call beyond the
array's size is refused."""
import numpy as np
import pytest

from oracle import oracle as orc
import three_llm_amd.tlm as tlm

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = tlm.Context(0)
    yield c
    c.close()


def f32(x):
    return np.ascontiguousarray(x, np.float32)


@pytest.mark.parametrize("heads,kv,D,theta,calls", [
    (32, 8, 64, 5e5, [(0, 600), (600, 37)]),     # Llama-3.2-1B heads: 600 rows, then 37 more
    (24, 8, 128, 5e5, [(0, 300), (300, 5)]),     # Llama-3.2-3B heads (head_dim 128)
    (14, 2, 64, 1e6, [(10, 127), (137, 1)]),     # Qwen2.5-0.5B heads after 10 cached positions
])
def test_noalloc_rows_equal_allocating_rows(ctx, heads, kv, D, theta, calls):
    print(f"[no-alloc] heads {heads}/{kv} x {D}, calls {calls}", flush=True)
    inv, af = orc.rope_parameters(D, theta)
    T = 1024
    rng = np.random.default_rng(heads + D)
    width = (heads + 2 * kv) * D
    ref = tlm.Attention(ctx, heads, kv, D, T, inv, attention_factor=af, kv_fmt=tlm.FMT_F16)
    nal = tlm.Attention(ctx, heads, kv, D, T, inv, attention_factor=af, kv_fmt=tlm.FMT_F16)
    p0 = calls[0][0]
    if p0:  # the same cached positions in both, through the one-position op
        out1 = ctx.buffer(4 * heads * D)
        for pos in range(p0):
            q = ctx.array(f32(rng.standard_normal(width)))
            ref(q, pos, out1)
            nal(q, pos, out1)
    for pos0, rows in calls:
        qkv = ctx.array(f32(rng.standard_normal((rows, width))))
        a = ref.rows(qkv, rows, pos0, ctx.buffer(2 * rows * heads * D)).read(np.uint16)
        out = ctx.buffer(2 * rows * heads * D)
        ctx.sync()
        free0 = ctx.memory()[0]
        nal.rows_noalloc(qkv, rows, pos0, out)
        ctx.sync()
        assert ctx.memory()[0] == free0, "the allocation-free entry point changed the free device memory"
        b = out.read(np.uint16)
        assert np.array_equal(a, b), f"rows {rows} at {pos0}: {int((a != b).sum())} fp16 outputs differ"
        ka, va = ref.read_cache(pos0 + rows)
        kb, vb = nal.read_cache(pos0 + rows)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # beyond the 4 MiB staging array: refused before any launch
    too_many = (4 << 20) // (2 * heads * D) + 1
    big = tlm.Attention(ctx, heads, kv, D, too_many + 8, inv, attention_factor=af, kv_fmt=tlm.FMT_F16)
    qkv = ctx.buffer(4 * too_many * width)
    with pytest.raises(tlm.TlmError) as err:
        big.rows_noalloc(qkv, too_many, 0, ctx.buffer(2 * too_many * heads * D))
    assert err.value.code == tlm.TLM_ERR_RANGE and "query staging" in str(err.value)
    # the largest size that fits still runs and matches
    fit = too_many - 1
    x = ctx.array(f32(rng.standard_normal((fit, width))))
    b = big.rows_noalloc(x, fit, 0, ctx.buffer(2 * fit * heads * D)).read(np.uint16)
    big.reset()
    a = big.rows(x, fit, 0, ctx.buffer(2 * fit * heads * D)).read(np.uint16)
    assert np.array_equal(a, b)
    for A in (ref, nal, big):
        A.close()
