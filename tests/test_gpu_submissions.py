"""Launch counts of the decode and prefill paths: the reference's submission
contract (src/test/submission.browser.test.ts:46-57: one submission per
decode token; 3 for an 18-token prefill in chunks of 7).

Here a decode token on the per-stage schedule is one launch of its captured
graph, preceded (when the host supplies the token) by one small kernel that
writes the token and the position: the counterpart of the reference's uniform
upload before its submit (DecoderTSLRunner.ts:487-501), which is not a
submission.  On the persistent schedule a decode token is its two kernels (the
layers; the LM head, whose last block does the greedy merge), enqueued
directly: a graph launch of the same kernels costs more per token.  A prompt chunk is
one graph launch too, after one such write naming the chunk: a batched chunk
(enough rows) is its captured sequence of row kernels, a shorter chunk the
decode graph's token steps captured back to back, as the reference encodes
a chunk's replays into one submission (:472-480,504-530).
"""
import numpy as np
import pytest

import three_llm_amd.runner as R
import three_llm_amd.tlm as tlm
import three_llm_amd.weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = tlm.Context(0)
    yield c
    c.close()


def _delta(model, before):
    now = model.counts()
    return {k: now[k] - before[k] for k in now}


def test_reference_fixture_one_graph_per_token(ctx, hf_fixture):
    case = hf_fixture["cases"][0]
    tensors = {k: np.asarray(v["values"], np.float32).reshape(v["shape"]) for k, v in hf_fixture["tensors"].items()}
    hw = W.from_hf(case["config"], tensors, W.Storage(linear="f16", head="f16", embed="f32", kv="f32"))
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 64, "prefillChunkSize": 7}, ctx=ctx)
    assert not runner.batchedPrefill  # head_dim 8: the fixture replays the decode graph
    m = runner.model
    assert m.counts() == {"graph_launches": 0, "kernel_launches": 0, "prefill_chunks": 0, "replayed_positions": 0,
                            "recomputed_positions": 0, "persistent_tokens": 0}
    runner.computeToken(1, 0, True)
    b = m.counts()
    runner.computeToken(5, 1, True)
    assert _delta(m, b) == {"graph_launches": 1, "kernel_launches": 1, "prefill_chunks": 0, "replayed_positions": 0,
                            "recomputed_positions": 0, "persistent_tokens": 0}
    runner.resetCache()
    b = m.counts()
    ids = hf_fixture["input_ids"]
    runner.prefillTokens(ids, 0, 18)  # chunks of 7, 7 and 4: one graph each
    assert _delta(m, b) == {"graph_launches": 3, "kernel_launches": 3, "prefill_chunks": 0,
                            "replayed_positions": 18, "recomputed_positions": 0, "persistent_tokens": 0}
    b = m.counts()
    out = runner.decodeGreedy(ids[18], 18, 4)  # the device feeds its own tokens: one write in all
    assert len(out) == 4
    assert _delta(m, b) == {"graph_launches": 4, "kernel_launches": 1, "prefill_chunks": 0, "replayed_positions": 0,
                            "recomputed_positions": 0, "persistent_tokens": 0}
    b = m.counts()
    runner.readLogits()
    runner.readCandidates(3)
    assert _delta(m, b)["graph_launches"] == 0
    runner.close()


def test_batched_prefill_one_pass_per_chunk(ctx):
    wl = W.WORKLOADS["tiny"]
    # intermediate 768: the batched GEMMs need multiples of 32 (the tiny config has 688)
    wl = W.Workload(wl.name + "-768", dict(wl.config, intermediate_size=768), wl.storage, 18, 8, 64)
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": 64, "prefillChunkSize": 7, "prefillBatchRows": 1}, ctx=ctx)
    assert runner.batchedPrefill
    m = runner.model
    toks = [int(t) for t in W.prompt_tokens(wl)][:18]
    b = m.counts()
    runner.prefillTokens(toks, 0, 18)
    d = _delta(m, b)
    # per chunk: the write naming it, then its captured row kernels (embedding
    # rows, per layer 7 or 8 row kernels and GEMMs, the last fold): one graph
    assert d == {"graph_launches": 3, "kernel_launches": 3, "prefill_chunks": 3, "replayed_positions": 0,
                 "recomputed_positions": 0, "persistent_tokens": 0}
    b = m.counts()
    runner.computeToken(toks[-1], 18, True)
    ps = int("persistent[off]" not in m.describe())  # the decode step's schedule
    assert _delta(m, b) == {"graph_launches": 1 - ps, "kernel_launches": 1 + 2 * ps, "prefill_chunks": 0,
                            "replayed_positions": 0, "recomputed_positions": 0, "persistent_tokens": ps}
    runner.close()


def test_long_replayed_chunk_splits_into_bounded_graphs(ctx, monkeypatch):
    """A replayed chunk whose token steps would record more kernels than one
    replay graph holds (2048) runs as several graphs: the tiny decoder on the
    per-stage schedule, 600 positions in one chunk -> more than one graph
    launch and fewer than one per position, with the cache rows and the next
    logits bit-identical to chunks of 7 (the same kernels either way)."""
    monkeypatch.setenv("TLM_PERSISTENT", "0")  # read at model creation
    wl = W.WORKLOADS["tiny"]
    wl = W.Workload(wl.name, wl.config, wl.storage, 601, 8, 640)
    hw = W.synthetic(wl)
    hw.keep = True
    toks = [int(t) for t in W.prompt_tokens(wl)]
    big = R.DecoderHIPRunner(hw, {"maxTokens": 640, "prefillChunkSize": 600, "prefillBatchRows": 0}, ctx=ctx)
    small = R.DecoderHIPRunner(hw, {"maxTokens": 640, "prefillChunkSize": 7, "prefillBatchRows": 0}, ctx=ctx)
    assert "persistent[off]" in big.model.describe()
    b = big.model.counts()
    big.prefillTokens(toks, 0, 600)
    d = _delta(big.model, b)
    assert d["replayed_positions"] == 600
    assert 1 < d["graph_launches"] < 600, d
    small.prefillTokens(toks, 0, 600)
    for l in range(wl.config["num_hidden_layers"]):
        for x, y in zip(big.model.kv_read(l, 0, 600), small.model.kv_read(l, 0, 600)):
            assert np.array_equal(x, y)
    big.computeToken(toks[600], 600, True)
    small.computeToken(toks[600], 600, True)
    assert np.array_equal(big.readLogits(), small.readLogits())
    big.close()
    small.close()
