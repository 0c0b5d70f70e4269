"""Builds the CPU oracle from the same canonical bytes the device receives.

Test infrastructure: only tests/, smoke() and bench.py's cpu_baseline use it."""
import numpy as np

from oracle import oracle as orc
import three_llm_amd.weights as W

_ORC_ID = {W.EMBED: orc.EMBED, W.LM_HEAD: orc.LM_HEAD, W.FINAL_NORM: orc.FINAL_NORM, W.ATTN_NORM: orc.ATTN_NORM,
           W.FFN_NORM: orc.FFN_NORM, W.WQKV: orc.WQKV, W.BQKV: orc.BQKV, W.WO: orc.WO, W.WGATE: orc.WGATE,
           W.WUP: orc.WUP, W.WDOWN: orc.WDOWN}


def device_values(hw, kind, layer=0):
    """fp32 values of what the device holds for a tensor (q4 dequantized by the
    oracle's restatement, fp16 widened exactly)."""
    data, scales = hw.tensor(kind, layer)
    fmt = hw.fmt(kind)
    if fmt == "q4":
        return orc.q4_dequant(data, scales)
    if fmt == "f16":
        return data.view(np.float16).astype(np.float32)
    return np.asarray(data, np.float32)


def oracle_model(hw, max_tokens, kv_f16=True, threads=1):
    r = hw.recipe
    inv, af = r.rope()
    orc.set_threads(threads)
    m = orc.Model(r.hidden_size, r.inner_size, r.layer_count, r.head_count, r.kv_head_count, r.head_dim,
                  r.vocab_size, max_tokens, r.norm_eps, inv, af, rotary_dim=r.rotary_dim,
                  sliding_window=r.sliding_window, kv_f16=kv_f16, attn_scale=r.attn_scale,
                  layer_windows=r.layer_windows if r.layer_types is not None else None)
    for kind, layer in hw.kinds():
        m.set(_ORC_ID[kind], layer, device_values(hw, kind, layer))
    if r.tied_embeddings:
        m.set(orc.LM_HEAD, 0, device_values(hw, W.EMBED, 0))
    return m


def close(actual, expected, atol, rtol):
    """max over elements of |a - e| - (atol + rtol |e|) must be <= 0."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape
    assert np.all(np.isfinite(a)), "non-finite output"
    excess = (np.abs(a - e) - (atol + rtol * np.abs(e))).reshape(-1)
    i = int(np.argmax(excess)) if excess.size else 0
    assert excess.size == 0 or excess[i] <= 0, f"element {i}: {a.flat[i]} vs {e.flat[i]} (excess {excess[i]:.3g})"


def top2_gap(logits):
    part = np.partition(np.asarray(logits, np.float64), -2)
    return float(part[-1] - part[-2])
