"""Writes tests/golden/node_runner.json: what the oracle computes for the
synthetic decoders the Node.js runner builds (node/runner.js,
DecoderHIPRunner.synthetic), the expectations node/test_runner_gpu.js checks
that runner against on the GPU.

Per workload (the tiny decoder, and the 24-layer Qwen2.5-0.5B shape): the
prompt ids, the oracle's logits after the prompt (all of them for the tiny
decoder; the 32 largest for Qwen's 151936), and the oracle's greedy stream
with each step's top-2 logit gap (the contract allows a different token only
after a step whose gap is under the logit tolerance).

CPU only:  python tests/golden/make_node_golden.py
"""
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "tests"))
import conftest  # noqa: E402,F401  (imports three-llm_amd as three_llm_amd)
from bridge import oracle_model, top2_gap  # noqa: E402
import three_llm_amd.weights as W  # noqa: E402

CASES = [("tiny", 16, 16, "all"), ("qwen2.5-0.5b", 16, 8, 32)]


def case(name, prompt_len, steps, keep):
    wl = W.WORKLOADS[name]
    wl = W.Workload(wl.name, wl.config, wl.storage, prompt_len, steps, 64, qkv_bias=wl.qkv_bias)
    hw = W.synthetic(wl)
    om = oracle_model(hw, 64, kv_f16=True, threads=8)
    prompt = [int(t) for t in W.prompt_tokens(wl)][:prompt_len]
    for i, t in enumerate(prompt[:-1]):
        om.prefill(t, i)
    logits = om.forward(prompt[-1], prompt_len - 1)
    if keep == "all":
        kept = {"ids": list(range(len(logits))), "values": [float(v) for v in logits]}
    else:
        top = np.argsort(-logits.astype(np.float64), kind="stable")[:keep]
        kept = {"ids": [int(i) for i in top], "values": [float(logits[i]) for i in top]}
    stream, gaps = [], []
    cur = logits
    for s in range(steps):
        tok = int(np.argmax(cur))
        stream.append(tok)
        gaps.append(top2_gap(cur))
        if s + 1 < steps:
            cur = om.forward(tok, prompt_len + s)
    om.close()
    return {"workload": name, "prompt": prompt, "logits": kept, "stream": stream, "gaps": gaps}


def main():
    out = {"tolerance": {"atol": 2e-2, "rtol": 1e-2},
           "cases": [case(*c) for c in CASES]}
    path = ROOT / "tests" / "golden" / "node_runner.json"
    path.write_text(json.dumps(out, separators=(",", ":")))
    print("wrote", path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
