"""Batch-1 decode benchmark of the per-token path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload qwen2.5-0.5b]

A step is one decode token at batch 1: three kernel launches (the persistent
layer kernel, the LM head, the greedy merge), with the token fed back on the
device.  The default workload is the Qwen2.5-0.5B-shaped decoder (24 layers,
hidden 896, q4 g32 linears, fp16 tied head): a 128-token random prompt, then
K = 256 greedy decode steps timed (positions 127..382), after W untimed
warm-up steps over the same positions.  Weights are synthetic N(0, 0.02).

Prints one JSON line.  Besides tok/s it reports the fraction of the HBM
roofline (algorithmic bytes per token over 8 TB/s), the roofline of the
step's dominant kernel (the layer part: about 90% of the step's time), the
LM head's (57% of the bytes) as an extra field, and a CPU baseline: the
oracle's single-threaded restatement of the reference CPU path timed on a
bounded sample of the same workload.  Prefill: the prompt's 127 positions as
one batched pass (MFMA GEMMs + flash attention; `prefill_tok_s`) and replaying
the decode graph per position as the reference does (`prefill_replay_tok_s`);
`prefill_chunk` is one 2048-position chunk on the Llama-3.2-1B shape with its
FLOP/s against the dense fp16 MFMA peak.  `long_window` is greedy decode on the
Llama-3.2-3B shape over a KV cache pre-filled with N(0, 1) rows to 16384
positions (split-K attention over the long window), with its HBM fraction.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK = 8.0e12  # bytes/s, MI355X HBM3E


def _package():
    import importlib.util
    if "three_llm_amd" in sys.modules:
        return sys.modules["three_llm_amd"]
    pkg_dir = ROOT / "three-llm_amd"
    spec = importlib.util.spec_from_file_location("three_llm_amd", pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["three_llm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bytes_per_token(hw, position: int, kv_first: int = 0) -> float:
    """Algorithmic HBM bytes to compute the token at `position` (reads the
    cache rows [kv_first, position]): weights once, one embedding row, norms,
    biases, the KV read and the KV write.  Activations are excluded."""
    r = hw.recipe
    H, I, V, L = r.hidden_size, r.inner_size, r.vocab_size, r.layer_count
    nqkv = r.q_size + 2 * r.kv_size
    bpw = {"q4": 0.5 + 2.0 / 32, "f16": 2.0, "f32": 4.0}
    lin = L * bpw[hw.storage.linear] * (nqkv * H + H * r.q_size + 2 * I * H + H * I)
    head = V * H * (2.0 if r.tied_embeddings else bpw[hw.storage.head])
    emb = H * (4 if hw.storage.embed == "f32" else 2)
    norms = (2 * L + 1) * H * 4 + (L * nqkv * 4 if r.qkv_bias else 0)
    esz = 4 if hw.storage.kv == "f32" else 2
    kv_row = L * 2 * r.kv_head_count * r.head_dim * esz
    return lin + head + emb + norms + (position + 1 - kv_first) * kv_row + kv_row


def layer_bytes(hw, position: int) -> float:
    """Algorithmic bytes of the layer part of the token at `position` (the
    persistent kernel): every layer's weights, norms and biases, the embedding
    row, the KV rows [0, position] read and the row at position written; the
    per-token bytes without the LM head and the final norm."""
    r = hw.recipe
    head = r.vocab_size * r.hidden_size * (2.0 if r.tied_embeddings else
                                           {"q4": 0.5 + 2.0 / 32, "f16": 2.0, "f32": 4.0}[hw.storage.head])
    return bytes_per_token(hw, position, 0) - head - r.hidden_size * 4


def lm_head_bytes(hw, cus: int) -> float:
    """Algorithmic bytes of one LM head launch: fp16 head rows, the normed
    hidden vector, the logits and the per-block argmax partials (one per
    block: ceil(T / per) blocks of per = ceil(T / (2 cus)) 64-row tiles)."""
    r = hw.recipe
    tiles = (r.vocab_size + 63) // 64
    per = max(-(-tiles // (2 * cus)), -(-tiles // 4096))
    blocks = -(-tiles // per)
    return r.vocab_size * r.hidden_size * 2.0 + r.hidden_size * 4 + r.vocab_size * 4 + blocks * 8


def read_traffic(kernel: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters, from the
    committed profile summary (None if that summary does not exist yet)."""
    p = ROOT / "profiles" / f"{kernel}_traffic.txt"
    if not p.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or 'unknown'."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(hw, prompt, budget_s: float):
    """The oracle (C restatement of the reference CPU path: fp32 storage,
    double accumulation, one thread) over positions 0, 1, ... of the same
    prompt until the time budget is spent."""
    sys.path.insert(0, str(ROOT))
    sys.path.insert(0, str(ROOT / "tests"))
    from bridge import oracle_model  # the checker, used here only as the baseline

    om = oracle_model(hw, max(len(prompt), 64), kv_f16=False, threads=1)
    t0 = time.perf_counter()
    n = 0
    while n < len(prompt) and (time.perf_counter() - t0) < budget_s:
        om.forward(int(prompt[n]), n)
        n += 1
    dt = time.perf_counter() - t0
    om.close()
    return n / dt, n, dt


MFMA_PEAK_F16 = 2.5e15  # dense fp16 MFMA FLOP/s, MI355X


def prefill_flops(r, n: int, p0: int = 0) -> float:
    """Useful FLOPs of one prefill chunk of n positions starting at p0: the
    linears (2 M N K each) and causal attention (QK^T and PV over the keys
    [0, pos] of each position); masked-out products are not counted."""
    H, I, L = r.hidden_size, r.inner_size, r.layer_count
    nqkv = r.q_size + 2 * r.kv_size
    lin = 2.0 * n * L * (H * nqkv + r.q_size * H + 2 * I * H + I * H)
    keys = sum(p + 1 for p in range(p0, p0 + n)) if not r.sliding_window else sum(
        min(p + 1, r.sliding_window) for p in range(p0, p0 + n))
    att = 4.0 * r.head_dim * r.head_count * keys * L
    return lin + att


def prefill_chunk_bench(W, R, ctx, workload: str, n: int) -> dict:
    """One prefill chunk of n random ids on a full-size model (the MFMA GEMM
    path): median of 9 timed chunks after one warm-up, FLOP/s and the
    fraction of the dense fp16 MFMA peak."""
    wl = W.WORKLOADS[workload]
    hw = W.synthetic(wl)
    hw.keep = True
    runner = R.DecoderHIPRunner(hw, {"maxTokens": n + 8, "prefillChunkSize": n}, ctx=ctx)
    ids = [int(t) for t in W.prompt_tokens(W.Workload(wl.name, wl.config, wl.storage, n, 0, n))]
    times = []
    for rep in range(10):
        runner.resetCache()
        ctx.sync()
        t0 = time.perf_counter()
        runner.prefillTokens(ids, 0, n)
        ctx.sync()
        if rep:
            times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    flops = prefill_flops(hw.recipe, n)
    out = {"workload": wl.name, "tokens": n, "batched": runner.batchedPrefill, "ms": round(dt * 1e3, 3),
           "tok_s": round(n / dt, 1), "tflops": round(flops / dt / 1e12, 1),
           "mfma_frac": round(flops / dt / MFMA_PEAK_F16, 4), "flops_per_chunk": flops,
           "peak": "2.5 PFLOP/s dense fp16 MFMA"}
    log(f"[bench] prefill chunk {wl.name} x {n}: {dt * 1e3:.2f} ms = {n / dt:.0f} tok/s, "
        f"{flops / dt / 1e12:.0f} TFLOP/s = {100 * flops / dt / MFMA_PEAK_F16:.1f}% of the fp16 MFMA peak")
    runner.close()
    return out


def long_window_bench(W, R, ctx, steps: int, warmup: int = 4) -> dict:
    """Greedy decode on the Llama-3.2-3B shape from position 16384, the fp16
    KV cache rows [0, 16384) pre-filled with N(0, 1) values: `steps` device-fed
    steps timed after `warmup` over the same positions; tok/s and the HBM
    fraction of the algorithmic bytes (weights, head, the KV rows read)."""
    wl = W.WORKLOADS["llama-3.2-3b"]
    hw = W.synthetic(wl)
    pos0 = wl.kv_prefill
    runner = R.DecoderHIPRunner(hw, {"maxTokens": pos0 + max(steps, warmup) + 1}, ctx=ctx)
    runner.model.kv_fill_normal(0xC0FFEE, pos0)
    last = int(W.prompt_tokens(wl)[-1])
    runner.decodeGreedy(last, pos0, warmup)
    ctx.sync()
    t0 = time.perf_counter()
    runner.decodeGreedy(last, pos0, steps)
    ctx.sync()
    wall = time.perf_counter() - t0
    mean_bytes = sum(bytes_per_token(hw, pos0 + i, 0) for i in range(steps)) / steps
    out = {"workload": wl.name, "kv_positions": pos0, "steps": steps, "tok_s": round(steps / wall, 1),
           "ms_per_step": round(wall * 1e3 / steps, 4), "bytes_per_token": round(mean_bytes),
           "hbm_roofline_frac": round(mean_bytes * steps / wall / HBM_PEAK, 4)}
    log(f"[bench] long window {wl.name} from position {pos0}: {steps / wall:.1f} tok/s "
        f"({wall * 1e6 / steps:.0f} us/token), {mean_bytes / 1e6:.1f} MB/token -> "
        f"{100 * out['hbm_roofline_frac']:.1f}% of HBM roofline")
    runner.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", default="qwen2.5-0.5b")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work (0 disables)")
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--prefill-workload", default="llama-3.2-1b",
                    help="model of the prefill-chunk measurement (the MFMA GEMM path)")
    ap.add_argument("--prefill-chunk", type=int, default=2048,
                    help="positions of the prefill-chunk measurement (0 skips it)")
    ap.add_argument("--long-window-steps", type=int, default=32,
                    help="decode steps of the long-window measurement (0 skips it)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill-chunk measurement (for profiling); prints its JSON object")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device-to-device copy of this many MiB, 5 times (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings), then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the multi-GPU (tensor-parallel) decode path is a design "
              "only, so --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    pkg = _package()
    W, R, tlm = pkg.weights, pkg.runner, pkg.tlm
    if args.copy_mib:
        ctx = tlm.Context(0)
        n = args.copy_mib << 20
        src, dst = ctx.buffer(n), ctx.buffer(n)
        for _ in range(5):
            dst.copy_from(src)
        ctx.sync()
        log(f"[bench] copied {args.copy_mib} MiB device-to-device 5 times")
        src.free()
        dst.free()
        ctx.close()
        return
    if args.prefill_only:
        ctx = tlm.Context(0)
        out = prefill_chunk_bench(W, R, ctx, args.prefill_workload, args.prefill_chunk or 2048)
        ctx.close()
        print(json.dumps(out), flush=True)
        return
    wl = W.WORKLOADS[args.workload]
    t0 = time.perf_counter()
    hw = W.synthetic(wl)
    hw.keep = True
    ctx = tlm.Context(0)
    dev_name, cus = ctx.info()
    max_tokens = max(wl.max_tokens, wl.kv_prefill + wl.prompt_len + args.steps + 1)
    runner = R.DecoderHIPRunner(hw, {"maxTokens": max_tokens}, ctx=ctx)
    log(f"[bench] {wl.name} on {dev_name}: weights ready in {time.perf_counter() - t0:.1f}s")
    log(f"[bench] layout: {runner.model.describe()}")
    prompt = [int(t) for t in W.prompt_tokens(wl)]
    start = wl.kv_prefill
    if wl.kv_prefill:
        runner.model.kv_fill_normal(0xC0FFEE, wl.kv_prefill)
    # prompt prefill: positions [start, start + n) without logits, batched
    # (MFMA GEMMs + flash attention) and, for comparison, the reference's
    # semantics (the decode graph replayed once per position)
    prefill_n = len(prompt) - 1
    prefill_s = replay_s = None
    if prefill_n > 0:
        toks_all = [0] * start + prompt
        runner.prefillTokens(toks_all, start, start + prefill_n)  # warm-up (row buffers, code objects)
        m = runner.model
        m.set_prefill(0, runner.prefillChunkSize)
        m.reset_cache()
        if wl.kv_prefill:
            m.kv_fill_normal(0xC0FFEE, wl.kv_prefill)
        ctx.sync()
        tp = time.perf_counter()
        runner.prefillTokens(toks_all, start, start + prefill_n)
        ctx.sync()
        replay_s = time.perf_counter() - tp
        if runner.batchedPrefill:
            m.set_prefill(runner.prefillBatchRows, runner.prefillChunkSize)
        times = []
        for _ in range(11):  # the median of 11 passes: the first ones after model set-up run slower
            m.reset_cache()
            if wl.kv_prefill:
                m.kv_fill_normal(0xC0FFEE, wl.kv_prefill)
            ctx.sync()
            tp = time.perf_counter()
            runner.prefillTokens(toks_all, start, start + prefill_n)
            ctx.sync()
            times.append(time.perf_counter() - tp)
        prefill_s = sorted(times)[len(times) // 2]
    last, pos0 = prompt[-1], start + prefill_n
    steps, warmup = args.steps, args.warmup
    if pos0 + max(steps, warmup) > max_tokens:
        raise SystemExit("bench.py: steps exceed the context")
    # warm-up over the same positions, then the timed region
    if warmup:
        runner.decodeGreedy(last, pos0, warmup)
    ctx.sync()
    t1 = time.perf_counter()
    tokens = runner.decodeGreedy(last, pos0, steps)  # K device-fed steps, one sync at the end
    ctx.sync()
    wall = time.perf_counter() - t1
    ev_ms = runner.model.time_decode(last, pos0, 0, steps)
    toks = steps / wall
    ms_step = wall * 1e3 / steps
    mean_bytes = sum(bytes_per_token(hw, pos0 + i, 0) for i in range(steps)) / steps
    hbm_frac = mean_bytes * toks / HBM_PEAK
    # the dominant kernel of the step: the layer part (the persistent kernel,
    # one launch per token; the layer graph where the window is long), timed
    # inside decode steps over the same positions (a pair of HIP events on the
    # model stream around each launch); then the LM head the same way
    n_k = min(steps, args.kernel_iters)
    # which schedule ran: the library counts the token steps it ran on the
    # persistent kernel (windows of at most 1024 positions; longer windows take
    # the per-stage layer graph)
    before = runner.model.counts()["persistent_tokens"]
    lay_ms = runner.model.time_layers(last, pos0, n_k)
    persistent = runner.model.counts()["persistent_tokens"] - before == n_k
    lay_bytes = sum(layer_bytes(hw, pos0 + i) for i in range(n_k)) / n_k
    lay_bw = lay_bytes / (lay_ms * 1e-3)
    lm_ms = runner.model.time_head(last, pos0, n_k)
    lm_bytes = lm_head_bytes(hw, ctx.info()[1])
    lm_bw = lm_bytes / (lm_ms * 1e-3)
    # host-driven loop (computeToken + sampleToken per token: one 4-byte
    # device-to-host read and one stream sync per token over PCIe)
    n_host = min(steps, 64)
    tok = last
    ctx.sync()
    th = time.perf_counter()
    for i in range(n_host):
        runner.computeToken(int(tok), pos0 + i, True)
        tok = runner.sampleToken(1, {"temperature": 0})
    host_tok_s = n_host / (time.perf_counter() - th)
    # the same loop sampling top-8 (temperature 0.8): device candidates, host draw
    import random as _random
    rnd = _random.Random(7)
    ctx.sync()
    th = time.perf_counter()
    for i in range(n_host):
        runner.computeToken(int(tok), pos0 + i, True)
        tok = runner.sampleToken(8, {"temperature": 0.8, "random": rnd.random})
    host_topk_tok_s = n_host / (time.perf_counter() - th)
    stage_ms = {name: runner.model.time_kernel(k, args.kernel_iters)
                for name, k in (("qkv", 4), ("attention", 1), ("o", 5), ("mlp", 2), ("top8", 6))}
    log(f"[bench] decode {toks:.1f} tok/s ({ms_step * 1e3:.1f} us/token wall, {ev_ms * 1e3 / steps:.1f} us/token "
        f"events), {mean_bytes / 1e6:.2f} MB/token -> {hbm_frac * 100:.1f}% of HBM roofline")
    log(f"[bench] layer part ({'persistent kernel' if persistent else 'layer graph'}) {lay_ms * 1e3:.1f} us/token "
        f"= {lay_bw / 1e9:.0f} GB/s of {lay_bytes / 1e6:.2f} MB")
    log(f"[bench] LM head {lm_ms * 1e3:.1f} us/launch in decode steps = {lm_bw / 1e9:.0f} GB/s; stage times, "
        f"back-to-back launches of layer 0 (us): "
        + ", ".join(f"{k} {v * 1e3:.1f}" for k, v in stage_ms.items()))
    log(f"[bench] host-driven loop (token read back every step): {host_tok_s:.1f} tok/s greedy, "
        f"{host_topk_tok_s:.1f} tok/s sampling top-8 candidates")
    if prefill_n > 0:
        log(f"[bench] prefill {prefill_n} tokens: {prefill_s * 1e3:.2f} ms batched "
            f"({'MFMA row batches' if runner.batchedPrefill else 'replay'}), {replay_s * 1e3:.2f} ms replaying the "
            f"decode graph; first tokens {[int(t) for t in tokens[:8]]}")
    cpu = None
    if args.cpu_budget > 0:
        ncpu = os.cpu_count()
        rate, n, dt = cpu_baseline(hw, prompt if len(prompt) > 1 else list(W.prompt_tokens(
            W.Workload("s", wl.config, wl.storage, 64, 0, 64))), args.cpu_budget)
        cpu = {"value": round(rate, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "cpu": cpu_model(), "host_threads": ncpu,
               "sample": f"oracle forward of the first {n} prompt positions of the same workload "
                         f"({dt:.1f} s, fp32 weights, double accumulation, 1 of {ncpu} host threads)"}
        log(f"[bench] cpu baseline {rate:.3f} tok/s over {n} tokens")
    result = {
        "metric": "decode tok/s @bs=1 and % of HBM roofline; prefill tok/s (Qwen2.5-0.5B shape)",
        "value": round(toks, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # arithmetic: fp32 activations and accumulation over q4 g32 weights
        # (fp16 scales), an fp16 LM head and an fp16 KV cache
        "dtype": "f32 math; q4 g32 linears, f16 head, f16 kv" if wl.storage.kv == "f16" else
                 f"f32 math; {wl.storage.linear} linears, {wl.storage.kv} kv",
        "data": "synthetic",
        "hbm_roofline_frac": round(hbm_frac, 4),
        "bytes_per_token": round(mean_bytes),
        "prefill_tok_s": round(prefill_n / prefill_s, 1) if prefill_n > 0 else None,
        "prefill_replay_tok_s": round(prefill_n / replay_s, 1) if prefill_n > 0 else None,
        "host_loop_tok_s": round(host_tok_s, 1),
        "host_loop_top8_tok_s": round(host_topk_tok_s, 1),
        "top8_candidates_us": round(stage_ms["top8"] * 1e3, 2),
        "config": {"workload": wl.name, "prompt": wl.prompt_len, "decode": steps, "batch": 1,
                   "linears": wl.storage.linear + (" g32 fp16 scales" if wl.storage.linear == "q4" else ""),
                   "head": "fp16 tied" if hw.recipe.tied_embeddings else wl.storage.head, "kv": wl.storage.kv,
                   "kv_prefill": wl.kv_prefill, "device": dev_name, "cus": cus},
        "roofline": {"bound": "hbm", "kernel": "ps_token_kernel" if persistent else "layer graph (per-stage kernels)",
                     "achieved": round(lay_bw / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(lay_bw / HBM_PEAK, 4),
                     "traffic": read_traffic("ps_token") if persistent else None,
                     "avg_launch_us": round(lay_ms * 1e3, 2), "algorithmic_bytes": round(lay_bytes),
                     "step_share": round(lay_ms / ms_step, 3)},
        "lm_head": {"bound": "hbm", "kernel": "lm_head_kernel", "achieved": round(lm_bw / 1e9, 1),
                    "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(lm_bw / HBM_PEAK, 4),
                    "traffic": read_traffic("lm_head"), "avg_launch_us": round(lm_ms * 1e3, 2),
                    "algorithmic_bytes": round(lm_bytes), "step_share": round(lm_ms / ms_step, 3)},
        "cpu_baseline": cpu,
    }
    runner.close()
    if args.prefill_chunk:
        result["prefill_chunk"] = prefill_chunk_bench(W, R, ctx, args.prefill_workload, args.prefill_chunk)
    if args.long_window_steps:
        result["long_window"] = long_window_bench(W, R, ctx, args.long_window_steps)
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
