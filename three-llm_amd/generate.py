"""The caller of the per-token path: the reference's generation loop and host
sampling, restated (runtime/generate.ts and the sampling half of
runtime/math.ts, paths relative to packages/three-llm/src/).

Everything here runs on the host and drives a runner through the controls
interface GenerateAsyncControls (generate.ts:31-49): computeToken,
prefillTokens, readLogits, sampleToken, resetCache, rewindable and
maxGpuCandidateCount.
"""
from __future__ import annotations

import math
import random as _random
from dataclasses import dataclass
from typing import Callable, List, Optional

import numpy as np


# ------------------------------------------------------------- sampling --

def apply_repeat_penalties(logits: np.ndarray, tokens: Optional[List[int]], repetitionPenalty=1.0,
                           presencePenalty=0.0, frequencyPenalty=0.0, repeatLastN=64, noRepeatNgramSize=0):
    """applyRepeatPenalties, math.ts:438-503."""
    if not tokens:
        return logits
    use_rep = repetitionPenalty != 1 and repetitionPenalty > 0
    use_pres = presencePenalty != 0
    use_freq = frequencyPenalty != 0
    ngram = max(0, int(math.floor(noRepeatNgramSize)))
    use_ngrams = ngram >= 2 and len(tokens) >= ngram - 1
    if not (use_rep or use_pres or use_freq or use_ngrams):
        return logits
    out = np.array(logits, np.float32, copy=True)
    if use_rep or use_pres or use_freq:
        start = max(0, len(tokens) - repeatLastN) if repeatLastN > 0 else 0
        counts = {}
        for t in tokens[start:]:
            counts[t] = counts.get(t, 0) + 1
        for t, count in counts.items():
            score = float(out[t])
            if use_rep:
                score = score * repetitionPenalty if score < 0 else score / repetitionPenalty
            if use_pres:
                score -= presencePenalty
            if use_freq:
                score -= frequencyPenalty * count
            out[t] = score
    if use_ngrams:
        prefix_len = ngram - 1
        prefix_start = len(tokens) - prefix_len
        for i in range(0, len(tokens) - ngram + 1):
            if all(tokens[i + j] == tokens[prefix_start + j] for j in range(prefix_len)):
                out[tokens[i + prefix_len]] = -np.inf
    return out


def needs_full_logits(options: dict) -> bool:
    """needsFullLogitsForSampling, math.ts:509-523."""
    return (options.get("forceFullLogits") is True
            or (options.get("repetitionPenalty", 1) != 1 and options.get("repetitionPenalty", 1) > 0)
            or options.get("presencePenalty", 0) != 0 or options.get("frequencyPenalty", 0) != 0
            or max(0, int(math.floor(options.get("noRepeatNgramSize", 0)))) >= 2)


def _softmax32(values: np.ndarray) -> np.ndarray:
    """softmax, math.ts:60-76 (double exponentials, fp32 storage)."""
    m = max(float(v) for v in values)
    ex = [math.exp(float(v) - m) for v in values]
    s = sum(ex)
    return np.array([float(np.float32(e)) / s for e in ex], np.float32)


def sample_top_k_candidates(candidates, temperature=0.8, random: Callable[[], float] = _random.random) -> int:
    """sampleTopKCandidates, math.ts:527-547."""
    if not candidates:
        return 0
    if temperature <= 0 or len(candidates) == 1:
        return candidates[0][0]
    values = np.array([c[1] / max(temperature, 1e-6) for c in candidates], np.float32)
    probs = _softmax32(values)
    r = random()
    for i, p in enumerate(probs):
        r -= float(p)
        if r <= 0:
            return candidates[i][0]
    return candidates[-1][0]


def sample_top_k(logits: np.ndarray, temperature=0.8, topK=40, random: Callable[[], float] = _random.random,
                 tokens=None, **penalties) -> int:
    """sampleTopK, math.ts:556-620 (greedy branch :581-593: first maximum wins)."""
    logits = apply_repeat_penalties(logits, tokens, **penalties)
    k = min(max(1, int(math.floor(topK))), len(logits))
    if temperature <= 0 or k == 1:
        best, best_v = 0, logits[0]
        for i in range(1, len(logits)):
            if logits[i] > best_v:
                best, best_v = i, logits[i]
        return best
    scaled = np.asarray(logits, np.float64) / max(temperature, 1e-6)
    # the reference keeps a sorted list of the k best (ties keep the earlier id)
    order = np.argsort(-scaled, kind="stable")[:k]
    candidates = [(int(i), float(scaled[i])) for i in order]
    values = np.array([c[1] for c in candidates], np.float32)
    probs = _softmax32(values)
    r = random()
    for i, p in enumerate(probs):
        r -= float(p)
        if r <= 0:
            return candidates[i][0]
    return candidates[-1][0]


_PENALTY_KEYS = ("repetitionPenalty", "presencePenalty", "frequencyPenalty", "repeatLastN", "noRepeatNgramSize")


def _sample_options(options: dict):
    return {k: options[k] for k in _PENALTY_KEYS if k in options}


# ---------------------------------------------------------------- planning --

def shared_prefix_length(a, b) -> int:
    """sharedPrefixLength, generate.ts:61-68."""
    a = a or []
    b = b or []
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


def prepare_generation_from_tokens(tokens, max_tokens, max_new_tokens, end_of_text_token_id):
    """prepareGenerationFromTokens, generate.ts:70-81."""
    budget = max(1, max_tokens - 1)
    input_tokens = [end_of_text_token_id] if len(tokens) == 0 else list(tokens)[-budget:]
    new_budget = max(0, min(max_new_tokens, max_tokens - len(input_tokens)))
    return input_tokens, new_budget


@dataclass
class PromptCachePlan:
    start: int
    logits: Optional[np.ndarray]
    reset: bool
    reused: int


def plan_prompt_cache(cached_tokens, cached_logits, input_tokens, rewindable) -> PromptCachePlan:
    """planPromptCache, generate.ts:98-118."""
    prefix = shared_prefix_length(cached_tokens, input_tokens)
    has_logits = cached_logits is not None
    if prefix > 0 and prefix == len(cached_tokens or []) and has_logits:
        return PromptCachePlan(prefix, cached_logits, False, prefix)
    if rewindable and prefix > 0:
        start = len(input_tokens) - 1 if prefix >= len(input_tokens) else prefix
        return PromptCachePlan(start, None, False, start)
    return PromptCachePlan(0, None, True, 0)


def gpu_candidate_count(options: dict, max_candidate_count: int) -> int:
    """gpuCandidateCount, generate.ts:120-130."""
    if max_candidate_count == 0 or options.get("gpuSampling") is False or needs_full_logits(options):
        return 0
    temperature = options.get("temperature", 0.8)
    top_k = max(1, int(math.floor(options.get("topK", 40))))
    if temperature <= 0 or top_k == 1:
        return 1
    if top_k <= max_candidate_count:
        return top_k
    return 0


def is_stop_token(weights, token_id: int) -> bool:
    """isStopToken, generate.ts:51-59."""
    stop = getattr(weights, "stopTokenIds", None)
    if isinstance(stop, list) and len(stop) > 0:
        return token_id in stop
    return token_id == weights.endOfTextTokenId


@dataclass
class GenerateControls:
    rewindable: bool
    resetCache: Callable[[], None]
    computeToken: Callable[[int, int, bool, int], None]
    readLogits: Callable[[], Optional[np.ndarray]]
    prefillTokens: Optional[Callable] = None
    sampleToken: Optional[Callable[[int, dict], int]] = None
    maxGpuCandidateCount: int = 0


def generate(runner, prompt: str, options: Optional[dict], controls: GenerateControls) -> dict:
    """generateAsync, generate.ts:210-305, as a synchronous loop (the device
    work is asynchronous underneath; only readbacks wait)."""
    options = dict(options or {})
    max_new = options.get("maxNewTokens", 32)
    if options.get("inputTokens") is not None:
        input_tokens, new_budget = prepare_generation_from_tokens(options["inputTokens"], runner.maxTokens, max_new,
                                                                  runner.weights.endOfTextTokenId)
    else:
        input_tokens, new_budget = runner.weights.prepareGeneration(prompt, runner.maxTokens, max_new)
    plan = plan_prompt_cache(runner._cacheTokens or [], runner._cacheLogits, input_tokens, controls.rewindable)
    signal = options.get("signal")
    candidate_count = gpu_candidate_count(options, controls.maxGpuCandidateCount)
    use_gpu_sampling = candidate_count > 0 and controls.sampleToken is not None
    if plan.reset:
        controls.resetCache()
    if options.get("onPrefill"):
        options["onPrefill"]({"cachedPromptTokens": plan.reused, "promptTokens": len(input_tokens)})
    all_tokens = list(input_tokens)
    generated: List[int] = []
    logits = plan.logits
    needs_prompt_logits = new_budget > 0
    prefill_end = len(input_tokens) - 1 if needs_prompt_logits else len(input_tokens)
    loop_start = plan.start

    def report(done):
        if options.get("onPrefillProgress"):
            options["onPrefillProgress"]({"cachedPromptTokens": plan.reused, "completedPromptTokens": done,
                                          "freshPromptTokens": len(input_tokens) - plan.start,
                                          "promptTokens": len(input_tokens)})

    if options.get("prefillMode") is not False and controls.prefillTokens is not None and plan.start < prefill_end:
        controls.prefillTokens(input_tokens, plan.start, prefill_end, report)
        loop_start = prefill_end
    aborted = lambda: signal is not None and getattr(signal, "aborted", False)  # noqa: E731
    for i in range(loop_start, len(input_tokens)):
        if aborted():
            break
        compute_logits = needs_prompt_logits and i == len(input_tokens) - 1
        controls.computeToken(input_tokens[i], i, compute_logits, candidate_count if use_gpu_sampling else 0)
        if compute_logits:
            logits = None if use_gpu_sampling else controls.readLogits()
        report(i + 1)
    if options.get("onPrefillComplete"):
        options["onPrefillComplete"]({"cachedPromptTokens": plan.reused, "promptTokens": len(input_tokens)})
    sample_opts = {"temperature": options.get("temperature", 0.8), "topK": options.get("topK", 40),
                   **_sample_options(options)}
    if options.get("random") is not None:
        sample_opts["random"] = options["random"]
    for _ in range(new_budget):
        if aborted():
            break
        if not use_gpu_sampling and logits is None:
            break
        if use_gpu_sampling:
            next_token = controls.sampleToken(candidate_count, {**sample_opts, "tokens": all_tokens})
        else:
            next_token = sample_top_k(logits, tokens=all_tokens, **sample_opts)
        if is_stop_token(runner.weights, next_token):
            break
        all_tokens.append(next_token)
        generated.append(next_token)
        if options.get("onToken"):
            options["onToken"](runner.weights.tokenizer.decode(all_tokens), next_token)
        controls.computeToken(next_token, len(all_tokens) - 1, True, candidate_count if use_gpu_sampling else 0)
        logits = None if use_gpu_sampling else controls.readLogits()
    runner._cacheTokens = list(all_tokens)
    runner._cacheLogits = logits
    tok = runner.weights.tokenizer
    return {"tokens": all_tokens, "generatedTokens": generated, "text": tok.decode(all_tokens),
            "generatedText": tok.decode(generated), "cachedPromptTokens": plan.reused,
            "promptTokens": len(input_tokens), "aborted": aborted()}
