"""DecoderHIPRunner: the reference's runner surface over libtlm.

Mirrors decoder/DecoderTSLRunner.ts:62-594 (paths relative to
packages/three-llm/src/): the same method names, argument meaning and
defaults (maxTokens = min(option, contextLimit), prefillChunkSize 32 when
prompts replay the decode graph, logitCandidateCount 8), driving the device
through the C ABI instead of three.js compute nodes.  One decode token is one HIP graph launch (the
reference's single queue submission per token, submission.browser.test.ts:54).
"""
from __future__ import annotations

from typing import Callable, List, Optional

import numpy as np

from . import generate as gen
from . import tlm
from .weights import HostWeights


class TinyTokenizer:
    """Token ids in, comma-joined ids out (the reference's test tokenizer,
    src/test/helpers.ts:23-33)."""

    def __init__(self, ids=(1, 2), eos: int = 0):
        self.ids = list(ids)
        self.endOfTextTokenId = eos

    def encode(self, text: str) -> List[int]:
        return list(self.ids)

    def decode(self, ids) -> str:
        return ",".join(str(int(i)) for i in ids)


class RunnerWeights:
    """The fields generateAsync reads from runner.weights (generate.ts:11-23)."""

    def __init__(self, host: HostWeights, tokenizer):
        r = host.recipe
        self.host = host
        self.recipe = r
        self.tokenizer = tokenizer
        self.endOfTextTokenId = r.end_of_text_token_id
        self.stopTokenIds = list(r.stop_token_ids)
        self.vocabSize = r.vocab_size
        self.hiddenSize = r.hidden_size

    def contextLimit(self) -> int:
        return self.recipe.context_limit

    def prepareGeneration(self, prompt: str, max_tokens: int, max_new_tokens: int):
        """prepareGeneration, load/tensors.ts:257-270."""
        encoded = self.tokenizer.encode(prompt)
        budget = max(1, max_tokens - 1)
        inputs = [self.endOfTextTokenId] if len(encoded) == 0 else list(encoded)[-budget:]
        return inputs, max(0, min(max_new_tokens, max_tokens - len(inputs)))


class DecoderHIPRunner:
    def __init__(self, weights: HostWeights, options: Optional[dict] = None, ctx: Optional[tlm.Context] = None,
                 tokenizer=None):
        options = options or {}
        self.ctx = ctx or tlm.Context(options.get("device", 0))
        self._own_ctx = ctx is None
        self.weights = RunnerWeights(weights, tokenizer or TinyTokenizer(eos=weights.recipe.end_of_text_token_id))
        limit = weights.recipe.context_limit
        self.maxTokens = min(options.get("maxTokens") or limit, limit)
        self.logitCandidateCount = min(options.get("logitCandidateCount") or 8, 16)  # device top-k holds <= 16
        desc, inv = weights.model_desc(self.maxTokens)
        self.model = tlm.Model(self.ctx, desc, inv, layer_windows=weights.recipe.layer_windows)
        weights.upload(self.model)
        self.model.finalize()
        # Batched (MFMA) prefill for chunks of at least prefillBatchRows
        # positions; the reference always replays the decode graph per position,
        # in submissions of prefillChunkSize (default 32).  With the batched
        # path on, a chunk is one batched pass, so the default chunk is 2048.
        self.prefillBatchRows = int(options.get("prefillBatchRows", 64))
        self.batchedPrefill = False
        chunk = options.get("prefillChunkSize")
        try:
            self.model.set_prefill(self.prefillBatchRows, max(chunk or 2048, 1))
            self.batchedPrefill = self.prefillBatchRows > 0
        except tlm.TlmError:
            self.model.set_prefill(0, 1)
        self.prefillChunkSize = chunk or (2048 if self.batchedPrefill else 32)
        self._cacheTokens: Optional[List[int]] = None
        self._cacheLogits: Optional[np.ndarray] = None

    @classmethod
    def from_checkpoint(cls, path: str, options: Optional[dict] = None, ctx: Optional[tlm.Context] = None,
                        storage=None, tokenizer=None) -> "DecoderHIPRunner":
        """createTSLRunner(url) for a local Hugging Face directory (config.json +
        safetensors shards, and the tokenizer when vocab.json / tokenizer.json
        is there; factory.ts:29-43, HFModelBundle.ts:106-135): linears packed
        to q4 g32 at upload unless `storage` says otherwise."""
        import os
        from . import checkpoint, tokenizer as tk
        hw, config = checkpoint.load_checkpoint(path, storage)
        if tokenizer is None and any(os.path.isfile(os.path.join(path, f))
                                     for f in ("vocab.json", "tokenizer.json")):
            tokenizer = tk.load_tokenizer(path, config, list(hw.recipe.stop_token_ids))
        return cls(hw, options, ctx=ctx, tokenizer=tokenizer)

    # ---- GenerateAsyncControls (generate.ts:31-49) ----
    def computeToken(self, tokenId: int, position: int, computeLogits: bool = True, sampleCandidateCount: int = 0):
        """DecoderTSLRunner.computeToken (:487-502): enqueue, do not wait."""
        self.model.compute_token(tokenId, position, logits=computeLogits)

    def prefillTokens(self, inputTokens, start: int, end: int, onProgress: Optional[Callable[[int], None]] = None):
        """DecoderTSLRunner.prefillTokens (:504-530): positions [start, end)
        without logits, in chunks of prefillChunkSize with progress callbacks."""
        tokens = np.asarray(inputTokens, np.int32)
        for offset in range(start, end, self.prefillChunkSize):
            count = min(self.prefillChunkSize, end - offset)
            self.model.prefill(tokens, offset, offset + count)
            if onProgress:
                onProgress(offset + count)

    def readLogits(self) -> np.ndarray:
        """DecoderTSLRunner.readLogits (:532-535)."""
        return self.model.read_logits()

    def sampleToken(self, candidateCount: int, options: Optional[dict] = None) -> int:
        """TSLLogitSampler.sampleToken (TSLLogits.ts:351-355): greedy reads the
        device argmax (4 bytes); top-k takes the k best candidates from the
        device (readCandidates, :336-349) and draws with sampleTopKCandidates."""
        options = options or {}
        if candidateCount <= 1 or options.get("temperature", 0.8) <= 0:
            return self.model.read_token()
        k = min(max(1, candidateCount), self.logitCandidateCount)
        candidates = self.readCandidates(k)
        kw = {"temperature": options.get("temperature", 0.8)}
        if options.get("random") is not None:
            kw["random"] = options["random"]
        return gen.sample_top_k_candidates(candidates, **kw)

    def readCandidates(self, count: int):
        """TSLLogitSampler.readCandidates: [(token, score)], best first."""
        return self.model.read_candidates(min(max(1, count), self.logitCandidateCount))

    def resetCache(self):
        """DecoderTSLRunner.resetCache (:541-546)."""
        self._cacheTokens = []
        self._cacheLogits = None
        self.model.reset_cache()

    def generate(self, prompt: str = "", options: Optional[dict] = None) -> dict:
        """DecoderTSLRunner.generate (:580-593) -> generateAsync."""
        return gen.generate(self, prompt, options, gen.GenerateControls(
            rewindable=True, resetCache=self.resetCache, computeToken=self.computeToken,
            readLogits=self.readLogits, prefillTokens=self.prefillTokens, sampleToken=self.sampleToken,
            maxGpuCandidateCount=self.logitCandidateCount))

    # ---- device-resident greedy decode (no host round trip per token) ----
    def decodeGreedy(self, tokenId: int, position: int, count: int) -> np.ndarray:
        return self.model.decode_greedy(tokenId, position, count)

    def close(self):
        self.model.close()
        if self._own_ctx:
            self.ctx.close()
