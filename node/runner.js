// DecoderHIPRunner for Node.js: the method set that the reference's
// generateAsync drives (GenerateAsyncControls, src/runtime/generate.ts:31-49)
// implemented over the N-API addon (tlm_addon.cc), beside createTSLRunner
// (src/runtime/factory.ts:29-43).  Plain ES2019 so that Node 12 runs it
// without a TypeScript compiler; a TypeScript build would carry the same
// code with types.
//
//   const addon = require('./build/Release/tlm_addon.node');
//   const {DecoderHIPRunner, generateGreedy, WORKLOADS} = require('./runner.js');
//   const runner = DecoderHIPRunner.synthetic(addon, WORKLOADS.tiny, {maxTokens: 64});
//   const out = await generateGreedy(runner, promptIds, 32);
'use strict';

// tlm.h enums
const FMT = {f16: 1, q4: 2, f32: 3};
const T = {
  EMBED: 0, LM_HEAD: 1, LM_HEAD_SCALES: 2, FINAL_NORM: 3, ATTN_NORM: 4, FFN_NORM: 5, WQKV: 6, WQKV_SCALES: 7,
  BQKV: 8, WO: 9, WO_SCALES: 10, WGATE: 11, WGATE_SCALES: 12, WUP: 13, WUP_SCALES: 14, WDOWN: 15, WDOWN_SCALES: 16,
};
const TLM_LOGITS = 1;

// Benchmark decoders (Hugging Face config fields of the Llama / Qwen2 recipe)
// and how their weights are stored; the synthetic weights are N(0, 0.02)
// from the library's counter-based generator, one stream per (tensor, layer),
// norms 1.0 -- the same bytes the Python host produces for these workloads.
const WORKLOADS = {
  tiny: {
    name: 'tiny-llama-2x256',
    config: {hidden_size: 256, intermediate_size: 688, num_hidden_layers: 2, num_attention_heads: 4,
      num_key_value_heads: 2, head_dim: 64, vocab_size: 4096, rope_theta: 1e4, rms_norm_eps: 1e-6,
      tie_word_embeddings: false},
    storage: {linear: 'f16', head: 'f16', embed: 'f16', kv: 'f16'},
    qkvBias: false,
  },
  'qwen2.5-0.5b': {
    name: 'qwen2.5-0.5b-shape-q4',
    config: {hidden_size: 896, intermediate_size: 4864, num_hidden_layers: 24, num_attention_heads: 14,
      num_key_value_heads: 2, head_dim: 64, vocab_size: 151936, rope_theta: 1e6, rms_norm_eps: 1e-6,
      tie_word_embeddings: true},
    storage: {linear: 'q4', head: 'f16', embed: 'f16', kv: 'f16'},
    qkvBias: true,
  },
};
const STREAM = {embed: 1, lm_head: 2, final_norm: 3, attn_norm: 4, ffn_norm: 5, wqkv: 6, bqkv: 7, wo: 8, wgate: 9,
  wup: 10, wdown: 11};
const SEED = 0x5EED;

// ropeParameters (src/runtime/rope.ts:4-52), default RoPE: 1 / theta^(2i/dim)
// stored in a Float32Array.
function ropeInvFreq(dim, theta) {
  const inv = new Float32Array(dim / 2);
  for (let i = 0; i < inv.length; i++) inv[i] = 1 / Math.pow(theta, (2 * i) / dim);
  return inv;
}

function withDefault(v, d) {
  return v === undefined || v === null ? d : v;
}

// The decoder dimensions the recipe derives (load/DecoderRecipe.ts:348-405).
function recipeOf(config) {
  const heads = config.num_attention_heads;
  const headDim = config.head_dim || config.hidden_size / heads;
  return {
    hidden: config.hidden_size, inner: config.intermediate_size, layers: config.num_hidden_layers, heads,
    kvHeads: config.num_key_value_heads || heads, headDim, vocab: config.vocab_size,
    rotaryDim: headDim, theta: config.rope_theta || 10000, eps: config.rms_norm_eps || 1e-5,
    tied: config.tie_word_embeddings === true,
  };
}

class DecoderHIPRunner {
  // desc: the tlm_model_desc fields (camelCase); tensors(kind, layer) gives
  // the canonical host tensors to upload.
  constructor(addon, ctx, desc, options) {
    options = options || {};
    this.addon = addon;
    this.ctx = ctx;
    this.maxTokens = desc.maxTokens;
    this.vocabSize = desc.vocabSize;
    this.model = addon.modelCreate(ctx, desc);
    this.prefillChunkSize = withDefault(options.prefillChunkSize, 2048);
    this.prefillBatchRows = withDefault(options.prefillBatchRows, 64);
    this._logits = new Float32Array(desc.vocabSize);
    this._cacheTokens = [];
    this._cacheLogits = null;
    this.softcap = withDefault(options.finalLogitSoftcap, 0);
    // what generateAsync reads from runner.weights (generate.ts:11-16); a
    // checkpoint loader supplies its tokenizer and stop tokens here
    this.weights = Object.assign({
      stopTokenIds: [], endOfTextTokenId: 0, tokenizer: {decode: (ids) => ids.join(' ')},
      prepareGeneration: null,
    }, options.weights || {});
  }

  // A runner over the synthetic weights of a benchmark workload.
  static synthetic(addon, workload, options) {
    options = options || {};
    const r = recipeOf(workload.config);
    const st = workload.storage;
    const ctx = addon.open(withDefault(options.device, 0));
    const desc = {
      hiddenSize: r.hidden, intermediateSize: r.inner, numLayers: r.layers, numHeads: r.heads,
      numKvHeads: r.kvHeads, headDim: r.headDim, vocabSize: r.vocab, maxTokens: withDefault(options.maxTokens, 512),
      rotaryDim: r.rotaryDim, slidingWindow: 0, linearFmt: FMT[st.linear], headFmt: FMT[st.head],
      embedFmt: FMT[st.embed], kvFmt: FMT[st.kv], qkvBias: workload.qkvBias ? 1 : 0, tied: r.tied ? 1 : 0,
      rmsEps: r.eps, attentionFactor: 1.0, invFreq: ropeInvFreq(r.rotaryDim, r.theta),
    };
    const runner = new DecoderHIPRunner(addon, ctx, desc, options);
    runner._ownCtx = true;
    runner.upload(syntheticTensors(addon, r, st, workload.qkvBias));
    runner.finalize();
    return runner;
  }

  // uploadAndReleaseStaticWeights (src/tsl/releaseCPU.ts:79-110): the device
  // keeps its copy; the host arrays may be dropped afterwards.
  upload(tensors) {
    for (const t of tensors) {
      this.addon.modelUpload(this.model, t.id, t.layer, t.data);
      if (t.scales) this.addon.modelUpload(this.model, t.scalesId, t.layer, t.scales);
    }
  }

  finalize() {
    this.addon.modelFinalize(this.model);
    if (this.prefillBatchRows > 0) {
      try {
        this.addon.modelSetPrefill(this.model, this.prefillBatchRows, this.prefillChunkSize);
      } catch (e) {  // this model cannot batch: replay the decode graph (the reference's semantics)
        this.prefillBatchRows = 0;
        this.addon.modelSetPrefill(this.model, 0, 1);
      }
    }
  }

  // ---- GenerateAsyncControls ----
  // Enqueues one token (no wait); the reads below are the Promises.
  computeToken(tokenId, position, computeLogits) {
    this.addon.computeToken(this.model, tokenId, position, computeLogits === false ? 0 : TLM_LOGITS);
  }

  // Chunks of prefillChunkSize positions, each run off the JS thread (the
  // library waits for a batched chunk's overflow flag), then onProgress.
  async prefillTokens(inputTokens, start, end, onProgress) {
    const tokens = Int32Array.from(inputTokens);
    for (let offset = start; offset < end; offset += this.prefillChunkSize) {
      const count = Math.min(this.prefillChunkSize, end - offset);
      await this.addon.prefillAsync(this.model, tokens, offset, offset + count);
      if (onProgress) await onProgress(offset + count);
    }
  }

  // readChunkedLogits (src/tsl/TSLLogits.ts:71-83): resolves when the device
  // has finished the token, with a copy of its logits.
  async readLogits() {
    await this.addon.readLogitsAsync(this.model, this._logits);
    return Float32Array.from(this._logits);
  }

  // TSLLogitSampler.sampleToken (src/tsl/TSLLogits.ts:379-383): greedy reads
  // the device argmax; otherwise the device's top-k candidates are drawn on
  // the host (sampleTopKCandidates).
  async sampleToken(candidateCount, opts) {
    opts = opts || {};
    if (candidateCount <= 1 || opts.temperature <= 0) return this.addon.readTokenAsync(this.model);
    return sampleTopKCandidates(await this.readCandidates(candidateCount), opts);
  }

  // The device's candidateCount best (token, score) pairs, best first
  // (TSLLogitSampler.readCandidates, src/tsl/TSLLogits.ts:359-377).
  async readCandidates(candidateCount) {
    const c = await this.addon.readCandidatesAsync(this.model, candidateCount, this.softcap);
    const out = [];
    for (let i = 0; i < candidateCount; i++) out.push([c.tokens[i], c.scores[i]]);
    return out;
  }

  resetCache() {
    this._cacheTokens = [];
    this._cacheLogits = null;
    this.addon.resetCache(this.model);
  }

  get rewindable() {
    return true;
  }

  get maxGpuCandidateCount() {
    return 16;
  }

  // The controls object generateAsync takes (DecoderTSLRunner.ts:574-593).
  controls() {
    return {
      rewindable: this.rewindable,
      resetCache: () => this.resetCache(),
      computeToken: (t, p, logits) => this.computeToken(t, p, logits),
      prefillTokens: (toks, s, e, progress) => this.prefillTokens(toks, s, e, progress),
      readLogits: () => this.readLogits(),
      sampleToken: (k, o) => this.sampleToken(k, o),
      maxGpuCandidateCount: this.maxGpuCandidateCount,
    };
  }

  // DecoderTSLRunner.generate: generateAsync over this runner's controls.
  generate(prompt, options) {
    return generateAsync(this, prompt, options, this.controls());
  }

  // The device-fed greedy loop (tokens never leave the device until the
  // end): resolves with the count tokens.
  decodeGreedy(tokenId, position, count) {
    return this.addon.decodeGreedyAsync(this.model, tokenId, position, count);
  }

  counts() {
    return this.addon.modelCounts(this.model);
  }

  close() {
    if (this.model) this.addon.modelDestroy(this.model);
    this.model = null;
    if (this._ownCtx && this.ctx) this.addon.close(this.ctx);
    this.ctx = null;
  }
}

// The canonical host tensors of a synthetic workload (the Python host's
// weights.synthetic / HostWeights.tensor): fp16 bits, q4 (packed + scales) or
// fp32, Hugging Face [out][in] orientation, Q|K|V rows concatenated.
function syntheticTensors(addon, r, st, qkvBias) {
  const nqkv = (r.heads + 2 * r.kvHeads) * r.headDim;
  const shape = {
    embed: [r.vocab, r.hidden], lm_head: [r.vocab, r.hidden], final_norm: [r.hidden], attn_norm: [r.hidden],
    ffn_norm: [r.hidden], wqkv: [nqkv, r.hidden], bqkv: [nqkv], wo: [r.hidden, r.heads * r.headDim],
    wgate: [r.inner, r.hidden], wup: [r.inner, r.hidden], wdown: [r.hidden, r.inner],
  };
  const ids = {embed: T.EMBED, lm_head: T.LM_HEAD, final_norm: T.FINAL_NORM, attn_norm: T.ATTN_NORM,
    ffn_norm: T.FFN_NORM, wqkv: T.WQKV, bqkv: T.BQKV, wo: T.WO, wgate: T.WGATE, wup: T.WUP, wdown: T.WDOWN};
  const scaleIds = {lm_head: T.LM_HEAD_SCALES, wqkv: T.WQKV_SCALES, wo: T.WO_SCALES, wgate: T.WGATE_SCALES,
    wup: T.WUP_SCALES, wdown: T.WDOWN_SCALES};
  const linear = new Set(['wqkv', 'wo', 'wgate', 'wup', 'wdown']);
  const fmtOf = (kind) => linear.has(kind) ? st.linear : kind === 'lm_head' ? st.head : kind === 'embed' ? st.embed
    : 'f32';
  const out = [];
  const add = (kind, layer) => {
    const sh = shape[kind];
    const n = sh.reduce((a, b) => a * b, 1);
    const w = kind.endsWith('_norm') ? new Float32Array(n).fill(1)
      : addon.synthNormal(SEED, STREAM[kind] * 4096 + layer, n, 0.02);
    const fmt = fmtOf(kind);
    if (fmt === 'q4') {
      const q = addon.quantizeQ4(w, sh[0], sh[1]);
      out.push({id: ids[kind], layer, data: q.packed, scalesId: scaleIds[kind], scales: q.scales});
    } else if (fmt === 'f16') {
      out.push({id: ids[kind], layer, data: addon.f32ToF16(w)});
    } else {
      out.push({id: ids[kind], layer, data: w});
    }
  };
  add('embed', 0);
  if (!r.tied) add('lm_head', 0);
  add('final_norm', 0);
  for (let l = 0; l < r.layers; l++) {
    for (const k of ['attn_norm', 'ffn_norm', 'wqkv', 'wo', 'wgate', 'wup', 'wdown']) add(k, l);
    if (qkvBias) add('bqkv', l);
  }
  return out;
}

// ------------------------------------------------------------ sampling --
// softmax (src/runtime/math.ts:60-76): double exponentials stored in a
// Float32Array.
function softmax(values) {
  let max = -Infinity;
  for (let i = 0; i < values.length; i++) max = Math.max(max, values[i]);
  const out = new Float32Array(values.length);
  let sum = 0;
  for (let i = 0; i < values.length; i++) {
    const v = Math.exp(values[i] - max);
    out[i] = v;
    sum += v;
  }
  for (let i = 0; i < out.length; i++) out[i] /= sum;
  return out;
}

// sampleTopKCandidates (src/runtime/math.ts:527-547): candidates are
// [token, score] pairs, best first; temperature 0.8 and Math.random unless
// given.
function sampleTopKCandidates(candidates, opts) {
  opts = opts || {};
  const temperature = withDefault(opts.temperature, 0.8);
  const random = opts.random || Math.random;
  if (candidates.length === 0) return 0;
  if (temperature <= 0 || candidates.length === 1) return candidates[0][0];
  const values = new Float32Array(candidates.length);
  for (let i = 0; i < candidates.length; i++) values[i] = candidates[i][1] / Math.max(temperature, 1e-6);
  const p = softmax(values);
  let r = random();
  for (let i = 0; i < p.length; i++) {
    r -= p[i];
    if (r <= 0) return candidates[i][0];
  }
  return candidates[candidates.length - 1][0];
}

// Greedy choice over full logits (the temperature-0 branch of sampleTopK,
// math.ts:581-593: the first maximum wins).
function argmax(logits) {
  let best = 0;
  for (let i = 1; i < logits.length; i++) if (logits[i] > logits[best]) best = i;
  return best;
}

// ------------------------------------------------------------- planning --
// sharedPrefixLength (src/runtime/generate.ts:61-68).
function sharedPrefixLength(a, b) {
  a = a || [];
  b = b || [];
  const n = Math.min(a.length, b.length);
  let i = 0;
  while (i < n && a[i] === b[i]) i++;
  return i;
}

// prepareGenerationFromTokens (generate.ts:70-81): the prompt's last
// maxTokens - 1 tokens (the end-of-text token for an empty one) and the new
// tokens that fit after it.
function prepareGenerationFromTokens(tokens, maxTokens, maxNewTokens, endOfTextTokenId) {
  const budget = Math.max(1, maxTokens - 1);
  const inputTokens = tokens.length === 0 ? [endOfTextTokenId] : tokens.slice(-budget);
  return {inputTokens, newTokenBudget: Math.max(0, Math.min(maxNewTokens, maxTokens - inputTokens.length))};
}

// planPromptCache (generate.ts:98-118): reuse the cached prefix (with its
// logits when the whole cache is a prefix of the prompt), rewind to the shared
// prefix, or reset.
function planPromptCache(cachedTokens, cachedLogits, inputTokens, rewindable) {
  const prefix = sharedPrefixLength(cachedTokens, inputTokens);
  const hasLogits = cachedLogits !== null && cachedLogits !== undefined;
  if (prefix > 0 && prefix === (cachedTokens || []).length && hasLogits)
    return {start: prefix, logits: cachedLogits, reset: false, reused: prefix};
  if (rewindable && prefix > 0) {
    const start = prefix >= inputTokens.length ? inputTokens.length - 1 : prefix;
    return {start, logits: null, reset: false, reused: start};
  }
  return {start: 0, logits: null, reset: true, reused: 0};
}

// needsFullLogitsForSampling (math.ts:509-523) and gpuCandidateCount
// (generate.ts:120-130): how many device candidates sampling needs (0: full
// logits on the host).
function needsFullLogits(o) {
  const rep = withDefault(o.repetitionPenalty, 1);
  return o.forceFullLogits === true || (rep !== 1 && rep > 0) || withDefault(o.presencePenalty, 0) !== 0 ||
    withDefault(o.frequencyPenalty, 0) !== 0 || Math.max(0, Math.floor(withDefault(o.noRepeatNgramSize, 0))) >= 2;
}

function gpuCandidateCount(options, maxCandidateCount) {
  if (maxCandidateCount === 0 || options.gpuSampling === false || needsFullLogits(options)) return 0;
  const temperature = withDefault(options.temperature, 0.8);
  const topK = Math.max(1, Math.floor(withDefault(options.topK, 40)));
  if (temperature <= 0 || topK === 1) return 1;
  if (topK <= maxCandidateCount) return topK;
  return 0;
}

// isStopToken (generate.ts:51-59).
function isStopToken(runner, tokenId) {
  const stops = runner.weights.stopTokenIds;
  if (Array.isArray(stops) && stops.length > 0) return stops.indexOf(tokenId) >= 0;
  return tokenId === runner.weights.endOfTextTokenId;
}

// applyRepeatPenalties (src/runtime/math.ts:438-503): repetition, presence
// and frequency penalties over the last repeatLastN tokens, and -Infinity for
// the token that would repeat an n-gram; a penalised copy, or the input.
function applyRepeatPenalties(logits, tokens, o) {
  if (!tokens || tokens.length === 0) return logits;
  const rep = withDefault(o.repetitionPenalty, 1), pres = withDefault(o.presencePenalty, 0);
  const freq = withDefault(o.frequencyPenalty, 0), lastN = withDefault(o.repeatLastN, 64);
  const useRep = rep !== 1 && rep > 0, usePres = pres !== 0, useFreq = freq !== 0;
  const ngram = Math.max(0, Math.floor(withDefault(o.noRepeatNgramSize, 0)));
  const useNgrams = ngram >= 2 && tokens.length >= ngram - 1;
  if (!useRep && !usePres && !useFreq && !useNgrams) return logits;
  const out = logits.slice();
  if (useRep || usePres || useFreq) {
    const counts = new Map();
    for (let i = lastN > 0 ? Math.max(0, tokens.length - lastN) : 0; i < tokens.length; i++)
      counts.set(tokens[i], (counts.get(tokens[i]) || 0) + 1);
    for (const [t, count] of counts) {
      let v = out[t];
      if (useRep) v = v < 0 ? v * rep : v / rep;
      if (usePres) v -= pres;
      if (useFreq) v -= freq * count;
      out[t] = v;
    }
  }
  if (useNgrams) {
    const plen = ngram - 1, pstart = tokens.length - plen;
    for (let i = 0; i <= tokens.length - ngram; i++) {
      let match = true;
      for (let j = 0; j < plen && match; j++) match = tokens[i + j] === tokens[pstart + j];
      if (match) out[tokens[i + plen]] = -Infinity;
    }
  }
  return out;
}

// sampleTopK (src/runtime/math.ts:556-620) over full logits: penalties, then
// greedy for temperature <= 0 or topK 1 (first maximum), else a draw from the
// softmax of the topK best logits / temperature (ties keep the lower id).
function sampleTopK(logits, o) {
  o = o || {};
  logits = applyRepeatPenalties(logits, o.tokens, o);
  const temperature = withDefault(o.temperature, 0.8);
  const k = Math.min(Math.max(1, Math.floor(withDefault(o.topK, 40))), logits.length);
  if (temperature <= 0 || k === 1) return argmax(logits);
  const t = Math.max(temperature, 1e-6);
  const best = [];  // [id, value], best first
  for (let i = 0; i < logits.length; i++) {
    const v = logits[i] / t;
    if (best.length === k && !(v > best[k - 1][1])) continue;
    let j = best.length < k ? best.length : k - 1;
    while (j > 0 && best[j - 1][1] < v) j--;  // after the equal values already kept
    best.splice(j, 0, [i, v]);
    if (best.length > k) best.pop();
  }
  const p = softmax(best.map((c) => c[1]));
  let r = (o.random || Math.random)();
  for (let i = 0; i < p.length; i++) {
    r -= p[i];
    if (r <= 0) return best[i][0];
  }
  return best[best.length - 1][0];
}

// ------------------------------------------------------------- generate --
// generateAsync (src/runtime/generate.ts:210-305), the same control flow:
// prompt tokens (options.inputTokens, or weights.prepareGeneration(prompt)),
// the prompt-cache plan, prefill in chunks with progress callbacks, the
// prompt's last token with logits, then sample -> stop token? -> onToken ->
// compute, until the budget or an aborted signal.  Resolves with the
// GenerationResult fields (finishGeneration) and stores the cache state.
async function generateAsync(runner, prompt, options, controls) {
  options = options || {};
  const maxNew = withDefault(options.maxNewTokens, 32);
  let prepared;
  if (options.inputTokens) {
    prepared = prepareGenerationFromTokens(options.inputTokens, runner.maxTokens, maxNew,
      runner.weights.endOfTextTokenId);
  } else if (typeof runner.weights.prepareGeneration === 'function') {
    prepared = runner.weights.prepareGeneration(prompt, runner.maxTokens, maxNew);
  } else {
    throw new Error('DecoderHIPRunner: no tokenizer to prepare the prompt; pass options.inputTokens');
  }
  const inputTokens = prepared.inputTokens, newTokenBudget = prepared.newTokenBudget;
  const plan = planPromptCache(runner._cacheTokens || [], runner._cacheLogits, inputTokens, controls.rewindable);
  const signal = options.signal;
  const aborted = () => signal !== undefined && signal !== null && signal.aborted === true;
  const candidateCount = gpuCandidateCount(options, controls.maxGpuCandidateCount || 0);
  const useGpuSampling = candidateCount > 0 && typeof controls.sampleToken === 'function';
  if (plan.reset) controls.resetCache();
  if (options.onPrefill) options.onPrefill({cachedPromptTokens: plan.reused, promptTokens: inputTokens.length});
  const allTokens = inputTokens.slice();
  const generatedTokens = [];
  let logits = plan.logits;
  const needsPromptLogits = newTokenBudget > 0;
  const prefillEnd = needsPromptLogits ? inputTokens.length - 1 : inputTokens.length;
  let promptLoopStart = plan.start;
  const report = async (completed) => {
    if (options.onPrefillProgress) {
      options.onPrefillProgress({cachedPromptTokens: plan.reused, completedPromptTokens: completed,
        freshPromptTokens: inputTokens.length - plan.start, promptTokens: inputTokens.length});
    }
  };
  if (options.prefillMode !== false && typeof controls.prefillTokens === 'function' && plan.start < prefillEnd) {
    await controls.prefillTokens(inputTokens, plan.start, prefillEnd, report);
    promptLoopStart = prefillEnd;
  }
  for (let i = promptLoopStart; i < inputTokens.length; i++) {
    if (aborted()) break;
    const computeLogits = needsPromptLogits && i === inputTokens.length - 1;
    await controls.computeToken(inputTokens[i], i, computeLogits, useGpuSampling ? candidateCount : 0);
    if (computeLogits) logits = useGpuSampling ? null : await controls.readLogits();
    await report(i + 1);
  }
  if (options.onPrefillComplete) {
    options.onPrefillComplete({cachedPromptTokens: plan.reused, promptTokens: inputTokens.length});
  }
  for (let i = 0; i < newTokenBudget; i++) {
    if (aborted()) break;
    if (!useGpuSampling && logits === null) break;
    const sampleOpts = Object.assign({}, options, {tokens: allTokens});
    const next = useGpuSampling ? await controls.sampleToken(candidateCount, sampleOpts)
      : sampleTopK(logits, sampleOpts);
    if (isStopToken(runner, next)) break;
    allTokens.push(next);
    generatedTokens.push(next);
    if (options.onToken) options.onToken(runner.weights.tokenizer.decode(allTokens), next);
    await controls.computeToken(next, allTokens.length - 1, true, useGpuSampling ? candidateCount : 0);
    logits = useGpuSampling ? null : await controls.readLogits();
  }
  runner._cacheTokens = allTokens.slice();
  runner._cacheLogits = logits;
  const tok = runner.weights.tokenizer;
  return {
    tokens: allTokens, generatedTokens, text: tok.decode(allTokens), generatedText: tok.decode(generatedTokens),
    cachedPromptTokens: plan.reused, promptTokens: inputTokens.length, aborted: aborted(),
  };
}

// The greedy path alone: prompt ids in, greedy ids out (no cache reuse).
async function generateGreedy(runner, inputTokens, maxNewTokens, stopTokenIds) {
  runner.resetCache();
  const saved = runner.weights.stopTokenIds;
  if (stopTokenIds) runner.weights.stopTokenIds = stopTokenIds;
  try {
    const r = await runner.generate('', {inputTokens, maxNewTokens, temperature: 0});
    return {tokens: r.tokens, generated: r.generatedTokens};
  } finally {
    runner.weights.stopTokenIds = saved;
  }
}

module.exports = {DecoderHIPRunner, generateAsync, generateGreedy, sampleTopKCandidates, sampleTopK,
  applyRepeatPenalties, planPromptCache,
  gpuCandidateCount, prepareGenerationFromTokens, isStopToken, softmax, syntheticTensors, recipeOf, ropeInvFreq,
  WORKLOADS, FMT, T};
