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
  computeToken(tokenId, position, computeLogits) {
    this.addon.computeToken(this.model, tokenId, position, computeLogits === false ? 0 : TLM_LOGITS);
  }

  async prefillTokens(inputTokens, start, end, onProgress) {
    const tokens = Int32Array.from(inputTokens);
    for (let offset = start; offset < end; offset += this.prefillChunkSize) {
      const count = Math.min(this.prefillChunkSize, end - offset);
      this.addon.prefill(this.model, tokens, offset, offset + count);
      if (onProgress) await onProgress(offset + count);
    }
  }

  async readLogits() {
    return Float32Array.from(this.addon.readLogits(this.model, this._logits));
  }

  // Greedy reads the device argmax; k > 1 returns the device candidates to the
  // caller's sampleTopKCandidates (TSLLogits.ts:336-355).
  async sampleToken(candidateCount, opts) {
    const temperature = opts && opts.temperature !== undefined ? opts.temperature : 0.8;
    if (!(candidateCount > 1) || temperature <= 0) return this.addon.readToken(this.model);
    throw new Error('DecoderHIPRunner: top-k sampling needs the host sampler (readCandidates)');
  }

  readCandidates(k) {
    return this.addon.readCandidates(this.model, k, 0);
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

  // The device-fed greedy loop (tokens never leave the device until the end).
  decodeGreedy(tokenId, position, count) {
    return this.addon.decodeGreedy(this.model, tokenId, position, count);
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

// The greedy path of generateAsync (src/runtime/generate.ts:210-305) over the
// runner's controls: prefill [0, n - 1), the last prompt token with logits,
// then sample, stop on a stop token, compute the next position.
async function generateGreedy(runner, inputTokens, maxNewTokens, stopTokenIds) {
  const stops = new Set(stopTokenIds || []);
  const all = inputTokens.slice();
  const generated = [];
  runner.resetCache();
  const prefillEnd = maxNewTokens > 0 ? inputTokens.length - 1 : inputTokens.length;
  if (prefillEnd > 0) await runner.prefillTokens(inputTokens, 0, prefillEnd);
  for (let i = prefillEnd; i < inputTokens.length; i++) runner.computeToken(inputTokens[i], i, true);
  for (let i = 0; i < maxNewTokens; i++) {
    const next = await runner.sampleToken(1, {temperature: 0});
    if (stops.has(next)) break;
    all.push(next);
    generated.push(next);
    runner.computeToken(next, all.length - 1, true);
  }
  return {tokens: all, generated};
}

module.exports = {DecoderHIPRunner, generateGreedy, syntheticTensors, recipeOf, ropeInvFreq, WORKLOADS, FMT, T};
