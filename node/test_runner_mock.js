// The Node host over a stand-in library (test_mock_tlm.c, the C ABI with a
// formula decoder), no GPU needed: the addon's Promise reads run off the JS
// thread and reject with the reading thread's tlm_last_error(); the runner's
// generate() follows generateAsync (src/runtime/generate.ts:210-305) --
// prompt-cache plan, prefill, greedy, device top-k sampling
// (sampleTopKCandidates, math.ts:527-547), host sampling with penalties
// (sampleTopK), stop tokens, onToken.
// Usage: TLM_LIB=<mock .so> node test_runner_mock.js <path of tlm_addon.node>
'use strict';
const assert = require('assert');
const path = require('path');

const tlm = require(path.resolve(process.argv[2] || path.join(__dirname, 'build', 'Release', 'tlm_addon.node')));
const R = require('./runner.js');

const V = 97;
// the mock's decoder (test_mock_tlm.c): the greedy successor and the logits
const next = (token, pos) => (7 * token + 3 * pos + 1) % V;
const logit = (token, pos, v) => v === next(token, pos) ? 1 : ((37 * v + token) % 101) / 1000;

function runner(options, maxTokens) {
  const ctx = tlm.open(0);
  const desc = {hiddenSize: 64, intermediateSize: 64, numLayers: 1, numHeads: 1, numKvHeads: 1, headDim: 64,
    vocabSize: V, maxTokens: maxTokens || 64, rotaryDim: 0};
  const r = new R.DecoderHIPRunner(tlm, ctx, desc, Object.assign({prefillBatchRows: 0}, options || {}));
  r._ownCtx = true;
  return r;
}

// Seeded uniform draws (a linear congruential generator) for the samplers.
function lcg(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296;
  };
}

// sampleTopKCandidates written out for the check: softmax of score / T in
// doubles stored as fp32, then the first cumulative sum past the draw.
function expectedDraw(cands, temperature, u) {
  const vals = cands.map((c) => Math.fround(c[1] / temperature));
  const m = Math.max.apply(null, vals);
  const ex = vals.map((v) => Math.fround(Math.exp(v - m)));
  const sum = ex.reduce((a, b) => a + b, 0);
  let r = u;
  for (let i = 0; i < ex.length; i++) {
    r -= Math.fround(ex[i] / sum);
    if (r <= 0) return cands[i][0];
  }
  return cands[cands.length - 1][0];
}

const checks = [];
function check(name, fn) {
  checks.push([name, fn]);
}

check('a read resolves off the JS thread: a timer fires while it waits', async () => {
  const r = runner();
  r.computeToken(5, 0, true);
  let ticked = false;
  const timer = new Promise((res) => setTimeout(() => { ticked = true; res(); }, 1));
  const logits = await r.readLogits();
  await timer;
  assert.ok(ticked);
  assert.strictEqual(logits.length, V);
  for (let v = 0; v < V; v++) assert.strictEqual(logits[v], Math.fround(logit(5, 0, v)));
  r.close();
});

check('a failed read rejects with the library error of the reading thread and its code', async () => {
  const r = runner({}, 13);  // the mock fails every read of such a model
  r.computeToken(1, 0, true);
  const reads = [() => r.readLogits(), () => r.sampleToken(1, {temperature: 0}), () => r.readCandidates(4),
    () => r.decodeGreedy(1, 0, 3), () => r.prefillTokens([1, 2, 3], 0, 3)];
  for (const read of reads) {
    let err = null;
    try {
      await read();
    } catch (e) {
      err = e;
    }
    assert.ok(err instanceof Error, 'rejected');
    assert.strictEqual(err.code, -2);  // TLM_ERR_HIP
    assert.strictEqual(err.message, 'TLMModel: mock read failure');
  }
  r.close();
});

check('while a read is pending every other call on the model throws TLM_ERR_STATE', async () => {
  const r = runner();
  r.computeToken(3, 0, true);
  const p = r.readLogits();
  for (const f of [() => r.computeToken(4, 1, true), () => tlm.readToken(r.model), () => r.close()]) {
    let err = null;
    try {
      f();
    } catch (e) {
      err = e;
    }
    assert.ok(err && err.code === -4 && /pending/.test(err.message), String(err && err.message));
  }
  await p;
  r.computeToken(4, 1, true);  // settled: usable again
  assert.strictEqual(await r.sampleToken(1, {temperature: 0}), next(4, 1));
  r.close();
});

check('generate, greedy: prefill, then the device argmax each step; onToken sees the text', async () => {
  const r = runner();
  const seen = [];
  const prompt = [3, 11, 8, 40];
  const out = await r.generate('', {inputTokens: prompt, maxNewTokens: 6, temperature: 0,
    onToken: (text, t) => seen.push([text, t])});
  let t = prompt[prompt.length - 1], pos = prompt.length - 1;
  const want = [];
  for (let i = 0; i < 6; i++) {
    const n = next(t, pos);
    want.push(n);
    t = n;
    pos++;
  }
  assert.deepStrictEqual(out.generatedTokens, want);
  assert.deepStrictEqual(out.tokens, prompt.concat(want));
  assert.strictEqual(out.promptTokens, 4);
  assert.strictEqual(out.cachedPromptTokens, 0);
  assert.deepStrictEqual(seen.map((s) => s[1]), want);
  assert.strictEqual(seen[5][0], prompt.concat(want).join(' '));
  assert.ok(r.counts().replayedPositions >= 3);  // the prompt's first 3 positions went through prefillTokens
  // the device-fed loop gives the same stream
  assert.deepStrictEqual(Array.from(await r.decodeGreedy(prompt[3], 3, 6)), want);
  r.close();
});

check('generate stops at a stop token (weights.stopTokenIds, else endOfTextTokenId)', async () => {
  const prompt = [2, 9];
  const first = next(9, 1);
  const r = runner({weights: {stopTokenIds: [next(first, 2)]}});
  const out = await r.generate('', {inputTokens: prompt, maxNewTokens: 8, temperature: 0});
  assert.deepStrictEqual(out.generatedTokens, [first]);
  const r2 = runner({weights: {endOfTextTokenId: first}});
  assert.deepStrictEqual((await r2.generate('', {inputTokens: prompt, maxNewTokens: 8, temperature: 0}))
    .generatedTokens, []);
  r.close();
  r2.close();
});

check('generate reuses the prompt cache: a continued prompt prefills only its new tokens', async () => {
  const r = runner();
  const a = await r.generate('', {inputTokens: [5, 6, 7], maxNewTokens: 2, temperature: 0});
  const progress = [];
  const b = await r.generate('', {inputTokens: a.tokens.concat([12, 13]), maxNewTokens: 2, temperature: 0,
    onPrefillProgress: (p) => progress.push(p)});
  assert.strictEqual(b.cachedPromptTokens, a.tokens.length);
  assert.strictEqual(progress[progress.length - 1].freshPromptTokens, 2);
  // the same tokens as a fresh run (rewind or not, the mock's state is the last token)
  const c = await runner().generate('', {inputTokens: a.tokens.concat([12, 13]), maxNewTokens: 2, temperature: 0});
  assert.deepStrictEqual(b.generatedTokens, c.generatedTokens);
  assert.deepStrictEqual(R.planPromptCache([1, 2, 3], null, [1, 2, 9], true), {start: 2, logits: null, reset: false,
    reused: 2});
  assert.deepStrictEqual(R.planPromptCache([1, 2, 3], null, [4], false), {start: 0, logits: null, reset: true,
    reused: 0});
  const L = new Float32Array(2);
  assert.strictEqual(R.planPromptCache([1, 2], L, [1, 2, 3], true).logits, L);
  r.close();
});

check('top-k sampling draws from the device candidates with sampleTopKCandidates', async () => {
  const r = runner();
  const prompt = [4, 20];
  const u = lcg(99);
  const draws = lcg(99);
  const out = await r.generate('', {inputTokens: prompt, maxNewTokens: 5, temperature: 0.01, topK: 4, random: u});
  let t = prompt[1], pos = 1;
  for (const got of out.generatedTokens) {
    const cands = [];
    for (let v = 0; v < V; v++) cands.push([v, Math.fround(logit(t, pos, v))]);
    cands.sort((a, b) => b[1] - a[1] || a[0] - b[0]);
    assert.strictEqual(got, expectedDraw(cands.slice(0, 4), 0.01, draws()));
    t = got;
    pos++;
  }
  assert.strictEqual(R.gpuCandidateCount({temperature: 0.7, topK: 8}, 16), 8);
  assert.strictEqual(R.gpuCandidateCount({temperature: 0.7, topK: 40}, 16), 0);
  assert.strictEqual(R.gpuCandidateCount({repetitionPenalty: 1.2}, 16), 0);
  assert.strictEqual(R.gpuCandidateCount({temperature: 0}, 16), 1);
  r.close();
});

check('penalties read the full logits and sample on the host (applyRepeatPenalties, sampleTopK)', async () => {
  const r = runner();
  const prompt = [1, 2];
  // repetitionPenalty halves the greedy token's logit (1 -> 0.5) once it is in
  // the history, so a repeat-prone stream changes; topK 1 keeps it greedy
  const out = await r.generate('', {inputTokens: prompt, maxNewTokens: 4, temperature: 0.5, topK: 1,
    repetitionPenalty: 2.0, repeatLastN: 64});
  let t = prompt[1], pos = 1;
  const hist = prompt.slice();
  for (const got of out.generatedTokens) {
    const logits = new Float32Array(V);
    for (let v = 0; v < V; v++) logits[v] = logit(t, pos, v);
    const pen = R.applyRepeatPenalties(logits, hist, {repetitionPenalty: 2.0, repeatLastN: 64});
    let best = 0;
    for (let v = 1; v < V; v++) if (pen[v] > pen[best]) best = v;
    assert.strictEqual(got, best);
    hist.push(got);
    t = got;
    pos++;
  }
  const l = new Float32Array([0.5, -0.5, 2, 1]);
  assert.deepStrictEqual(Array.from(R.applyRepeatPenalties(l, [1, 2, 2], {repetitionPenalty: 2, presencePenalty: 0.1,
    frequencyPenalty: 0.05})), [0.5, Math.fround(-0.5 * 2 - 0.1 - 0.05), Math.fround(2 / 2 - 0.1 - 0.1), 1]);
  assert.strictEqual(R.applyRepeatPenalties(l, [0, 3, 0], {noRepeatNgramSize: 2})[3], -Infinity);
  assert.strictEqual(R.sampleTopK(new Float32Array([1, 5, 5, 2]), {temperature: 0.5, topK: 2, random: () => 0.9}), 2);
  assert.strictEqual(R.sampleTopKCandidates([[7, 1], [3, 0.5]], {temperature: 0}), 7);
  r.close();
});

(async () => {
  let n = 0;
  for (const [name, fn] of checks) {
    await fn();
    n++;
    console.log('ok ' + n + ' - ' + name);
  }
  console.log('1..' + n);
})().catch((e) => {
  console.error(e && e.stack ? e.stack : e);
  process.exit(1);
});
