// GPU check of the Node.js host: node/runner.js's DecoderHIPRunner, on the
// synthetic tiny decoder and the 24-layer Qwen2.5-0.5B-shaped decoder, against
// the oracle's expectations in tests/golden/node_runner.json (written by
// tests/golden/make_node_golden.py): the logits after the prompt within
// max-abs 2e-2 / rel 1e-2, and the greedy stream of generateGreedy equal to
// the oracle's until a step whose top-2 logit gap is under 2e-2; then the
// device-fed greedy loop equal to the host loop, and one graph launch per
// decode token (the reference's submission contract); the device's top-8
// candidates equal the 8 best logits, and generate() with top-k sampling
// runs on them.
//
// Usage: node test_runner_gpu.js <path of tlm_addon.node>   (needs an MI355X)
'use strict';
const assert = require('assert');
const fs = require('fs');
const path = require('path');

const addon = require(path.resolve(process.argv[2] || path.join(__dirname, 'build', 'Release', 'tlm_addon.node')));
const {DecoderHIPRunner, generateGreedy, WORKLOADS} = require('./runner.js');

const golden = JSON.parse(fs.readFileSync(path.join(__dirname, '..', 'tests', 'golden', 'node_runner.json'), 'utf8'));
const {atol, rtol} = golden.tolerance;

function checkLogits(got, kept, label) {
  let worst = -Infinity;
  for (let j = 0; j < kept.ids.length; j++) {
    const e = kept.values[j], a = got[kept.ids[j]];
    assert.ok(Number.isFinite(a), `${label}: logit ${kept.ids[j]} not finite`);
    worst = Math.max(worst, Math.abs(a - e) - (atol + rtol * Math.abs(e)));
  }
  assert.ok(worst <= 0, `${label}: logits exceed the tolerance by ${worst}`);
  return worst;
}

function checkStream(got, c, label) {
  for (let s = 0; s < c.stream.length; s++) {
    if (got[s] !== c.stream[s]) {
      assert.ok(c.gaps[s] < atol, `${label}: token ${s} is ${got[s]}, the oracle's ${c.stream[s]} (gap ${c.gaps[s]})`);
      return s;  // a near-tie: the streams may part from here
    }
  }
  return c.stream.length;
}

async function main() {
  let passed = 0;
  for (const c of golden.cases) {
    const wl = WORKLOADS[c.workload];
    const t0 = Date.now();
    const runner = DecoderHIPRunner.synthetic(addon, wl, {maxTokens: 64});
    const label = wl.name;
    console.log(`# ${label}: weights uploaded in ${Date.now() - t0} ms`);
    // logits after the prompt (prefill of [0, n - 1), the last id with logits)
    runner.resetCache();
    await runner.prefillTokens(c.prompt, 0, c.prompt.length - 1);
    runner.computeToken(c.prompt[c.prompt.length - 1], c.prompt.length - 1, true);
    const worst = checkLogits(await runner.readLogits(), c.logits, label);
    console.log(`ok ${++passed} - ${label}: logits after the prompt (worst excess ${worst.toExponential(2)})`);
    // greedy stream through the generate loop
    const out = await generateGreedy(runner, c.prompt, c.stream.length);
    const same = checkStream(out.generated, c, label);
    console.log(`ok ${++passed} - ${label}: greedy stream = oracle for ${same} of ${c.stream.length} tokens`);
    // the device-fed loop equals the host loop; per token one graph launch, or
    // on the persistent schedule its two kernels (the layers; the LM head, whose
    // last block does the greedy merge)
    runner.resetCache();
    await runner.prefillTokens(c.prompt, 0, c.prompt.length - 1);
    runner.computeToken(c.prompt[c.prompt.length - 1], c.prompt.length - 1, true);
    const first = await runner.sampleToken(1, {temperature: 0});
    const before = runner.counts();
    const n = c.stream.length - 1;
    const t1 = process.hrtime.bigint();
    const dev = Array.from(await runner.decodeGreedy(first, c.prompt.length, n));
    const us = Number(process.hrtime.bigint() - t1) / 1e3;
    const after = runner.counts();
    assert.deepStrictEqual([first].concat(dev), out.generated.slice(0, n + 1));
    const ps = after.persistentTokens - before.persistentTokens;
    if (process.env.TLM_GRAPHS !== '0') {  // TLM_GRAPHS=0 (profiling) launches each kernel directly
      assert.strictEqual(after.graphLaunches - before.graphLaunches, n - ps);
      assert.strictEqual(after.kernelLaunches - before.kernelLaunches, 1 + 2 * ps);
    }
    console.log(`ok ${++passed} - ${label}: device loop = host loop, ${after.graphLaunches - before.graphLaunches} ` +
                `graph launches, ${ps} persistent tokens (${(us / n).toFixed(1)} us/token incl. one sync)`);
    // device top-k: the k best logits in the greedy order (TSLLogitSampler),
    // and generate() with top-k sampling draws its tokens from those lists
    runner.resetCache();
    runner.computeToken(c.prompt[0], 0, true);
    const logits = await runner.readLogits();
    const cands = await runner.readCandidates(8);
    const order = Array.from(logits.keys()).sort((a, b) => logits[b] - logits[a] || a - b).slice(0, 8);
    assert.deepStrictEqual(cands.map((x) => x[0]), order);
    cands.forEach((x) => assert.strictEqual(x[1], logits[x[0]]));
    let u = 0.3;
    const drawn = [];
    const sampled = await runner.generate('', {inputTokens: c.prompt, maxNewTokens: 4, temperature: 0.7, topK: 8,
      random: () => (u = (u * 7.13 + 0.17) % 1), onToken: (text, t) => drawn.push(t)});
    assert.strictEqual(sampled.generatedTokens.length, 4);
    assert.deepStrictEqual(drawn, sampled.generatedTokens);
    console.log(`ok ${++passed} - ${label}: device top-8 = the 8 best logits; top-k generate drew ` +
                JSON.stringify(sampled.generatedTokens));
    runner.close();
  }
  console.log('1..' + passed);
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : e);
  process.exit(1);
});
