"use strict";
/*
 * The decode loop (node/session.js) on the GPU against a restatement of the
 * reference's loop (src/runtime/gemma-session.ts:659-782, 1305-1345) driven
 * by the oracle sampler (oracle/sampler_ref.js) and the oracle byte-DFA
 * masker (oracle/constraint_ref.js), over a synthetic vocabulary and a
 * deterministic synthetic model: the same tokens, stops, draw counts,
 * log-probabilities and errors, for plain draws with penalties over a
 * history that starts with the prompt, GPU-greedy and penalised T=0 rows,
 * stop ids, a compiled constraint with acceptToken and termination rules,
 * the optional reasoning channel inside a constraint, and required
 * reasoning (forced prefix, text-only channel, END_CHANNEL at 16 / 64).
 */
const assert = require("assert");
const path = require("path");
const { test, run } = require("./harness");

const ROOT = path.join(__dirname, "..", "..");
const g = require(path.join(ROOT, "gemma-webgpu-engine_amd", "node"));
const session = require(path.join(ROOT, "gemma-webgpu-engine_amd", "node", "session.js"));
const oracle = require(path.join(ROOT, "oracle", "sampler_ref.js"));
const { ByteDfaMasker } = require(path.join(ROOT, "oracle", "constraint_ref.js"));

const V = 3000;
const START = 100;
const END = 101;
const SPECIAL = new Set([0, 1, 2, 50, START, END, 106]);

// ------------------------------------------------------------ vocabulary
function makeTokenizer() {
  const rng = new oracle.SeededRandom(4242);
  const alphabet = ["a", "b", "c", "d", " ", "1", "2", "{", "}", "\"", ":", ",", "é", "x"];
  const table = [];
  for (let id = 0; id < V; id += 1) {
    if (SPECIAL.has(id)) { table.push(null); continue; }
    if (id === 200) { table.push(Buffer.from("thought")); continue; }
    if (id === 201) { table.push(Buffer.from("\n")); continue; }
    const n = 1 + Math.floor(rng.next() * 3);
    let w = "";
    for (let k = 0; k < n; k += 1) w += alphabet[Math.floor(rng.next() * alphabet.length)];
    table.push(Buffer.from(w, "utf8"));
  }
  return {
    vocabularySize: V,
    tokenBytes: (id) => (id >= 0 && id < V ? table[id] : null),
    encodeText: (text) => {
      assert.strictEqual(text, "thought\n");
      return [200, 201];
    },
    table,
  };
}

// --------------------------------------------------------------- model
function row(seed) {
  const rng = new oracle.SeededRandom(seed);
  const out = new Float32Array(V);
  for (let i = 0; i < V; i += 2) {
    const u1 = Math.max(rng.next(), 1e-12);
    const u2 = rng.next();
    const r = Math.sqrt(-2 * Math.log(u1)) * 3;
    out[i] = r * Math.cos(2 * Math.PI * u2);
    if (i + 1 < V) out[i + 1] = r * Math.sin(2 * Math.PI * u2);
  }
  return out;
}
function argmax(x) {
  let best = 0;
  for (let i = 1; i < x.length; i += 1) if (x[i] > x[best]) best = i;
  return best;
}
// logits keyed by (position, last token); bias: (logits, position) => void
function makeModel(prompt, bias) {
  let pos = 0;
  const out = (last, mode) => {
    const l = row(1000 + 7919 * pos + last);
    if (bias) bias(l, pos);
    pos += 1;
    return mode === "greedy" ? { prediction: { token: argmax(l) } } : { logits: l, prediction: { token: argmax(l) } };
  };
  return { first: out(prompt[prompt.length - 1], "logits"), evaluateToken: (t, mode) => out(t, mode) };
}

// ------------------------------------------------ the reference's loop
function logSoftmaxAt(l, t) {
  let m = -Infinity;
  for (const x of l) if (x > m) m = x;
  let s = 0;
  for (const x of l) s += Math.exp(x - m);
  return (l[t] - m) - Math.log(s);
}
function referenceLoop(prompt, model, tok, options, thinking) {
  const decoding = Object.assign({}, options);
  delete decoding.constraint;
  delete decoding.requireReasoning;
  delete decoding.captureTokenLogProbabilities;
  const cfg = g.resolveGemmaGenerationConfig(decoding);
  const requireReasoning = options.requireReasoning === true;
  const capture = options.captureTokenLogProbabilities === true;
  const greedyGpu = cfg.temperature === 0 && cfg.repetitionPenalty === 1 && cfg.frequencyPenalty === 0 && cfg.presencePenalty === 0;
  let dfa = null;
  let masker = null;
  let state = 0;
  let viable = null;
  if (options.constraint) {
    dfa = g.compileGenerationConstraint(options.constraint).dfa;
    const offsets = new Float64Array(V + 1);
    tok.table.forEach((b, k) => { offsets[k + 1] = offsets[k] + (b ? b.length : 0); });
    const bytes = new Uint8Array(offsets[V]);
    tok.table.forEach((b, k) => { if (b) bytes.set(b, offsets[k]); });
    masker = new ByteDfaMasker(Int32Array.from(dfa.next), dfa.finals, dfa.stateCount, offsets, bytes);
    viable = masker.viable;
    state = dfa.initial;
  }
  let active = !!dfa;
  let allow = thinking;
  let inCh = false;
  let content = 0;
  const forced = requireReasoning ? [START, 200, 201] : [];
  const mode = dfa || requireReasoning || capture || !greedyGpu ? "logits" : "greedy";
  const random = new oracle.SeededRandom(cfg.seed);
  let draws = 0;
  const rnd = () => { draws += 1; return random.next(); };
  const history = prompt.slice();
  const outTokens = [];
  const lps = [];
  const stops = new Set(cfg.stopTokenIds);
  const ends = new Set([1, 50, 106]);
  let out = model.first;
  let stoppedOnEndToken = false;
  let stoppedOnStopToken = false;
  for (let index = 0; index < cfg.maxNewTokens; index += 1) {
    let token = out.prediction ? out.prediction.token : 0;
    if (index < forced.length) token = forced[index];
    else if (requireReasoning && inCh) {
      if (content >= 64) token = END;
      else {
        const m = new Float32Array(V).fill(-Infinity);
        for (let id = 0; id < V; id += 1) if (tok.table[id] !== null) m[id] = out.logits[id];
        if (content >= 16) m[END] = out.logits[END];
        token = oracle.sampleToken(m, history, cfg, rnd);
      }
    } else if (dfa && active) {
      const term = new Set([1, 50, 106].concat(cfg.stopTokenIds));
      const legal = new Set(Array.from(masker.legalTokenIds(state)).concat(allow ? [START] : []).filter((id) => !term.has(id)));
      if (dfa.finals[state]) term.forEach((id) => legal.add(id));
      if (legal.size === 0) throw new Error("Generation constraint reached a tokenization dead end");
      const m = new Float32Array(V).fill(-Infinity);
      legal.forEach((id) => { m[id] = out.logits[id]; });
      token = oracle.sampleToken(m, history, cfg, rnd);
    } else if (requireReasoning || !greedyGpu || (dfa && !active)) {
      token = oracle.sampleToken(out.logits, history, cfg, rnd);
    }
    if (ends.has(token)) { stoppedOnEndToken = true; break; }
    if (stops.has(token)) { stoppedOnStopToken = true; break; }
    const lp = capture ? logSoftmaxAt(out.logits, token) : null;
    const starts = allow && token === START;
    allow = false;
    if (starts) { active = false; inCh = true; }
    else if (dfa && active) {
      const b = tok.table[token];
      if (!b) throw new Error(`Constraint selected non-text token ${token}`);
      for (const x of b) {
        state = dfa.next[state * 256 + x];
        if (state < 0 || !viable[state]) throw new Error("Selected token violates the generation constraint");
      }
    }
    outTokens.push(token);
    if (lp !== null) lps.push(lp);
    history.push(token);
    if (inCh && token === END) { inCh = false; if (dfa) active = true; }
    else if (inCh && index >= forced.length) content += 1;
    if (index + 1 < cfg.maxNewTokens) out = model.evaluateToken(token, mode);
  }
  if (dfa && !dfa.finals[state]) {
    throw new Error("Max tokens reached before the generation constraint completed; increase maxNewTokens");
  }
  return { tokenIds: outTokens, stoppedOnEndToken, stoppedOnStopToken, draws, tokenLogProbabilities: lps };
}

async function compare(name, options, opts) {
  const tok = makeTokenizer();
  const prompt = opts.prompt || [2, 300, 301, 302, 303];
  let want;
  let wantError = null;
  try {
    want = referenceLoop(prompt, makeModel(prompt, opts.bias), tok, options, opts.thinking === true);
  } catch (e) {
    wantError = e.message;
  }
  let got;
  let gotError = null;
  try {
    got = await session.generate({ promptTokenIds: prompt, model: makeModel(prompt, opts.bias), tokenizer: tok,
      options, thinking: opts.thinking === true });
  } catch (e) {
    gotError = e.message;
  }
  assert.strictEqual(gotError, wantError, name + ": error");
  if (wantError) return null;
  assert.deepStrictEqual(got.tokenIds, want.tokenIds, name + ": tokens");
  assert.strictEqual(got.stoppedOnEndToken, want.stoppedOnEndToken, name + ": end token");
  assert.strictEqual(got.stoppedOnStopToken, want.stoppedOnStopToken, name + ": stop token");
  assert.strictEqual(got.draws, want.draws, name + ": draws");
  assert.strictEqual(got.tokenLogProbabilities.length, want.tokenLogProbabilities.length, name + ": log-probabilities");
  got.tokenLogProbabilities.forEach((x, k) => assert.ok(Math.abs(x - want.tokenLogProbabilities[k]) <= 1e-9 * Math.max(1, Math.abs(x)),
    `${name}: log-probability ${k}: ${x} vs ${want.tokenLogProbabilities[k]}`));
  return got;
}

let asyncTests = [];
function atest(name, fn) {
  asyncTests.push({ name, fn });
}

atest("plain draws with penalties over prompt + generated history", async () => {
  const got = await compare("plain", { temperature: 0.8, topK: 40, topP: 0.9, repetitionPenalty: 1.3, repetitionWindow: 64,
    presencePenalty: 0.2, frequencyPenalty: 0.1, seed: 11, maxNewTokens: 40, captureTokenLogProbabilities: true }, {});
  assert.ok(got.draws === got.tokenIds.length + (got.stoppedOnEndToken || got.stoppedOnStopToken ? 1 : 0));
});

atest("GPU-greedy rows take the model's prediction, penalised T=0 rows sample, stop ids end", async () => {
  const tok = makeTokenizer();
  const prompt = [2, 300, 301];
  const first = await session.generate({ promptTokenIds: prompt, model: makeModel(prompt), tokenizer: tok,
    options: { temperature: 0, maxNewTokens: 12 } });
  const stops = first.tokenIds.length > 5 ? [first.tokenIds[5]] : [];
  const got = await compare("greedy", { temperature: 0, maxNewTokens: 12, stopTokenIds: stops }, { prompt });
  assert.strictEqual(got.draws, 0);
  await compare("penalised T=0", { temperature: 0, repetitionPenalty: 1.5, repetitionWindow: 8, maxNewTokens: 20 }, {});
});

atest("end tokens stop the loop before the token is kept", async () => {
  const got = await compare("eos", { temperature: 1.0, seed: 3, maxNewTokens: 50 },
    { bias: (l, pos) => { if (pos === 6) l[50] = 40; } });
  assert.strictEqual(got.stoppedOnEndToken, true);
  assert.strictEqual(got.tokenIds.length, 6);
});

atest("a compiled constraint: legal ids, acceptToken, termination while accepting", async () => {
  const constraint = { type: "regex", pattern: "[a-d ]{2,12}" };
  for (const seed of [1, 2, 3, 4, 5, 6]) {
    await compare("regex seed " + seed, { temperature: 1.0, topP: 0.95, seed, maxNewTokens: 10, constraint },
      { bias: (l, pos) => { if (pos >= 4) l[1] += 6; } });
  }
  // a budget too small: the reference's error
  await compare("regex short", { temperature: 1.0, seed: 9, maxNewTokens: 1, constraint: { type: "regex", pattern: "a{20}" } }, {});
});

atest("thinking: the reasoning channel may open inside a constraint", async () => {
  const constraint = { type: "regex", pattern: "[a-d]{1,6}" };
  await compare("channel", { temperature: 0.9, seed: 21, maxNewTokens: 24, constraint }, {
    thinking: true,
    bias: (l, pos) => { if (pos === 0) l[START] = 30; if (pos === 5) l[END] = 30; if (pos >= 8) l[1] += 5; },
  });
});

atest("required reasoning: forced prefix, text-only channel, END_CHANNEL at 16 and 64", async () => {
  const got = await compare("required", { temperature: 1.0, seed: 5, maxNewTokens: 90, requireReasoning: true,
    captureTokenLogProbabilities: true }, { thinking: true, bias: (l) => { l[END] += 3; } });
  assert.deepStrictEqual(got.tokenIds.slice(0, 3), [START, 200, 201]);
  const forcedEnd = await compare("required cap", { temperature: 1.0, seed: 6, maxNewTokens: 80, requireReasoning: true },
    { thinking: true, bias: (l) => { l[END] = -50; l[1] = -50; l[50] = -50; l[106] = -50; } });
  assert.strictEqual(forcedEnd.tokenIds[3 + 64], END);
  await assert.rejects(session.generate({ promptTokenIds: [2], model: makeModel([2]), tokenizer: makeTokenizer(),
    options: { requireReasoning: true } }), /^Error: Required reasoning needs enableThinking$/);
});

// the harness runs synchronous tests; chain the async ones through it
(async () => {
  for (const t of asyncTests) {
    let err = null;
    try { await t.fn(); } catch (e) { err = e; }
    test(t.name, () => { if (err) throw err; });
  }
  run();
})();
