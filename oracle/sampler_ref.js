"use strict";
/*
 * ORACLE — test infrastructure only (tests/ and bench.py's cpu_baseline leg).
 *
 * JavaScript restatement of the reference sampler, run on Node so that the
 * arithmetic is the JS engine's own (Math.exp, Math.log, the stable
 * Array.prototype.sort, f64 + - * /). It follows
 * src/runtime/sampling.ts:3-16 (SeededRandom) and :18-96 (sampleToken,
 * cumulativeCut, argmax) step by step; the order of operations is kept
 * because the sampled ids must be bit-exact. Written for Node 12 (no `??`).
 */

const MULBERRY_STEP = 0x6d2b79f5;

class SeededRandom {
  constructor(seed) {
    this.state = (seed >>> 0) || MULBERRY_STEP;
  }

  next() {
    this.state += MULBERRY_STEP;
    let z = this.state;
    z = Math.imul(z ^ (z >>> 15), z | 1);
    z ^= z + Math.imul(z ^ (z >>> 7), z | 61);
    return ((z ^ (z >>> 14)) >>> 0) / 4294967296;
  }
}

function keepLeadingMass(list, threshold) {
  let running = 0;
  let kept = 0;
  do {
    running += list[kept].probability;
    kept += 1;
  } while (kept < list.length && running < threshold);
  return list.slice(0, Math.max(1, kept));
}

function firstMaximum(values) {
  let best = 0;
  for (let i = 1; i < values.length; i += 1) {
    if (values[i] > values[best]) best = i;
  }
  return best;
}

/* sampleToken; returns {token, probability} (probability 1 for greedy). */
function sampleWithProbability(rawLogits, history, config, random) {
  if (rawLogits.length === 0) throw new Error("Cannot sample empty logits");
  const values = Array.from(rawLogits);
  const seen = new Map();
  const window = config.repetitionWindow === 0 ? [] : history.slice(-config.repetitionWindow);
  for (let i = 0; i < window.length; i += 1) {
    const id = window[i];
    const prior = seen.get(id);
    seen.set(id, prior === undefined ? 1 : prior + 1);
  }
  seen.forEach((count, id) => {
    if (id < 0 || id >= values.length) return;
    const v = values[id];
    values[id] = v < 0 ? v * config.repetitionPenalty : v / config.repetitionPenalty;
    values[id] -= config.presencePenalty + count * config.frequencyPenalty;
  });
  if (config.temperature === 0) return { token: firstMaximum(values), probability: 1 };

  const ranked = values
    .map((v, id) => ({ token: id, logit: v / config.temperature, probability: 0, surprise: 0 }))
    .sort((a, b) => b.logit - a.logit);
  const top = ranked[0].logit;
  let mass = 0;
  for (let i = 0; i < ranked.length; i += 1) {
    ranked[i].probability = Math.exp(ranked[i].logit - top);
    mass += ranked[i].probability;
  }
  for (let i = 0; i < ranked.length; i += 1) ranked[i].probability /= mass;

  let pool = config.topK > 0 ? ranked.slice(0, config.topK) : ranked;
  if (config.minP > 0) {
    const floor = pool[0].probability * config.minP;
    pool = pool.filter((entry) => entry.probability >= floor);
  }
  if (config.typicalP < 1) {
    let entropy = 0;
    for (let i = 0; i < pool.length; i += 1) entropy = entropy - pool[i].probability * Math.log(pool[i].probability);
    for (let i = 0; i < pool.length; i += 1) pool[i].surprise = Math.abs(-Math.log(pool[i].probability) - entropy);
    pool.sort((a, b) => a.surprise - b.surprise);
    pool = keepLeadingMass(pool, config.typicalP);
    pool.sort((a, b) => b.probability - a.probability);
  }
  if (config.topP < 1) pool = keepLeadingMass(pool, config.topP);

  let poolMass = 0;
  for (let i = 0; i < pool.length; i += 1) poolMass = poolMass + pool[i].probability;
  let cursor = random() * poolMass;
  for (let i = 0; i < pool.length; i += 1) {
    cursor -= pool[i].probability;
    if (cursor <= 0) return { token: pool[i].token, probability: pool[i].probability };
  }
  const last = pool[pool.length - 1];
  return { token: last.token, probability: last.probability };
}

function sampleToken(rawLogits, history, config, random) {
  return sampleWithProbability(rawLogits, history, config, random).token;
}

module.exports = { SeededRandom, sampleToken, sampleWithProbability };
