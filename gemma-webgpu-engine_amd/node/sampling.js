"use strict";
/*
 * The reference's sampling entry points (src/runtime/sampling.ts) with the
 * same names, arguments, results and errors, computed by the HIP kernels:
 *   SeededRandom(seed).next()            sampling.ts:3-16
 *   sampleToken(rawLogits, history, config, random)   sampling.ts:18-65
 *   tokenLogProbability(rawLogits, token)             sampling.ts:67-80
 * One engine per vocabulary size (rows of one) serves these single-row calls;
 * Engine.sampleRows is the batched form.
 */
const { native } = require("./native");
const { Engine } = require("./engine");

const MULBERRY_INCREMENT = 0x6d2b79f5;

const singleRowEngines = new Map();

function engineFor(vocabSize) {
  let e = singleRowEngines.get(vocabSize);
  if (!e) {
    const device = process.env.GSAMPLE_DEVICE ? Number(process.env.GSAMPLE_DEVICE) : 0;
    e = new Engine({ vocabSize, maxRows: 1, device });
    singleRowEngines.set(vocabSize, e);
  }
  return e;
}

/* Releases the engines the single-row functions created. */
function releaseEngines() {
  singleRowEngines.forEach((e) => e.destroy());
  singleRowEngines.clear();
}

/* Mulberry32 as a counter: draw n of SeededRandom(seed) is evaluated in
 * closed form by the library (the same code the kernels run). */
class SeededRandom {
  constructor(seed) {
    this.seed = seed >>> 0 || MULBERRY_INCREMENT;
    this.draws = 0;
  }

  next() {
    const value = native().seededRandom(this.seed, this.draws);
    this.draws += 1;
    return value;
  }
}

/* The logits as float32, the element type the kernels read: a Float32Array
 * (the reference's per-token readback copy, src/webgpu/decode-model.ts:185)
 * passes as is; other array-likes are rounded to float32 element by element. */
function asFloat32(rawLogits) {
  return rawLogits instanceof Float32Array ? rawLogits : Float32Array.from(rawLogits);
}

function sampleTokenWithProbability(rawLogits, history, config, random) {
  if (rawLogits.length === 0) throw new Error("Cannot sample empty logits");
  const logits = asFloat32(rawLogits);
  const engine = engineFor(logits.length);
  // one draw per non-greedy call, as sampling.ts:31,59
  const uniform = config.temperature === 0 ? 0 : random();
  const row = Object.assign({}, config, { uniform });
  const r = engine.sampleRows({ logits, rows: 1, configs: [row], histories: [history || []] });
  return { token: r.tokens[0], probability: r.probabilities[0], flags: r.flags[0] };
}

function sampleToken(rawLogits, history, config, random) {
  return sampleTokenWithProbability(rawLogits, history, config, random).token;
}

function tokenLogProbability(rawLogits, token) {
  if (!Number.isInteger(token) || token < 0 || token >= rawLogits.length) {
    throw new Error("Token " + token + " is outside logits length " + rawLogits.length);
  }
  const logits = asFloat32(rawLogits);
  return engineFor(logits.length).tokenLogProbabilities(logits, 1, [token])[0];
}

module.exports = {
  SeededRandom,
  sampleToken,
  sampleTokenWithProbability,
  tokenLogProbability,
  engineFor,
  releaseEngines,
};
