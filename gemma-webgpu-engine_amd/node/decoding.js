"use strict";
/*
 * DecodingConfig defaults and validation: the option surface of
 * src/runtime/decoding.ts:1-59 (same field names, defaults, check order and
 * messages).
 */

const DEFAULT_DECODING_CONFIG = {
  temperature: 0.8,
  topK: 40,
  topP: 0.95,
  minP: 0,
  typicalP: 1,
  repetitionPenalty: 1.05,
  repetitionWindow: 64,
  frequencyPenalty: 0,
  presencePenalty: 0,
  maxNewTokens: 256,
  seed: 42,
  stopTokenIds: [],
};

function finiteNumber(x) {
  return typeof x === "number" && Number.isFinite(x);
}

/* validateDecodingConfig (src/runtime/decoding.ts:31-59): the input is laid
 * over the defaults, every failed check adds its message, in this order. */
function validateDecodingConfig(input) {
  const v = Object.assign({}, DEFAULT_DECODING_CONFIG, input);
  const errors = [];
  if (!finiteNumber(v.temperature) || v.temperature < 0) errors.push("temperature must be >= 0");
  if (!Number.isInteger(v.topK) || v.topK < 0) errors.push("topK must be a non-negative integer");
  ["topP", "minP", "typicalP"].forEach((key) => {
    const x = v[key];
    if (!finiteNumber(x) || x < 0 || x > 1) errors.push(key + " must be between 0 and 1");
  });
  if (!finiteNumber(v.repetitionPenalty) || v.repetitionPenalty <= 0) errors.push("repetitionPenalty must be > 0");
  if (!Number.isInteger(v.repetitionWindow) || v.repetitionWindow < 0) {
    errors.push("repetitionWindow must be a non-negative integer");
  }
  if (!finiteNumber(v.frequencyPenalty) || v.frequencyPenalty < 0) {
    errors.push("frequencyPenalty must be finite and non-negative");
  }
  if (!finiteNumber(v.presencePenalty) || v.presencePenalty < 0) {
    errors.push("presencePenalty must be finite and non-negative");
  }
  if (!Number.isInteger(v.maxNewTokens) || v.maxNewTokens < 1) errors.push("maxNewTokens must be a positive integer");
  if (!Number.isInteger(v.seed)) errors.push("seed must be an integer");
  const stops = v.stopTokenIds;
  if (!Array.isArray(stops) || stops.some((id) => !Number.isInteger(id) || id < 0)) {
    errors.push("stopTokenIds must contain non-negative integers");
  }
  return { ok: errors.length === 0, errors };
}

module.exports = { DEFAULT_DECODING_CONFIG, validateDecodingConfig };
