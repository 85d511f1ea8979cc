"use strict";
/*
 * generate() option resolution: src/runtime/generation-config.ts:47-77
 * (greedy defaults with penalties off, validation with the joined message,
 * the stop-id bound, and the GPU-greedy routing predicate).
 */
const { DEFAULT_DECODING_CONFIG, validateDecodingConfig } = require("./decoding");

const VOCAB_SIZE = 262144;
const DEFAULT_MAX_NEW_TOKENS = 256;

const DEFAULT_GENERATION_CONFIG = Object.assign({}, DEFAULT_DECODING_CONFIG, {
  temperature: 0,
  topK: 0,
  topP: 1,
  minP: 0,
  typicalP: 1,
  repetitionPenalty: 1,
  repetitionWindow: 0,
  frequencyPenalty: 0,
  presencePenalty: 0,
  maxNewTokens: DEFAULT_MAX_NEW_TOKENS,
  stopTokenIds: [],
});

/* resolveGemmaGenerationConfig (generation-config.ts:62-70). */
function resolveGemmaGenerationConfig(options) {
  const config = Object.assign({}, DEFAULT_GENERATION_CONFIG, options);
  const result = validateDecodingConfig(config);
  if (!result.ok) throw new Error("Invalid Gemma decoding config: " + result.errors.join("; "));
  if (config.stopTokenIds.some((id) => id >= VOCAB_SIZE)) {
    throw new Error("Gemma stop token IDs must be below " + VOCAB_SIZE);
  }
  return Object.assign({}, config, { stopTokenIds: config.stopTokenIds.slice() });
}

/* usesGemmaGpuGreedy (generation-config.ts:72-77). */
function usesGemmaGpuGreedy(config) {
  return config.temperature === 0 &&
    config.repetitionPenalty === 1 &&
    config.frequencyPenalty === 0 &&
    config.presencePenalty === 0;
}

module.exports = {
  VOCAB_SIZE,
  DEFAULT_GENERATION_CONFIG,
  resolveGemmaGenerationConfig,
  usesGemmaGpuGreedy,
};
