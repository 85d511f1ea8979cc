"use strict";
/*
 * gsample for Node: the reference's sampling-stage API (sampling.ts,
 * decoding.ts, generation-config.ts, constraints.ts, token-byte-trie.ts)
 * over the libgsample N-API addon, plus the batched Engine.
 */
const decoding = require("./decoding");
const generationConfig = require("./generation-config");
const sampling = require("./sampling");
const constraints = require("./constraints");
const trie = require("./token-byte-trie");
const tokenBytes = require("./token-bytes");
const engine = require("./engine");
const session = require("./session");
const { native, ADDON_PATH } = require("./native");

module.exports = Object.assign({}, decoding, generationConfig, sampling, constraints, trie, tokenBytes, engine, { generate: session.generate, session,
  native,
  ADDON_PATH,
});
