"use strict";
/*
 * Loads the N-API addon (lib/gsample_node.node, built by
 * `make -C gemma-webgpu-engine_amd/csrc`). There is no fallback: a missing
 * addon or library is an error, never a silent CPU path.
 */
const path = require("path");

const ADDON_PATH = path.join(__dirname, "..", "lib", "gsample_node.node");
let addon = null;

function native() {
  if (addon) return addon;
  try {
    addon = require(ADDON_PATH);
  } catch (error) {
    const e = new Error(
      "gsample native addon could not be loaded from " + ADDON_PATH +
      " (build it with `make -C gemma-webgpu-engine_amd/csrc`): " + error.message);
    e.code = "GS_ADDON_MISSING";
    throw e;
  }
  return addon;
}

module.exports = { native, ADDON_PATH };
