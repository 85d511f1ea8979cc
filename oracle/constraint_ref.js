"use strict";
/*
 * ORACLE — test infrastructure only (tests/ and bench.py's cpu_baseline leg).
 *
 * JavaScript restatement of the reference's constraint masking for a
 * byte-level DFA, run on Node beside sampler_ref.js:
 *   viableStates      src/runtime/constraints.ts:300-322 (findViableStates):
 *                     states from which a final state is reachable
 *   legalTokenIds     src/runtime/constraints.ts:56-92: a token is legal iff
 *                     every state reached along its bytes exists and is
 *                     viable; ids ascending; cached per state as the
 *                     reference caches them (:62-69)
 *   maskConstraintLogits  src/runtime/constraints.ts:159-173: a fresh
 *                     Float32Array of -Infinity with the legal and
 *                     termination ids' raw logits copied in
 * The reference walks a token-byte trie; walking each token's bytes gives the
 * same set (the trie only shares prefixes), which the GPU tests check
 * against the mask kernel on every state.
 */

function viableStates(next, finals, nStates) {
  const preds = Array.from({ length: nStates }, () => []);
  for (let s = 0; s < nStates; s += 1) {
    for (let c = 0; c < 256; c += 1) {
      const t = next[s * 256 + c];
      if (t >= 0) preds[t].push(s);
    }
  }
  const viable = new Uint8Array(nStates);
  const stack = [];
  for (let s = 0; s < nStates; s += 1) if (finals[s]) { viable[s] = 1; stack.push(s); }
  while (stack.length) {
    const t = stack.pop();
    for (const p of preds[t]) if (!viable[p]) { viable[p] = 1; stack.push(p); }
  }
  return viable;
}

class ByteDfaMasker {
  /* next: Int32Array[nStates * 256] (-1: no edge), finals: Uint8Array[nStates],
   * offsets: token byte offsets [V + 1], bytes: Uint8Array */
  constructor(next, finals, nStates, offsets, bytes) {
    this.next = next;
    this.nStates = nStates;
    this.viable = viableStates(next, finals, nStates);
    this.offsets = offsets;
    this.bytes = bytes;
    this.cache = new Map();
  }

  legalTokenIds(state) {
    const hit = this.cache.get(state);
    if (hit) return hit;
    const ids = [];
    const V = this.offsets.length - 1;
    for (let t = 0; t < V; t += 1) {
      const b0 = this.offsets[t];
      const b1 = this.offsets[t + 1];
      if (b1 === b0) continue;  // tokens without bytes are never legal
      let s = state;
      let ok = true;
      for (let k = b0; k < b1; k += 1) {
        s = this.next[s * 256 + this.bytes[k]];
        if (s < 0 || !this.viable[s]) { ok = false; break; }
      }
      if (ok) ids.push(t);
    }
    const frozen = Object.freeze(ids);
    this.cache.set(state, frozen);
    return frozen;
  }
}

function maskConstraintLogits(rawLogits, legalTokenIds, terminationTokenIds) {
  const masked = new Float32Array(rawLogits.length).fill(-Infinity);
  for (const id of legalTokenIds) {
    if (id >= 0 && id < rawLogits.length) masked[id] = rawLogits[id];
  }
  for (const id of terminationTokenIds) {
    if (id >= 0 && id < rawLogits.length) masked[id] = rawLogits[id];
  }
  return masked;
}

module.exports = { viableStates, ByteDfaMasker, maskConstraintLogits };
