"use strict";
/*
 * TokenByteTrie (src/runtime/token-byte-trie.ts:1-41) in the form the GPU
 * masker reads: the token byte strings as a CSR (offsets Int32Array[V+1],
 * bytes Uint8Array). Tokens whose bytes are null or empty get an empty range
 * and are never legal, as the trie skips them (token-byte-trie.ts:24-25);
 * tokenCount counts the others. Duplicate strings need no shared node: each
 * token walks its own bytes in the mask kernel.
 */
class TokenByteTrie {
  constructor(source) {
    const V = source.vocabularySize;
    const offsets = new Int32Array(V + 1);
    const pieces = new Array(V);
    let total = 0;
    let tokenCount = 0;
    for (let id = 0; id < V; id += 1) {
      const bytes = source.tokenBytes(id);
      const n = bytes && bytes.length ? bytes.length : 0;
      pieces[id] = n ? bytes : null;
      if (n) tokenCount += 1;
      total += n;
      if (total > 2147483647) throw new RangeError("token bytes exceed 2^31 bytes");
      offsets[id + 1] = total;
    }
    const all = new Uint8Array(Math.max(1, total));
    for (let id = 0; id < V; id += 1) if (pieces[id]) all.set(pieces[id], offsets[id]);
    this.vocabularySize = V;
    this.offsets = offsets;
    this.bytes = total ? all : new Uint8Array(0);
    this.tokenCount = tokenCount;
  }

  /* TokenByteSource view of the table. */
  tokenBytes(tokenId) {
    if (!Number.isInteger(tokenId) || tokenId < 0 || tokenId >= this.vocabularySize) return null;
    const a = this.offsets[tokenId];
    const b = this.offsets[tokenId + 1];
    return a === b ? null : this.bytes.subarray(a, b);
  }
}

module.exports = { TokenByteTrie };
