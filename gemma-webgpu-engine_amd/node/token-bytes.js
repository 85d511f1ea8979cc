"use strict";
/*
 * The Gemma token byte table and its on-disk form.
 *
 * createTokenByteTable (src/runtime/gemma-tokenizer.ts:346-360): vocabulary
 * size = largest id + 1; special ids (the tokenizer's all_special_ids) and
 * ids the vocabulary does not name are null; a byte-fallback piece
 * "<0xHH>" (two upper-case hex digits) is that one byte; any other piece is
 * the UTF-8 of its text with every "▁" (the SentencePiece space) turned
 * into " ".
 *
 * loadTokenizerJson reads a Hugging Face tokenizer.json (the file the
 * reference's tokenizer loads, gemma-tokenizer.ts:14-16): the model's vocab
 * (an object piece -> id, or a Unigram list [piece, score] whose index is the
 * id) plus added_tokens; special ids are the added tokens marked special.
 *
 * The on-disk table ("GSVB" version 1, little-endian):
 *   magic "GSVB", u32 version, u32 V, u32 flags (0), u64 total bytes,
 *   u8 present[V] (1: a byte string, 0: null), u32 offsets[V + 1], bytes.
 * TokenByteTrie and the engine's gs_set_vocab take the same CSR (offsets,
 * bytes); null and empty entries are never legal (token-byte-trie.ts:24-25).
 */
const fs = require("fs");

const EOS_TOKEN_IDS = Object.freeze([1, 50, 106]);          // gemma-tokenizer.ts:17
const GEMMA_START_CHANNEL_TOKEN_ID = 100;                     // :18
const GEMMA_END_CHANNEL_TOKEN_ID = 101;                       // :19
const BYTE_FALLBACK = /^<0x([0-9A-F]{2})>$/;
const MAGIC = 0x42565347;  // "GSVB"

/* vocabulary: Map or object piece -> id; specialIds: iterable of ids */
function createTokenByteTable(vocabulary, specialIds) {
  const entries = vocabulary instanceof Map ? Array.from(vocabulary.entries()) : Object.entries(vocabulary);
  let size = 0;
  for (const [, id] of entries) size = Math.max(size, id + 1);
  const table = new Array(size).fill(null);
  const special = new Set(specialIds);
  const encoder = new TextEncoder();
  for (const [piece, id] of entries) {
    if (special.has(id)) continue;
    const m = BYTE_FALLBACK.exec(piece);
    table[id] = m ? Uint8Array.of(parseInt(m[1], 16)) : encoder.encode(piece.split("▁").join(" "));
  }
  return table;
}

/* { vocabulary: Map piece -> id, specialIds: number[] } of a tokenizer.json */
function readTokenizerJson(path) {
  const json = JSON.parse(fs.readFileSync(path, "utf8"));
  const vocabulary = new Map();
  const vocab = json.model && json.model.vocab;
  if (Array.isArray(vocab)) vocab.forEach((entry, id) => vocabulary.set(entry[0], id));
  else if (vocab && typeof vocab === "object") for (const [piece, id] of Object.entries(vocab)) vocabulary.set(piece, id);
  else throw new Error("tokenizer.json has no model vocab");
  const specialIds = [];
  for (const t of json.added_tokens || []) {
    vocabulary.set(t.content, t.id);
    if (t.special) specialIds.push(t.id);
  }
  return { vocabulary, specialIds };
}

function loadTokenizerJson(path) {
  const { vocabulary, specialIds } = readTokenizerJson(path);
  return createTokenByteTable(vocabulary, specialIds);
}

/* TokenByteSource over a table (token-byte-trie.ts:1-4) */
function tokenByteSource(table) {
  return {
    vocabularySize: table.length,
    tokenBytes(tokenId) {
      if (!Number.isInteger(tokenId) || tokenId < 0 || tokenId >= table.length) return null;
      return table[tokenId];
    },
  };
}

function writeTokenByteTable(path, table) {
  const V = table.length;
  let total = 0;
  for (const b of table) if (b) total += b.length;
  const header = Buffer.alloc(24);
  header.writeUInt32LE(MAGIC, 0);
  header.writeUInt32LE(1, 4);
  header.writeUInt32LE(V, 8);
  header.writeUInt32LE(0, 12);
  header.writeUInt32LE(total % 4294967296, 16);
  header.writeUInt32LE(Math.floor(total / 4294967296), 20);
  const present = Buffer.alloc(V);
  const offsets = Buffer.alloc(4 * (V + 1));
  const bytes = Buffer.alloc(total);
  let at = 0;
  table.forEach((b, id) => {
    present[id] = b ? 1 : 0;
    offsets.writeUInt32LE(at, 4 * id);
    if (b) { bytes.set(b, at); at += b.length; }
  });
  offsets.writeUInt32LE(at, 4 * V);
  fs.writeFileSync(path, Buffer.concat([header, present, offsets, bytes]));
}

function readTokenByteTable(path) {
  const buf = fs.readFileSync(path);
  if (buf.length < 24 || buf.readUInt32LE(0) !== MAGIC) throw new Error("not a GSVB token byte table");
  if (buf.readUInt32LE(4) !== 1) throw new Error("unsupported GSVB version " + buf.readUInt32LE(4));
  const V = buf.readUInt32LE(8);
  const total = buf.readUInt32LE(16) + buf.readUInt32LE(20) * 4294967296;
  const pAt = 24;
  const oAt = pAt + V;
  const bAt = oAt + 4 * (V + 1);
  if (buf.length !== bAt + total) throw new Error("GSVB size does not match its header");
  const table = new Array(V);
  for (let id = 0; id < V; id += 1) {
    const a = buf.readUInt32LE(oAt + 4 * id);
    const b = buf.readUInt32LE(oAt + 4 * id + 4);
    table[id] = buf[pAt + id] ? Uint8Array.from(buf.subarray(bAt + a, bAt + b)) : null;
  }
  return table;
}

module.exports = {
  EOS_TOKEN_IDS,
  GEMMA_START_CHANNEL_TOKEN_ID,
  GEMMA_END_CHANNEL_TOKEN_ID,
  createTokenByteTable,
  readTokenizerJson,
  loadTokenizerJson,
  tokenByteSource,
  writeTokenByteTable,
  readTokenByteTable,
};
