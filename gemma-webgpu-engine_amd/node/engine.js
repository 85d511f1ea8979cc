"use strict";
/*
 * Engine: one libgsample context (one GPU, one vocab size, a largest batch)
 * and the batched calls over it. Every computation runs in the library's HIP
 * kernels; this file only packs arguments.
 *
 * The per-row options are DecodingConfig's sampling fields
 * (src/runtime/decoding.ts:1-14) plus what the session supplies around
 * sampleToken (src/runtime/gemma-session.ts:659-777, 1305-1329): the draw
 * (SeededRandom(seed) draw number drawIndex, or an explicit uniform value),
 * the Gemma final-logit softcap, the constraint mask slot, whether the
 * constraint is accepting, and the termination / extra-legal ids.
 */
const { native } = require("./native");
const { DEFAULT_DECODING_CONFIG, validateDecodingConfig } = require("./decoding");

const GS_F32 = 0;
const GS_BF16 = 1;
const GS_RNG_SEEDED = 0;
const GS_RNG_EXPLICIT = 1;
const GS_ROW_FORCE_EXACT = 1;
const GS_FORCED_TERMINATION = 1;
const GS_FORCED_EXTRA = 2;

const FLAGS = Object.freeze({
  TOPP_TIE: 1,
  EXACT_PATH: 2,
  NEAR_TIE: 4,
  DEAD_END: 8,
  NONFINITE: 16,
  EMPTY_CANDIDATES: 32,
  GREEDY: 64,
  UNSUPPORTED: 128,
  INVALID_SLOT: 256,
  INDEX_CHECK: 512,
});

const STAGES = Object.freeze(["lmhead", "scan", "finish", "exact", "deep"]);

let layoutCache = null;
function layouts() {
  if (!layoutCache) layoutCache = native().layouts();
  return layoutCache;
}

/* An id as the kernels see it: integers in int32 range pass, anything else
 * becomes -1, which every consumer skips (the reference skips ids outside
 * [0, V): sampling.ts:27, constraints.ts:166,169). */
function idOrSkip(id) {
  return Number.isInteger(id) && id >= -2147483648 && id <= 2147483647 ? id : -1;
}

function dtypeCode(dtype) {
  if (dtype === undefined || dtype === "f32") return GS_F32;
  if (dtype === "bf16") return GS_BF16;
  throw new TypeError("dtype must be \"f32\" or \"bf16\"");
}

class DeviceBuffer {
  constructor(engine, bytes) {
    this.engine = engine;
    this.bytes = bytes;
    this.handle = native().deviceAlloc(engine.context(), bytes);
  }

  write(typedArray, byteOffset) {
    const off = byteOffset || 0;
    if (off < 0 || off + typedArray.byteLength > this.bytes) throw new RangeError("write past the end of the buffer");
    native().copyToDevice(this.engine.context(), this.handle, off, typedArray);
    return this;
  }

  read(typedArray, byteOffset) {
    const off = byteOffset || 0;
    if (off < 0 || off + typedArray.byteLength > this.bytes) throw new RangeError("read past the end of the buffer");
    native().copyToHost(this.engine.context(), typedArray, this.handle, off);
    return typedArray;
  }

  free() {
    if (this.handle) native().deviceFree(this.engine.context(), this.handle);
    this.handle = null;
  }
}

class Engine {
  /* options: { vocabSize, maxRows = 1, device = 0 } */
  constructor(options) {
    const o = options || {};
    if (!Number.isInteger(o.vocabSize) || o.vocabSize <= 0) throw new RangeError("vocabSize must be a positive integer");
    this.vocabSize = o.vocabSize;
    this.maxRows = o.maxRows === undefined ? 1 : o.maxRows;
    this.device = o.device === undefined ? 0 : o.device;
    this.ctx = native().create(this.device, this.vocabSize, this.maxRows);
    this.loadedVocab = null;
    this.loadedDfa = null;
  }

  context() {
    if (!this.ctx) throw new Error("engine has been destroyed");
    return this.ctx;
  }

  destroy() {
    if (this.ctx) native().destroy(this.ctx);
    this.ctx = null;
  }

  allocate(bytes) {
    return new DeviceBuffer(this, bytes);
  }

  /* Packs per-row options into gs_row_config records. */
  packConfigs(configs) {
    const L = layouts().rowConfig;
    const buf = new Uint8Array(L.size * configs.length);
    const dv = new DataView(buf.buffer);
    configs.forEach((given, r) => {
      const c = Object.assign({}, DEFAULT_DECODING_CONFIG, given);
      const check = validateDecodingConfig(c);
      if (!check.ok) throw new Error("Invalid Gemma decoding config: " + check.errors.join("; "));
      const b = r * L.size;
      dv.setFloat64(b + L.temperature, c.temperature, true);
      dv.setFloat64(b + L.top_p, c.topP, true);
      dv.setFloat64(b + L.min_p, c.minP, true);
      dv.setFloat64(b + L.typical_p, c.typicalP, true);
      dv.setFloat64(b + L.repetition_penalty, c.repetitionPenalty, true);
      dv.setFloat64(b + L.frequency_penalty, c.frequencyPenalty, true);
      dv.setFloat64(b + L.presence_penalty, c.presencePenalty, true);
      dv.setFloat64(b + L.softcap, c.softcap || 0, true);
      const explicit = typeof c.uniform === "number";
      dv.setFloat64(b + L.uniform, explicit ? c.uniform : 0, true);
      dv.setBigInt64(b + L.seed, BigInt(c.seed === undefined ? 42 : c.seed), true);
      dv.setBigUint64(b + L.draw_index, BigInt(c.drawIndex || 0), true);
      dv.setInt32(b + L.top_k, Math.min(c.topK, this.vocabSize), true);
      dv.setInt32(b + L.repetition_window, Math.min(c.repetitionWindow, 2147483647), true);
      dv.setInt32(b + L.rng_mode, explicit ? GS_RNG_EXPLICIT : GS_RNG_SEEDED, true);
      dv.setInt32(b + L.mask_slot, c.maskSlot === undefined ? -1 : c.maskSlot, true);
      dv.setInt32(b + L.accepting, c.accepting ? 1 : 0, true);
      dv.setInt32(b + L.options, c.forceExact ? GS_ROW_FORCE_EXACT : 0, true);
    });
    return buf;
  }

  /* History CSR holding each row's last repetitionWindow ids (the only ids
   * the penalties read, sampling.ts:22-24). */
  packHistories(histories, configs) {
    if (!histories) return [null, null];
    const rows = configs.length;
    const offsets = new Int32Array(rows + 1);
    const parts = [];
    for (let r = 0; r < rows; r += 1) {
      const h = histories[r] || [];
      const w = configs[r].repetitionWindow === undefined
        ? DEFAULT_DECODING_CONFIG.repetitionWindow : configs[r].repetitionWindow;
      const start = w === 0 ? h.length : Math.max(0, h.length - w);
      parts.push([h, start]);
      offsets[r + 1] = offsets[r] + (h.length - start);
    }
    const ids = new Int32Array(Math.max(1, offsets[rows]));
    for (let r = 0; r < rows; r += 1) {
      const h = parts[r][0];
      let k = offsets[r];
      for (let i = parts[r][1]; i < h.length; i += 1) ids[k++] = idOrSkip(h[i]);
    }
    return [offsets, ids];
  }

  /* Termination ids (legal only while the constraint accepts) and extra legal
   * ids, as selectConstrainedToken forms them (gemma-session.ts:1315-1323):
   * an id in both lists is a termination id. */
  packForced(forced, rows) {
    if (!forced) return [null, null, null];
    const offsets = new Int32Array(rows + 1);
    const ids = [];
    const kinds = [];
    for (let r = 0; r < rows; r += 1) {
      const f = forced[r] || {};
      const term = new Set((f.termination || []).map(idOrSkip));
      term.forEach((id) => { ids.push(id); kinds.push(GS_FORCED_TERMINATION); });
      new Set((f.extra || []).map(idOrSkip)).forEach((id) => {
        if (!term.has(id)) { ids.push(id); kinds.push(GS_FORCED_EXTRA); }
      });
      offsets[r + 1] = ids.length;
    }
    return [offsets, Int32Array.from(ids.length ? ids : [0]), Uint8Array.from(kinds.length ? kinds : [0])];
  }

  /*
   * Samples `rows` rows in one batched launch sequence.
   * request: {
   *   logits: Float32Array | Uint16Array (bf16 bits) on the host, or a DeviceBuffer,
   *   dtype: "f32" | "bf16", rows, rowStride (default vocabSize),
   *   configs: per-row options (DecodingConfig fields + seed, drawIndex | uniform,
   *            softcap, maskSlot, accepting, forceExact),
   *   histories: per-row token ids (prompt + generated) or null,
   *   forced: per-row { termination: ids, extra: ids } or null,
   *   maskTable: DeviceBuffer from buildMasks, maskSlots
   * }
   * Returns { tokens: Int32Array, probabilities: Float64Array, flags: Uint32Array };
   * a failing row throws its reference error.
   */
  sampleRows(request) {
    const rows = request.rows === undefined ? 1 : request.rows;
    const configs = request.configs;
    if (!Array.isArray(configs) || configs.length !== rows) throw new RangeError("one config per row is required");
    const stride = request.rowStride === undefined ? this.vocabSize : request.rowStride;
    const packed = this.packConfigs(configs);
    const [hoff, hids] = this.packHistories(request.histories, configs);
    const [foff, fids, fkinds] = this.packForced(request.forced, rows);
    const R = layouts().rowResult;
    const results = new Uint8Array(R.size * rows);
    if (!Number.isInteger(rows) || rows < 0 || rows > this.maxRows) throw new RangeError("rows must be 0..maxRows");
    if (!Number.isInteger(stride) || stride < this.vocabSize) throw new RangeError("rowStride must be >= vocabSize");
    const esize = dtypeCode(request.dtype) === GS_BF16 ? 2 : 4;
    if (request.logits instanceof DeviceBuffer) {
      const need = rows > 0 ? ((rows - 1) * stride + this.vocabSize) * esize : 0;
      if (request.logits.bytes < need) throw new RangeError("logits buffer holds fewer than rows x rowStride elements");
    } else if (!request.logits || request.logits.length < rows * stride) {
      throw new RangeError("logits array holds fewer than rows x rowStride elements");
    }
    const maskSlots = request.maskSlots || 0;
    if (request.maskTable && request.maskTable.bytes < maskSlots * 4 * Math.ceil(this.vocabSize / 32)) {
      throw new RangeError("maskTable holds fewer than maskSlots masks");
    }
    const logits = request.logits instanceof DeviceBuffer ? request.logits.handle : request.logits;
    const table = request.maskTable ? request.maskTable.handle : null;
    native().sampleHost(this.context(), logits, dtypeCode(request.dtype), rows, stride, packed, hoff, hids,
      foff, fids, fkinds, table, maskSlots, results);
    const dv = new DataView(results.buffer);
    const out = {
      tokens: new Int32Array(rows),
      probabilities: new Float64Array(rows),
      flags: new Uint32Array(rows),
    };
    for (let r = 0; r < rows; r += 1) {
      out.tokens[r] = dv.getInt32(r * R.size + R.token, true);
      out.flags[r] = dv.getUint32(r * R.size + R.flags, true);
      out.probabilities[r] = dv.getFloat64(r * R.size + R.probability, true);
    }
    return out;
  }

  /* tokenLogProbability per row over host f32 rows [rows][vocabSize]. */
  tokenLogProbabilities(logits, rows, tokens) {
    return native().tokenLogProbHost(this.context(), logits, rows, Int32Array.from(tokens, idOrSkip));
  }

  /* maskConstraintLogits on the device. */
  maskLogits(rawLogits, legalTokenIds, terminationTokenIds) {
    return native().maskLogitsHost(this.context(), rawLogits, Int32Array.from(legalTokenIds, idOrSkip),
      Int32Array.from(terminationTokenIds, idOrSkip));
  }

  /* Constraint tables: a TokenByteTrie (its CSR) and a ByteLevelDfa; loaded
   * once and reloaded only when a different object is passed. */
  useVocab(trie) {
    if (this.loadedVocab === trie) return;
    if (trie.vocabularySize !== this.vocabSize) throw new RangeError("trie vocabulary size differs from the engine's");
    native().setVocab(this.context(), trie.offsets, trie.bytes);
    this.loadedVocab = trie;
  }

  useDfa(dfa) {
    if (this.loadedDfa === dfa) return;
    native().setDfa(this.context(), dfa.stateCount, dfa.next, dfa.finals);
    this.loadedDfa = dfa;
  }

  /* Legal-token bitmasks of `states` into a DeviceBuffer (one row of
   * ceil(V/32) words per state); the table rows are the rows' maskSlot. */
  buildMasks(states, table) {
    const words = Math.ceil(this.vocabSize / 32);
    const out = table || this.allocate(4 * words * states.length);
    if (out.bytes < 4 * words * states.length) throw new RangeError("mask table is smaller than states x ceil(V/32) words");
    native().buildMasks(this.context(), Int32Array.from(states), out.handle);
    return out;
  }

  legalTokenIds(state) {
    return native().legalTokenIds(this.context(), state);
  }

  dfaAdvance(states, tokens) {
    return native().dfaAdvance(this.context(), Int32Array.from(states), Int32Array.from(tokens));
  }

  dfaAdvanceBytes(state, bytes) {
    return native().dfaAdvanceBytes(this.context(), state, bytes);
  }

  dfaAccepting(state) {
    return native().dfaAccepting(this.context(), state);
  }

  /* logits[m][v] = softcap * tanh(hidden[m] . weight[v] / softcap) with bf16
   * hidden [mRows][width] and weight [vocabSize][width] DeviceBuffers. */
  lmhead(hidden, weight, mRows, width, softcap, logits) {
    if (!Number.isInteger(mRows) || mRows <= 0 || !Number.isInteger(width) || width <= 0) {
      throw new RangeError("mRows and width must be positive integers");
    }
    if (hidden.bytes < 2 * mRows * width || weight.bytes < 2 * this.vocabSize * width ||
        logits.bytes < 4 * mRows * this.vocabSize) {
      throw new RangeError("lm_head buffers are smaller than [mRows][width], [vocabSize][width] and [mRows][vocabSize]");
    }
    native().lmhead(this.context(), hidden.handle, weight.handle, mRows, width, softcap, logits.handle);
    return logits;
  }

  /* The int2 QAT head (the reference's producer, cpuQatLinear bit for bit):
   * logits[m][v] = srq(rowScales[v] * sum_k (code[v][k] - 2) * srq(x[m][k], inputScale), outputScale).
   * x: f32 [mRows][width], codes: 2-bit codes as u32 words, layout "row-major" ([vocabSize][width/16],
   * the checkpoint's) or "block-major" ([width/64][vocabSize][4]), rowScales: f32 [vocabSize]; all
   * DeviceBuffers. */
  qatLmhead(x, mRows, width, codes, layout, rowScales, inputScale, outputScale, logits) {
    if (!Number.isInteger(mRows) || mRows <= 0 || !Number.isInteger(width) || width <= 0) {
      throw new RangeError("mRows and width must be positive integers");
    }
    if (x.bytes < 4 * mRows * width || codes.bytes < this.vocabSize * width / 4 || rowScales.bytes < 4 * this.vocabSize ||
        logits.bytes < 4 * mRows * this.vocabSize) {
      throw new RangeError("QAT head buffers are smaller than [mRows][width] f32, vocabSize x width 2-bit codes, " +
        "[vocabSize] f32 and [mRows][vocabSize] f32");
    }
    const code = layout === "block-major" ? 1 : layout === "row-major" || layout === undefined ? 0 : -1;
    if (code < 0) throw new RangeError("layout must be \"row-major\" or \"block-major\"");
    native().qatLmhead(this.context(), x.handle, mRows, width, codes.handle, code, rowScales.handle,
      inputScale || 0, outputScale || 0, logits.handle);
    return logits;
  }

  /* the QAT head into `scratch` (f32 [rows][vocabSize]), then sampleRows on it. */
  qatLmheadSample(x, width, codes, layout, rowScales, inputScale, outputScale, scratch, request) {
    this.qatLmhead(x, request.rows, width, codes, layout, rowScales, inputScale, outputScale, scratch);
    return this.sampleRows(Object.assign({}, request, { logits: scratch, dtype: "f32", rowStride: this.vocabSize }));
  }

  /* lm_head into `scratch` (f32 [rows][vocabSize]), then sampleRows on it. */
  lmheadSample(hidden, weight, width, softcap, scratch, request) {
    this.lmhead(hidden, weight, request.rows, width, softcap, scratch);
    return this.sampleRows(Object.assign({}, request, { logits: scratch, dtype: "f32", rowStride: this.vocabSize }));
  }

  timingBegin(maxCalls) {
    native().timingBegin(this.context(), maxCalls);
  }

  /* { lmhead: [ms, calls], scan: [...], finish: [...], exact: [...] } */
  timingEnd() {
    const t = native().timingEnd(this.context());
    const out = {};
    STAGES.forEach((name, k) => { out[name] = [t.stageMs[k], t.calls[k]]; });
    return out;
  }
}

module.exports = {
  Engine,
  DeviceBuffer,
  FLAGS,
  STAGES,
  GS_FORCED_TERMINATION,
  GS_FORCED_EXTRA,
  idOrSkip,
};
