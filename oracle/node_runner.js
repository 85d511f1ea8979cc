"use strict";
/*
 * ORACLE runner — test infrastructure only. Runs the JavaScript restatement
 * of the reference sampler (sampler_ref.js) over rows of a logits file, on
 * one Node thread, and reports ids, probabilities and wall time.
 *
 * usage: node node_runner.js spec.json
 * spec: {
 *   logits: path to raw little-endian rows (f32 or bf16), dtype: "f32"|"bf16",
 *   rows: R, vocab: V, pick: [row indices to run] (default all),
 *   configs: [DecodingConfig per picked row] | DecodingConfig,
 *   history_offsets: path (int64, R+1) | null, history_ids: path (int32) | null,
 *   seeds: [per picked row] (SeededRandom(seed), first draw) | null,
 *   uniforms: [per picked row] (random() returns this) | null,
 *   warmup: rows to run untimed first (default 0),
 *   out: path for the JSON result
 * }
 */
const fs = require("fs");
const os = require("os");
const { SeededRandom, sampleWithProbability } = require("./sampler_ref.js");

function readTyped(path, Ctor) {
  const b = fs.readFileSync(path);
  const copy = new Uint8Array(b.length);
  copy.set(b);
  return new Ctor(copy.buffer, 0, b.length / Ctor.BYTES_PER_ELEMENT);
}

function rowView(spec, all, r) {
  const V = spec.vocab;
  if (spec.dtype === "bf16") {
    const out = new Float32Array(V);
    const bits = new Uint32Array(out.buffer);
    for (let i = 0; i < V; i += 1) bits[i] = all[r * V + i] << 16;
    return out;
  }
  return all.subarray(r * V, (r + 1) * V);
}

function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const all = spec.dtype === "bf16" ? readTyped(spec.logits, Uint16Array) : readTyped(spec.logits, Float32Array);
  let offsets = null;
  let ids = null;
  if (spec.history_offsets) {
    const o = readTyped(spec.history_offsets, Float64Array);
    offsets = o;
    ids = readTyped(spec.history_ids, Int32Array);
  }
  const pick = spec.pick || Array.from({ length: spec.rows }, (_, i) => i);
  const results = [];
  const warmup = spec.warmup || 0;
  const runRow = (k) => {
    const r = pick[k];
    const logits = rowView(spec, all, r);
    const config = Array.isArray(spec.configs) ? spec.configs[k] : spec.configs;
    let history = [];
    if (offsets) history = Array.from(ids.subarray(offsets[r], offsets[r + 1]));
    let random;
    if (spec.uniforms) {
      const u = spec.uniforms[k];
      random = () => u;
    } else {
      const gen = new SeededRandom(spec.seeds[k]);
      random = () => gen.next();
    }
    return sampleWithProbability(logits, history, config, random);
  };
  for (let k = 0; k < Math.min(warmup, pick.length); k += 1) runRow(k);
  const t0 = process.hrtime.bigint();
  for (let k = 0; k < pick.length; k += 1) results.push(runRow(k));
  const t1 = process.hrtime.bigint();
  const seconds = Number(t1 - t0) / 1e9;
  const cpus = os.cpus();
  fs.writeFileSync(spec.out, JSON.stringify({
    tokens: results.map((x) => x.token),
    probabilities: results.map((x) => x.probability),
    seconds,
    rows: pick.length,
    node: process.version,
    cpu_model: cpus.length ? cpus[0].model : "unknown",
    host_cpus: cpus.length,
  }));
}

main();
