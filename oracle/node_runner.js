"use strict";
/*
 * ORACLE runner — test infrastructure only. Runs the JavaScript restatement
 * of the reference sampler (sampler_ref.js), and for constrained rows the
 * masking restatement (constraint_ref.js), over rows of a logits file, and
 * reports ids, probabilities and wall time.
 *
 * usage: node node_runner.js spec.json
 * spec: {
 *   logits: path to raw little-endian rows (f32 or bf16), dtype: "f32"|"bf16",
 *   rows: R, vocab: V, pick: [row indices to run] (default all),
 *   configs: [DecodingConfig per picked row] | DecodingConfig,
 *   history_offsets: path (f64, R+1) | null, history_ids: path (int32) | null,
 *   seeds: [per picked row] (SeededRandom(seed), first draw) | null,
 *   uniforms: [per picked row] (random() returns this) | null,
 *   constraint: { next: path (int32 S*256), finals: path (u8 S), states: S,
 *                 vocab_offsets: path (f64 V+1), vocab_bytes: path (u8),
 *                 row_states: [DFA state per picked row], termination: [ids] } | null,
 *   warmup: rows to run untimed first (default 0),
 *   threads: worker threads the picked rows are split over (default 1: the
 *            main thread alone, as the reference runs),
 *   out: path for the JSON result
 * }
 * The timed region starts once every thread has loaded its inputs and run
 * its warm-up rows, and ends when the last thread has sampled its rows.
 */
const fs = require("fs");
const os = require("os");
const { SeededRandom, sampleWithProbability } = require("./sampler_ref.js");
const { ByteDfaMasker, maskConstraintLogits } = require("./constraint_ref.js");

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

/* The logits file in a SharedArrayBuffer, which worker threads read in place. */
function readShared(path) {
  const b = fs.readFileSync(path);
  const sab = new SharedArrayBuffer(b.length);
  new Uint8Array(sab).set(b);
  return sab;
}

/* Loads the inputs and returns runRow(k) for picked row k. */
function prepare(spec, shared) {
  const Ctor = spec.dtype === "bf16" ? Uint16Array : Float32Array;
  const all = shared ? new Ctor(shared) : readTyped(spec.logits, Ctor);
  let offsets = null;
  let ids = null;
  if (spec.history_offsets) {
    offsets = readTyped(spec.history_offsets, Float64Array);
    ids = readTyped(spec.history_ids, Int32Array);
  }
  let masker = null;
  if (spec.constraint) {
    const c = spec.constraint;
    masker = new ByteDfaMasker(readTyped(c.next, Int32Array), readTyped(c.finals, Uint8Array), c.states,
                               readTyped(c.vocab_offsets, Float64Array), readTyped(c.vocab_bytes, Uint8Array));
  }
  const pick = spec.pick || Array.from({ length: spec.rows }, (_, i) => i);
  return (k) => {
    const r = pick[k];
    let logits = rowView(spec, all, r);
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
    if (masker) {
      // selectConstrainedToken: legal ids of the state (cached per state),
      // the masked copy, then sampleToken on it (gemma-session.ts:1305-1329)
      const legal = masker.legalTokenIds(spec.constraint.row_states[k]);
      logits = maskConstraintLogits(logits, legal, spec.constraint.termination || []);
    }
    return sampleWithProbability(logits, history, config, random);
  };
}

function runInline(spec) {
  const runRow = prepare(spec);
  const n = (spec.pick || Array.from({ length: spec.rows })).length;
  for (let k = 0; k < Math.min(spec.warmup || 0, n); k += 1) runRow(k);
  const t0 = process.hrtime.bigint();
  const results = [];
  for (let k = 0; k < n; k += 1) results.push(runRow(k));
  const seconds = Number(process.hrtime.bigint() - t0) / 1e9;
  return { results, seconds };
}

function runThreaded(spec, threads) {
  const { Worker } = require("worker_threads");
  const pick = spec.pick || Array.from({ length: spec.rows }, (_, i) => i);
  const n = pick.length;
  const parts = [];
  for (let w = 0; w < threads; w += 1) {
    const lo = Math.floor((w * n) / threads);
    const hi = Math.floor(((w + 1) * n) / threads);
    if (hi > lo) parts.push([lo, hi]);
  }
  const subSpec = ([lo, hi]) => {
    const s = Object.assign({}, spec, { pick: pick.slice(lo, hi) });
    if (Array.isArray(spec.configs)) s.configs = spec.configs.slice(lo, hi);
    if (spec.seeds) s.seeds = spec.seeds.slice(lo, hi);
    if (spec.uniforms) s.uniforms = spec.uniforms.slice(lo, hi);
    if (spec.constraint) {
      s.constraint = Object.assign({}, spec.constraint, { row_states: spec.constraint.row_states.slice(lo, hi) });
    }
    s.warmup = Math.min(spec.warmup || 0, hi - lo);
    return s;
  };
  const shared = readShared(spec.logits);
  return new Promise((resolve, reject) => {
    const workers = parts.map((p) => new Worker(__filename, { workerData: { spec: subSpec(p), shared } }));
    let ready = 0;
    let done = 0;
    let t0 = 0n;
    const out = new Array(parts.length);
    workers.forEach((w, i) => {
      w.on("error", reject);
      w.on("message", (m) => {
        if (m.ready) {
          ready += 1;
          if (ready === workers.length) {
            t0 = process.hrtime.bigint();
            workers.forEach((x) => x.postMessage("go"));
          }
        } else {
          out[i] = m.results;
          done += 1;
          if (done === workers.length) {
            const seconds = Number(process.hrtime.bigint() - t0) / 1e9;
            resolve({ results: [].concat(...out), seconds });
          }
        }
      });
    });
  });
}

function workerMain() {
  const { parentPort, workerData } = require("worker_threads");
  const spec = workerData.spec;
  const runRow = prepare(spec, workerData.shared);
  for (let k = 0; k < (spec.warmup || 0); k += 1) runRow(k);
  parentPort.once("message", () => {
    const results = [];
    for (let k = 0; k < spec.pick.length; k += 1) results.push(runRow(k));
    parentPort.postMessage({ results });
  });
  parentPort.postMessage({ ready: true });
}

async function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const threads = Math.max(1, spec.threads || 1);
  const { results, seconds } = threads > 1 ? await runThreaded(spec, threads) : runInline(spec);
  const cpus = os.cpus();
  fs.writeFileSync(spec.out, JSON.stringify({
    tokens: results.map((x) => x.token),
    probabilities: results.map((x) => x.probability),
    seconds,
    rows: results.length,
    threads,
    node: process.version,
    cpu_model: cpus.length ? cpus[0].model : "unknown",
    host_cpus: cpus.length,
  }));
}

let isWorker = false;
try {
  isWorker = !require("worker_threads").isMainThread;
} catch (e) {
  isWorker = false;
}
if (isWorker) workerMain();
else main().catch((e) => { console.error(e); process.exit(1); });
