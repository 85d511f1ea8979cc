"use strict";
/*
 * The constraint compiler (regex / JSON / JSON Schema -> byte-level DFA
 * tables) without a GPU:
 *  - the known answers of the reference's tests/constraints.spec.ts:27-157,
 *    with legal ids from the oracle's byte-DFA masker (oracle/constraint_ref.js)
 *    and acceptance walked over the tables;
 *  - whole-string acceptance against the platform's RegExp (full match, "u"),
 *    on random strings, for patterns with classes, escapes, quantifiers,
 *    alternation and non-ASCII ranges;
 *  - the byte table against a restatement of the reference's byte walk
 *    (constraints.ts:222-290: pending UTF-8 bytes, completion ranges,
 *    viability) over the same code-point DFA, on random byte strings: the
 *    same steps die and the same prefixes accept;
 *  - JSON grammars on serialized random values, and the rejections the
 *    reference's tests name.
 */
const assert = require("assert");
const path = require("path");
const { test, run } = require("./harness");

const ROOT = path.join(__dirname, "..", "..");
const { compileRegexToByteDfa, compileRegexToCodePointDfa } = require(path.join(ROOT, "gemma-webgpu-engine_amd", "node", "regex-dfa.js"));
const { compileConstraintTables } = require(path.join(ROOT, "gemma-webgpu-engine_amd", "node", "constraint-compiler.js"));
const { ByteDfaMasker } = require(path.join(ROOT, "oracle", "constraint_ref.js"));

const encoder = new TextEncoder();

// xorshift32, deterministic
function rng(seed) {
  let x = seed >>> 0 || 1;
  return () => {
    x ^= x << 13; x >>>= 0;
    x ^= x >>> 17;
    x ^= x << 5; x >>>= 0;
    return x / 4294967296;
  };
}

// viable states of a byte table: co-reachable to a final state
function byteViable(dfa) {
  const n = dfa.stateCount;
  const preds = Array.from({ length: n }, () => []);
  for (let s = 0; s < n; s += 1) for (let b = 0; b < 256; b += 1) {
    const t = dfa.next[s * 256 + b];
    if (t >= 0) preds[t].push(s);
  }
  const v = new Uint8Array(n);
  const stack = [];
  for (let s = 0; s < n; s += 1) if (dfa.finals[s]) { v[s] = 1; stack.push(s); }
  while (stack.length) for (const p of preds[stack.pop()]) if (!v[p]) { v[p] = 1; stack.push(p); }
  return v;
}

// a constraint over tables, as the engine's acceptToken / accepting /
// validateFinal behave (the GPU tests run the engine's own)
class TableConstraint {
  constructor(tables) {
    this.dfa = tables.dfa;
    this.validateOutput = tables.validateOutput;
    this.viable = byteViable(this.dfa);
    this.state = this.dfa.initial;
  }
  get accepting() { return this.dfa.finals[this.state] === 1; }
  acceptBytes(bytes) {
    let s = this.state;
    for (const b of bytes) {
      s = this.dfa.next[s * 256 + b];
      if (s < 0 || !this.viable[s]) throw new Error("Selected token violates the generation constraint");
    }
    this.state = s;
  }
  legalTokenIds(tokens) {
    const V = tokens.length;
    const offsets = new Float64Array(V + 1);
    const parts = tokens.map((t) => (t === null ? new Uint8Array(0) : typeof t === "string" ? encoder.encode(t) : t));
    parts.forEach((p, k) => { offsets[k + 1] = offsets[k] + p.length; });
    const bytes = new Uint8Array(offsets[V]);
    parts.forEach((p, k) => bytes.set(p, offsets[k]));
    const masker = new ByteDfaMasker(Int32Array.from(this.dfa.next), this.dfa.finals, this.dfa.stateCount, offsets, bytes);
    return Array.from(masker.legalTokenIds(this.state));
  }
  validateFinal(text) {
    if (!this.accepting) throw new Error("Generated output ended before the constraint accepted it");
    this.validateOutput(text);
  }
}

const compile = (c) => new TableConstraint(compileConstraintTables(c));

function acceptText(constraint, text) {
  const c = compile(constraint);
  c.acceptBytes(encoder.encode(text));
  c.validateFinal(text);
}

function accepts(dfa, bytes) {
  let s = dfa.initial;
  for (const b of bytes) {
    s = dfa.next[s * 256 + b];
    if (s < 0) return false;
  }
  return dfa.finals[s] === 1;
}

// ------------------------------------------- constraints.spec.ts:27-157
test("prunes a token list through a full-match regex DFA (constraints.spec.ts:27-39)", () => {
  const tokens = [null, "a", "b", "c", "ab", "ac", "x"];
  const c = compile({ type: "regex", pattern: "a(?:b|c)" });
  assert.deepStrictEqual(c.legalTokenIds(tokens), [1, 4, 5]);
  c.acceptBytes(encoder.encode("a"));
  assert.strictEqual(c.accepting, false);
  assert.deepStrictEqual(c.legalTokenIds(tokens), [2, 3]);
  c.acceptBytes(encoder.encode("b"));
  assert.strictEqual(c.accepting, true);
  c.validateFinal("ab");
});

test("preserves UTF-8 decoder state across token boundaries (:41-57)", () => {
  const arabic = encoder.encode("أ");
  const tokens = [null, arabic.slice(0, 1), arabic.slice(1), arabic, Uint8Array.of(0xff)];
  const c = compile({ type: "regex", pattern: "أ" });
  assert.deepStrictEqual(c.legalTokenIds(tokens), [1, 3]);
  c.acceptBytes(arabic.slice(0, 1));
  assert.strictEqual(c.accepting, false);
  assert.deepStrictEqual(c.legalTokenIds(tokens), [2]);
  c.acceptBytes(arabic.slice(1));
  assert.strictEqual(c.accepting, true);
});

test("rejects incomplete UTF-8 prefixes that cannot start the grammar (:59-70)", () => {
  const tokens = [null, Uint8Array.of(0xef), Uint8Array.of(0xbf), Uint8Array.of(0xbd), "{"];
  const c = compile({ type: "regex", pattern: "\\{" });
  assert.deepStrictEqual(c.legalTokenIds(tokens), [4]);
});

test("enforces bounded JSON syntax incrementally (:72-81)", () => {
  acceptText({ type: "json", maxDepth: 3, whitespace: "none" }, "{\"x\":[true,null,-1.5e2]}");
  assert.throws(() => {
    const c = compile({ type: "json", maxDepth: 2 });
    c.acceptBytes(encoder.encode("{]"));
  }, /violates the generation constraint/);
});

test("enforces an open JSON object root without prescribing properties (:83-93)", () => {
  const constraint = { type: "json-object", maxDepth: 3, whitespace: "none" };
  acceptText(constraint, "{\"city\":\"Paris\",\"facts\":[true,2]}");
  acceptText(constraint, "{}");
  assert.throws(() => acceptText(constraint, "[\"Paris\"]"), /violates the generation constraint/);
  assert.throws(() => acceptText(constraint, "\"Paris\""), /violates the generation constraint/);
});

test("enforces the supported closed JSON Schema subset (:95-113)", () => {
  const schema = {
    type: "object",
    properties: { kind: { enum: ["move", "wait"] }, count: { type: "integer" } },
    required: ["kind", "count"],
    additionalProperties: false,
  };
  acceptText({ type: "json-schema", schema, whitespace: "none" }, "{\"kind\":\"move\",\"count\":2}");
  assert.throws(() => acceptText({ type: "json-schema", schema, whitespace: "none" },
    "{\"kind\":\"invalid\",\"count\":2}"), /violates the generation constraint/);
});

test("enforces anchored string patterns while generating schema values (:115-133)", () => {
  const schema = {
    type: "object",
    properties: {
      hebrew: { type: "string", pattern: String.raw`^[\u0590-\u05FF ?!]+$` },
      arabic: { type: "string", pattern: String.raw`^[\u0600-\u06FF ?!]+$` },
    },
    required: ["hebrew", "arabic"],
    additionalProperties: false,
  };
  acceptText({ type: "json-schema", schema, whitespace: "none" }, "{\"hebrew\":\"שלום!\",\"arabic\":\"مرحبا!\"}");
  assert.throws(() => acceptText({ type: "json-schema", schema, whitespace: "none" },
    "{\"hebrew\":\"שלום!\",\"arabic\":\"איך أمشي؟\"}"), /violates the generation constraint/);
});

test("rejects unsupported regular and schema constructs (:135-157)", () => {
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "a(?=b)" }), /Unsupported generation constraint/);
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "(a)\\1" }), /Unsupported generation constraint/);
  assert.throws(() => compileConstraintTables({
    type: "json-schema",
    schema: {
      type: "object",
      properties: { required: { type: "boolean" }, optional: { type: "string" } },
      required: ["required"],
      additionalProperties: false,
    },
  }), /require every declared property/);
  assert.throws(() => compileConstraintTables({ type: "json-schema", schema: { type: "string", pattern: "[a-z]+" } }),
    /must be anchored/);
});

test("option errors keep the reference's messages and order", () => {
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "" }), /^Error: Regex constraint pattern must not be empty$/);
  assert.throws(() => compileConstraintTables({ type: "json", maxDepth: 9 }),
    /JSON constraint maxDepth must be an integer between 1 and 8/);
  assert.throws(() => compileConstraintTables({ type: "json", whitespace: "tabs" }), /Unsupported JSON whitespace mode: tabs/);
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "^a$" }), /Unsupported generation constraint: regex assertions are not supported/);
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "a\\bc" }), /regex assertions are not supported/);
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "(?<x>a)\\k<x>" }), /regex backreferences are not supported/);
  assert.throws(() => compileConstraintTables({ type: "regex", pattern: "a(" }), /Unsupported generation constraint: Invalid regular expression/);
  assert.throws(() => compileConstraintTables({ type: "json-schema", schema: { type: "object", properties: {}, required: [] } }),
    /require additionalProperties: false/);
  assert.throws(() => compileConstraintTables({ type: "json-schema", schema: { type: "array" } }), /require one object-valued items schema/);
  assert.throws(() => compileConstraintTables({ type: "json-schema", schema: { type: "array", items: { type: "null" }, minItems: 65 } }),
    /minItems must be an integer between 0 and 64/);
  assert.throws(() => compileConstraintTables({ type: "json-schema", schema: { type: "string", format: "date" } }),
    /Unsupported JSON Schema keywords: format/);
  assert.throws(() => compileConstraintTables({ type: "json-schema", schema: { type: "string", pattern: "^[\"a]$" } }),
    /cannot admit JSON escapes/);
});

// ------------------------------------------- regex language vs RegExp
const PATTERNS = [
  "a(?:b|c)", "[a-c]+x?", "(?:ab|a)*b", "\\d{2,4}-[A-Z]{2}", "x{3}|y{0,2}z", "[^a-c]{1,3}",
  "(?:foo|bar)+(?:baz)?", "\\w+\\s\\w+", "[\\u0590-\\u05FF ?!]+", "[\\u0600-\\u06FF]{2}", "é+|ß",
  "[\\u{1F600}-\\u{1F64F}]x", ".", "a.c", "\\x41\\u0042\\u{43}", "[\\-\\]\\\\]+", "(?<name>q)+r",
  "[\\d\\s]+", "\\S\\W", "[^]", "(?:)|a", "[^\\u0000-\\u007F]+", "\\uD83D\\uDE00", "a*?b+?c??",
];
const ALPHABET = ["a", "b", "c", "x", "y", "z", "q", "r", "f", "o", "A", "Z", "0", "5", "9", "-", " ", "\t", "\n",
  "é", "ß", "ש", "ل", "م", "ر", "😀", "🙏", "?", "!", "]", "\\", "A", "B", "C", "\u{10FFFF}", "ÿ", "€", "\uD7FB", "\uE000",
  "\u0800", "\u0FFF", "\u{10000}"];

test("acceptance equals RegExp full match on random strings", () => {
  const rand = rng(7);
  let checked = 0;
  for (const p of PATTERNS) {
    const dfa = compileRegexToByteDfa(p);
    const re = new RegExp(`^(?:${p})$`, "u");
    for (let k = 0; k < 1500; k += 1) {
      const n = Math.floor(rand() * 6);
      let s = "";
      for (let j = 0; j < n; j += 1) s += ALPHABET[Math.floor(rand() * ALPHABET.length)];
      assert.strictEqual(accepts(dfa, encoder.encode(s)), re.test(s), `${p} on ${JSON.stringify(s)}`);
      checked += 1;
    }
  }
  assert.ok(checked > 30000);
});

// the reference's byte walk (constraints.ts:222-290) over a code-point DFA
function referenceWalk(cp, bytes) {
  const edge = (node, c) => {
    for (const [lo, hi, t] of cp.states[node].out) if (lo <= c && c <= hi) return t;
    return -1;
  };
  const completion = (pending) => {
    const lead = pending[0];
    const length = lead <= 0xdf ? 2 : lead <= 0xef ? 3 : 4;
    if (pending.length >= length) return null;
    const secondMin = lead === 0xe0 ? 0xa0 : lead === 0xf0 ? 0x90 : 0x80;
    const secondMax = lead === 0xed ? 0x9f : lead === 0xf4 ? 0x8f : 0xbf;
    if (pending.length > 1 && (pending[1] < secondMin || pending[1] > secondMax)) return null;
    for (let k = 2; k < pending.length; k += 1) if (pending[k] < 0x80 || pending[k] > 0xbf) return null;
    const lo = pending.slice();
    const hi = pending.slice();
    while (lo.length < length) {
      const k = lo.length;
      lo.push(k === 1 ? secondMin : 0x80);
      hi.push(k === 1 ? secondMax : 0xbf);
    }
    const dec = (b) => {
      let c = b[0] & (b.length === 2 ? 0x1f : b.length === 3 ? 0x0f : 0x07);
      for (let k = 1; k < b.length; k += 1) c = (c << 6) | (b[k] & 0x3f);
      return c;
    };
    return [dec(lo), dec(hi)];
  };
  const viable = (st) => {
    if (!st.pending.length) return cp.viable[st.node] === 1;
    const r = completion(st.pending);
    if (!r) return false;
    return cp.states[st.node].out.some(([lo, hi, t]) => cp.viable[t] && lo <= r[1] && hi >= r[0]);
  };
  const step = (st, b) => {
    if (!st.pending.length) {
      if (b <= 0x7f) { const t = edge(st.node, b); return t < 0 ? null : { node: t, pending: [] }; }
      if ((b >= 0xc2 && b <= 0xdf) || (b >= 0xe0 && b <= 0xef) || (b >= 0xf0 && b <= 0xf4)) return { node: st.node, pending: [b] };
      return null;
    }
    if (b < 0x80 || b > 0xbf) return null;
    const bs = st.pending.concat([b]);
    const len = st.pending[0] <= 0xdf ? 2 : st.pending[0] <= 0xef ? 3 : 4;
    if (bs.length < len) return { node: st.node, pending: bs };
    if ((bs[0] === 0xe0 && bs[1] < 0xa0) || (bs[0] === 0xed && bs[1] > 0x9f) ||
        (bs[0] === 0xf0 && bs[1] < 0x90) || (bs[0] === 0xf4 && bs[1] > 0x8f)) return null;
    let c = bs[0] & (len === 2 ? 0x1f : len === 3 ? 0x0f : 0x07);
    for (let k = 1; k < bs.length; k += 1) c = (c << 6) | (bs[k] & 0x3f);
    const t = edge(st.node, c);
    return t < 0 ? null : { node: t, pending: [] };
  };
  // per byte: alive (the state exists and is viable) and, at the end, accepting
  let st = { node: 0, pending: [] };
  const alive = [];
  for (const b of bytes) {
    st = st && step(st, b);
    const ok = !!st && viable(st);
    alive.push(ok);
    if (!ok) break;
  }
  const accepting = alive.length === bytes.length && alive.every((x) => x) &&
    st.pending.length === 0 && cp.states[st.node].final;
  return { alive, accepting };
}

test("byte tables follow the reference's pending UTF-8 walk byte for byte", () => {
  const rand = rng(11);
  const pieces = ALPHABET.map((s) => encoder.encode(s));
  let steps = 0;
  for (const p of PATTERNS.concat([String.raw`"(?:[^"\\\x00-\x1F]|\\["\\/bfnrt]|\\u[0-9A-Fa-f]{4})*"`, "[\\u0800-\\u0FFF\\uD7F0-\\uE010]+"])) {
    const cp = compileRegexToCodePointDfa(p);
    const dfa = compileRegexToByteDfa(p);
    const viable = byteViable(dfa);
    for (let k = 0; k < 800; k += 1) {
      // bytes of random characters, cut anywhere, with stray bytes mixed in
      const bytes = [];
      const n = 1 + Math.floor(rand() * 6);
      for (let j = 0; j < n; j += 1) {
        const r = rand();
        if (r < 0.15) bytes.push(0x80 + Math.floor(rand() * 0x40));  // a stray continuation byte
        else if (r < 0.25) bytes.push(0xc0 + Math.floor(rand() * 0x40));  // a lead byte, valid or not
        else for (const b of pieces[Math.floor(rand() * pieces.length)]) bytes.push(b);
      }
      const ref = referenceWalk(cp, bytes);
      let s = dfa.initial;
      for (let j = 0; j < ref.alive.length; j += 1) {
        s = s < 0 ? -1 : dfa.next[s * 256 + bytes[j]];
        const ok = s >= 0 && viable[s] === 1;
        assert.strictEqual(ok, ref.alive[j], `${p}: byte ${j} of ${bytes.map((b) => b.toString(16))}`);
        steps += 1;
      }
      if (ref.alive.length === bytes.length && ref.alive[ref.alive.length - 1]) {
        assert.strictEqual(dfa.finals[s] === 1, ref.accepting, `${p}: accepting after ${bytes.map((b) => b.toString(16))}`);
      }
    }
  }
  assert.ok(steps > 10000, steps);
});

// ------------------------------------------------------------ JSON values
function randomJson(rand, depth) {
  const r = rand();
  if (depth <= 0 || r < 0.5) {
    const k = Math.floor(rand() * 6);
    if (k === 0) return Math.floor(rand() * 2000) - 1000;
    if (k === 1) return Number((rand() * 100 - 50).toFixed(3));
    if (k === 2) return rand() < 0.5;
    if (k === 3) return null;
    if (k === 4) return "s" + Math.floor(rand() * 100) + (rand() < 0.3 ? "\"\\é\n😀" : "");
    return 1.5e21;
  }
  if (r < 0.75) return Array.from({ length: Math.floor(rand() * 4) }, () => randomJson(rand, depth - 1));
  const o = {};
  for (let k = Math.floor(rand() * 4); k > 0; k -= 1) o["k" + Math.floor(rand() * 50)] = randomJson(rand, depth - 1);
  return o;
}
function depthOfJson(v) {
  if (v === null || typeof v !== "object") return 0;
  const kids = Array.isArray(v) ? v : Object.values(v);
  return 1 + kids.reduce((m, x) => Math.max(m, depthOfJson(x)), 0);
}

test("JSON grammars accept serialized values within their depth, and only those", () => {
  const rand = rng(5);
  const compiled = {};
  for (const depth of [1, 2, 3]) {
    compiled[depth] = compileConstraintTables({ type: "json", maxDepth: depth, whitespace: "none" }).dfa;
  }
  const obj2 = compileConstraintTables({ type: "json-object", maxDepth: 2, whitespace: "compact" }).dfa;
  for (let k = 0; k < 600; k += 1) {
    const v = randomJson(rand, 4);
    const text = JSON.stringify(v);
    const d = depthOfJson(v);
    for (const depth of [1, 2, 3]) {
      assert.strictEqual(accepts(compiled[depth], encoder.encode(text)), d <= depth, `depth ${depth}: ${text}`);
    }
    const spaced = JSON.stringify(v, null, 1).replace(/\n */g, " ");
    const isObject = v !== null && typeof v === "object" && !Array.isArray(v);
    assert.strictEqual(accepts(obj2, encoder.encode(" " + spaced + "  ")), isObject && d <= 2, `object ${spaced}`);
  }
  // text that is not JSON
  for (const bad of ["{\"a\":}", "[1,]", "01", "\"\u0001\"", "tru", "{\"a\" 1}", "[1 2]", "-", "1.", ".5", "\"\\x\""]) {
    assert.strictEqual(accepts(compiled[3], encoder.encode(bad)), false, bad);
  }
});

test("JSON Schema grammar and final check agree on their subset", () => {
  const schema = {
    type: "object",
    properties: {
      name: { type: "string", pattern: "^[a-z]{1,8}$" },
      tags: { type: "array", items: { enum: ["x", "y", 3] }, minItems: 1, maxItems: 3 },
      size: { type: ["integer", "null"] },
      mode: { oneOf: [{ const: "fast" }, { const: "slow" }] },
    },
    required: ["name", "tags", "size", "mode"],
    additionalProperties: false,
  };
  const good = ["{\"name\":\"ab\",\"tags\":[\"x\"],\"size\":3,\"mode\":\"fast\"}",
    "{\"name\":\"abcdefgh\",\"tags\":[\"x\",3,\"y\"],\"size\":null,\"mode\":\"slow\"}"];
  const bad = ["{\"name\":\"ab\",\"tags\":[],\"size\":3,\"mode\":\"fast\"}",
    "{\"name\":\"AB\",\"tags\":[\"x\"],\"size\":3,\"mode\":\"fast\"}",
    "{\"name\":\"ab\",\"tags\":[\"x\",\"x\",\"x\",\"x\"],\"size\":3,\"mode\":\"fast\"}",
    "{\"name\":\"ab\",\"tags\":[\"x\"],\"size\":3.5,\"mode\":\"fast\"}",
    "{\"tags\":[\"x\"],\"name\":\"ab\",\"size\":3,\"mode\":\"fast\"}"];
  for (const text of good) acceptText({ type: "json-schema", schema, whitespace: "none" }, text);
  for (const text of bad) {
    assert.throws(() => acceptText({ type: "json-schema", schema, whitespace: "none" }, text),
      /violates the generation constraint|ended before/, text);
  }
  // validateFinal's own check, for what the grammar lets through: oneOf with
  // two matching alternatives
  const twice = compile({ type: "json-schema", schema: { oneOf: [{ type: "integer" }, { type: "number" }] }, whitespace: "none" });
  twice.acceptBytes(encoder.encode("2"));
  assert.throws(() => twice.validateFinal("2"), /does not satisfy its schema/);
});

test("default JSON depth compiles within the reference's node budget", () => {
  const t0 = Date.now();
  const dfa = compileConstraintTables({ type: "json" }).dfa;
  assert.ok(dfa.stateCount > 100 && dfa.stateCount < 32767, dfa.stateCount);
  assert.ok(accepts(dfa, encoder.encode(" {\"a\": [1, {\"b\": [null]}]} ")));
  assert.ok(!accepts(dfa, encoder.encode("[[[[[1]]]]]")));  // depth 5
  console.log(`  json depth 4: ${dfa.stateCount} byte states in ${Date.now() - t0} ms`);
});

run();
