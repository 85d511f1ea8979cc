"use strict";
/*
 * Regular expressions (JavaScript syntax, "u" flag) compiled to the
 * byte-level DFA tables the engine masks with: next[state * 256 + byte]
 * (-1: no edge), finals[state], initial state 0.
 *
 * The reference (src/runtime/constraints.ts:186-220) builds a code-point DFA
 * with refa and walks it a byte at a time, buffering the bytes of a UTF-8
 * sequence as "pending" (transitionByte, :222-246) and accepting a pending
 * state only while some completion of it reaches a viable state
 * (isViableConstraintState / pendingUtf8CompletionRange, :253-290). Here the
 * same walk is compiled into the table ahead of time:
 *   1. parse the pattern (assertions and backreferences rejected, as the
 *      reference does, :189-196) into ranges of code points;
 *   2. a Thompson NFA over code-point ranges, then the subset construction
 *      over the ranges' elementary intervals (the code-point DFA);
 *   3. viability on the code-point DFA (co-reachable to a final state,
 *      :300-322);
 *   4. every (code-point state, pending prefix) pair the reference can reach
 *      and keep becomes a byte state: ASCII bytes take the code-point edge,
 *      lead bytes C2-DF / E0-EF / F0-F4 and continuation bytes 80-BF narrow
 *      the interval of code points the prefix can still complete to, which
 *      excludes overlong forms and surrogates exactly as the reference's
 *      completion ranges do. A prefix stays only while that interval meets
 *      an edge into a viable state; pending states with the same future
 *      (the same edges over their interval, the same bytes left) are one;
 *   5. Moore minimisation of the byte table.
 * accepting = final byte state (pending states are never final), which is
 * the reference's "pending empty and final" (:52-54).
 *
 * One difference is by construction: a state the pattern can leave only
 * through lone surrogate code points (U+D800-DFFF, which no UTF-8 sequence
 * encodes) is viable in the code-point DFA but has no byte path onward; the
 * byte table treats it as dead one step earlier than the reference.
 */

const MAX_CP = 0x10ffff;

class RegexLimitError extends Error {}

// ------------------------------------------------------------ code-point sets
// A set is a sorted array of disjoint, non-adjacent [lo, hi] ranges.
function normalize(ranges) {
  const r = ranges.filter((x) => x[0] <= x[1]).map((x) => [x[0], x[1]]).sort((a, b) => a[0] - b[0]);
  const out = [];
  for (const x of r) {
    const last = out[out.length - 1];
    if (last && x[0] <= last[1] + 1) last[1] = Math.max(last[1], x[1]);
    else out.push(x);
  }
  return out;
}
function complement(set) {
  const out = [];
  let next = 0;
  for (const [lo, hi] of set) {
    if (lo > next) out.push([next, lo - 1]);
    next = hi + 1;
  }
  if (next <= MAX_CP) out.push([next, MAX_CP]);
  return out;
}
const DIGIT = [[0x30, 0x39]];
const WORD = normalize([[0x30, 0x39], [0x41, 0x5a], [0x5f, 0x5f], [0x61, 0x7a]]);
const SPACE = normalize([[0x09, 0x0d], [0x20, 0x20], [0xa0, 0xa0], [0x1680, 0x1680], [0x2000, 0x200a],
  [0x2028, 0x2029], [0x202f, 0x202f], [0x205f, 0x205f], [0x3000, 0x3000], [0xfeff, 0xfeff]]);
const DOT = complement(normalize([[0x0a, 0x0a], [0x0d, 0x0d], [0x2028, 0x2029]]));

// ------------------------------------------------------------------ parser
// AST: {k: "set", set} | {k: "seq", items} | {k: "alt", items} |
//      {k: "rep", node, min, max}   (max Infinity: unbounded)
function parseRegex(source) {
  // the platform's own parser settles what is valid "u" syntax and its error
  // text; the walk below then reads a pattern known to be well formed
  // eslint-disable-next-line no-new
  new RegExp(source, "u");
  const cps = Array.from(source, (ch) => ch.codePointAt(0));
  let i = 0;
  const peek = (o) => cps[i + (o || 0)];
  const eat = (c) => {
    if (cps[i] === c) { i += 1; return true; }
    return false;
  };
  const isDigit = (c) => c >= 0x30 && c <= 0x39;
  const hexVal = (c) => {
    if (c >= 0x30 && c <= 0x39) return c - 0x30;
    if (c >= 0x41 && c <= 0x46) return c - 0x41 + 10;
    if (c >= 0x61 && c <= 0x66) return c - 0x61 + 10;
    return -1;
  };
  const readHex = (n) => {
    let v = 0;
    for (let k = 0; k < n; k += 1) v = v * 16 + hexVal(cps[i++]);
    return v;
  };
  const unsupportedAssertion = () => { throw new Error("regex assertions are not supported"); };
  const unsupportedBackreference = () => { throw new Error("regex backreferences are not supported"); };

  // \u escapes: \u{...}, or \uXXXX with a following \uXXXX low surrogate
  // joined into one code point
  function readUnicodeEscape() {
    if (eat(0x7b)) {
      let v = 0;
      while (cps[i] !== 0x7d) v = v * 16 + hexVal(cps[i++]);
      i += 1;
      return v;
    }
    const hi = readHex(4);
    if (hi >= 0xd800 && hi <= 0xdbff && cps[i] === 0x5c && cps[i + 1] === 0x75 && cps[i + 2] !== 0x7b) {
      const save = i;
      i += 2;
      const lo = readHex(4);
      if (lo >= 0xdc00 && lo <= 0xdfff) return 0x10000 + ((hi - 0xd800) << 10) + (lo - 0xdc00);
      i = save;
    }
    return hi;
  }

  // one escape after "\" (inClass: inside [...]); returns a set
  function readEscape(inClass) {
    const c = cps[i++];
    switch (c) {
      case 0x64: return DIGIT;                 // \d
      case 0x44: return complement(DIGIT);     // \D
      case 0x77: return WORD;                  // \w
      case 0x57: return complement(WORD);      // \W
      case 0x73: return SPACE;                 // \s
      case 0x53: return complement(SPACE);     // \S
      case 0x74: return [[0x09, 0x09]];        // \t
      case 0x6e: return [[0x0a, 0x0a]];        // \n
      case 0x76: return [[0x0b, 0x0b]];        // \v
      case 0x66: return [[0x0c, 0x0c]];        // \f
      case 0x72: return [[0x0d, 0x0d]];        // \r
      case 0x63: {                             // \cX
        const x = cps[i++];
        return [[x % 32, x % 32]];
      }
      case 0x78: {                             // \xHH
        const v = readHex(2);
        return [[v, v]];
      }
      case 0x75: {                             // \u
        const v = readUnicodeEscape();
        return [[v, v]];
      }
      case 0x70: case 0x50:                    // \p{...} \P{...}
        throw new Error("unicode property escapes are not supported");
      case 0x62:                               // \b
        if (inClass) return [[0x08, 0x08]];
        return unsupportedAssertion();
      case 0x42:                               // \B
        return unsupportedAssertion();
      case 0x6b:                               // \k<name>
        return unsupportedBackreference();
      case 0x30:                               // \0 (never followed by a digit in "u" mode)
        return [[0, 0]];
      default:
        if (c >= 0x31 && c <= 0x39) return unsupportedBackreference();
        return [[c, c]];                       // identity escape of a syntax character, "/" or "-"
    }
  }

  function parseClass() {
    // after "["
    const negate = eat(0x5e);
    const parts = [];
    const atom = () => {
      if (eat(0x5c)) return { set: readEscape(true) };
      return { set: [[cps[i], cps[i++]]] };
    };
    while (cps[i] !== 0x5d) {
      const a = atom();
      if (cps[i] === 0x2d && cps[i + 1] !== 0x5d) {
        i += 1;
        const b = atom();
        parts.push([a.set[0][0], b.set[0][0]]);
      } else {
        for (const r of a.set) parts.push(r);
      }
    }
    i += 1;
    const set = normalize(parts);
    return negate ? complement(set) : set;
  }

  function parseAtom() {
    const c = peek();
    if (c === 0x28) {                          // (
      i += 1;
      if (eat(0x3f)) {                         // (?
        if (eat(0x3a)) {                       // (?:
          const node = parseAlt();
          i += 1;
          return node;
        }
        if (cps[i] === 0x3d || cps[i] === 0x21) return unsupportedAssertion();  // (?= (?!
        if (cps[i] === 0x3c && (cps[i + 1] === 0x3d || cps[i + 1] === 0x21)) return unsupportedAssertion();
        if (eat(0x3c)) {                       // (?<name>
          while (cps[i] !== 0x3e) i += 1;
          i += 1;
        }
      }
      const node = parseAlt();
      i += 1;                                  // )
      return node;
    }
    if (c === 0x5b) {                          // [
      i += 1;
      return { k: "set", set: parseClass() };
    }
    if (c === 0x2e) {                          // .
      i += 1;
      return { k: "set", set: DOT };
    }
    if (c === 0x5e || c === 0x24) return unsupportedAssertion();  // ^ $
    if (c === 0x5c) {                          // \
      i += 1;
      return { k: "set", set: readEscape(false) };
    }
    i += 1;
    return { k: "set", set: [[c, c]] };
  }

  function parseQuantified() {
    let node = parseAtom();
    for (;;) {
      let min;
      let max;
      const c = peek();
      if (c === 0x2a) { min = 0; max = Infinity; i += 1; }
      else if (c === 0x2b) { min = 1; max = Infinity; i += 1; }
      else if (c === 0x3f) { min = 0; max = 1; i += 1; }
      else if (c === 0x7b) {
        i += 1;
        min = 0;
        while (isDigit(cps[i])) min = min * 10 + (cps[i++] - 0x30);
        max = min;
        if (eat(0x2c)) {
          if (cps[i] === 0x7d) max = Infinity;
          else {
            max = 0;
            while (isDigit(cps[i])) max = max * 10 + (cps[i++] - 0x30);
          }
        }
        i += 1;                                // }
      } else {
        return node;
      }
      eat(0x3f);                               // lazy: the same language
      node = { k: "rep", node, min, max };
    }
  }

  function parseSeq() {
    const items = [];
    while (i < cps.length && cps[i] !== 0x7c && cps[i] !== 0x29) items.push(parseQuantified());
    return items.length === 1 ? items[0] : { k: "seq", items };
  }

  function parseAlt() {
    const items = [parseSeq()];
    while (eat(0x7c)) items.push(parseSeq());
    return items.length === 1 ? items[0] : { k: "alt", items };
  }

  const ast = parseAlt();
  return ast;
}

// --------------------------------------------------------------------- NFA
// Thompson construction: states hold eps[] and edges [[lo, hi, to]].
// maxPositions bounds the character positions (one per character-set leaf
// of the expanded pattern): an epsilon-free automaton of the pattern has one
// node per position plus its initial node, the count the reference's NFA
// node limit applies to (constraints.ts:9,205-210).
class Nfa {
  constructor(maxStates, maxPositions) {
    this.eps = [];
    this.edges = [];
    this.maxStates = maxStates;
    this.maxPositions = maxPositions || Infinity;
    this.positions = 0;
  }
  add() {
    if (this.eps.length >= this.maxStates) throw new RegexLimitError(`more than ${this.maxStates} NFA states`);
    this.eps.push([]);
    this.edges.push([]);
    return this.eps.length - 1;
  }
  // fragment of node between fresh states; returns [start, end]
  build(node) {
    if (node.k === "set") {
      this.positions += 1;
      if (this.positions >= this.maxPositions) {
        throw new RegexLimitError(`more than ${this.maxPositions - 1} NFA nodes`);
      }
      const s = this.add();
      const e = this.add();
      for (const [lo, hi] of node.set) this.edges[s].push([lo, hi, e]);
      return [s, e];
    }
    if (node.k === "seq") {
      const s = this.add();
      let cur = s;
      for (const item of node.items) {
        const [a, b] = this.build(item);
        this.eps[cur].push(a);
        cur = b;
      }
      return [s, cur];
    }
    if (node.k === "alt") {
      const s = this.add();
      const e = this.add();
      for (const item of node.items) {
        const [a, b] = this.build(item);
        this.eps[s].push(a);
        this.eps[b].push(e);
      }
      return [s, e];
    }
    // rep: min copies, then (max - min) optional copies or a loop
    const s = this.add();
    let cur = s;
    for (let k = 0; k < node.min; k += 1) {
      const [a, b] = this.build(node.node);
      this.eps[cur].push(a);
      cur = b;
    }
    if (node.max === Infinity) {
      const [a, b] = this.build(node.node);
      const e = this.add();
      this.eps[cur].push(a, e);
      this.eps[b].push(a, e);
      return [s, e];
    }
    const e = this.add();
    for (let k = node.min; k < node.max; k += 1) {
      const [a, b] = this.build(node.node);
      this.eps[cur].push(a, e);
      cur = b;
    }
    this.eps[cur].push(e);
    return [s, e];
  }
}

// ------------------------------------------------------- code-point DFA
// states: {final, out: [[lo, hi, to]] sorted, disjoint}
function subsetConstruction(nfa, start, accept, maxStates) {
  const mark = new Int32Array(nfa.eps.length);
  let stamp = 0;
  const closure = (seed) => {
    stamp += 1;
    const out = [];
    const stack = [];
    for (const s of seed) if (mark[s] !== stamp) { mark[s] = stamp; stack.push(s); out.push(s); }
    while (stack.length) {
      const s = stack.pop();
      for (const t of nfa.eps[s]) if (mark[t] !== stamp) { mark[t] = stamp; stack.push(t); out.push(t); }
    }
    return out.sort((a, b) => a - b);
  };
  const states = [];
  const index = new Map();
  const intern = (set) => {
    const key = set.join(",");
    let id = index.get(key);
    if (id === undefined) {
      if (states.length >= maxStates) throw new RegexLimitError(`more than ${maxStates} DFA states`);
      id = states.length;
      index.set(key, id);
      states.push({ set, final: set.includes(accept), out: null });
    }
    return id;
  };
  intern(closure([start]));
  for (let d = 0; d < states.length; d += 1) {
    const st = states[d];
    // elementary intervals of the states' edges: sweep their endpoints
    const edges = [];
    for (const s of st.set) for (const e of nfa.edges[s]) edges.push(e);
    const points = new Set();
    for (const [lo, hi] of edges) { points.add(lo); points.add(hi + 1); }
    const cuts = Array.from(points).sort((a, b) => a - b);
    const out = [];
    for (let k = 0; k + 1 < cuts.length; k += 1) {
      const lo = cuts[k];
      const hi = cuts[k + 1] - 1;
      const targets = [];
      for (const [elo, ehi, to] of edges) if (elo <= lo && ehi >= hi) targets.push(to);
      if (!targets.length) continue;
      const to = intern(closure(targets));
      const last = out[out.length - 1];
      if (last && last[2] === to && last[1] + 1 === lo) last[1] = hi;
      else out.push([lo, hi, to]);
    }
    st.out = out;
    st.set = null;
  }
  return states;
}

// findViableStates (constraints.ts:300-322) on the code-point DFA
function viableStates(states) {
  const preds = states.map(() => []);
  states.forEach((st, s) => { for (const [, , t] of st.out) preds[t].push(s); });
  const viable = new Uint8Array(states.length);
  const stack = [];
  states.forEach((st, s) => { if (st.final) { viable[s] = 1; stack.push(s); } });
  while (stack.length) {
    const t = stack.pop();
    for (const p of preds[t]) if (!viable[p]) { viable[p] = 1; stack.push(p); }
  }
  return viable;
}

// -------------------------------------------------- byte-level expansion
// UTF-8 lengths' valid code points; 3-byte forms skip the surrogates, which
// leaves a contiguous interval for every lead byte (ED: D000-D7FF)
function leadInfo(b) {
  if (b >= 0xc2 && b <= 0xdf) return { left: 1, lo: (b & 0x1f) << 6, size: 64, valid: [0x80, 0x7ff] };
  if (b >= 0xe0 && b <= 0xef) return { left: 2, lo: (b & 0x0f) << 12, size: 4096, valid: [0x800, 0xffff] };
  if (b >= 0xf0 && b <= 0xf4) return { left: 3, lo: (b & 0x07) << 18, size: 262144, valid: [0x10000, MAX_CP] };
  return null;
}
function clipInterval(lo, hi, valid) {
  let a = Math.max(lo, valid[0]);
  let b = Math.min(hi, valid[1]);
  if (valid[1] === 0xffff) {
    // no surrogates: an interval inside D800-DFFF is empty; one reaching
    // into it from below is cut at D7FF (every lead's interval lies on one
    // side, so no interval spans the gap)
    if (a >= 0xd800 && b <= 0xdfff) return null;
    if (a < 0xd800 && b >= 0xd800) b = Math.min(b, 0xd7ff);
    if (a <= 0xdfff && b > 0xdfff && a >= 0xd800) a = 0xe000;
  }
  return a <= b ? [a, b] : null;
}

function buildByteTable(states, viable, maxStates) {
  // byte state ids: code-point state s -> s; pending states after them
  const S = states.length;
  const next = [];   // Int32Array per state, filled below
  const finals = [];
  const pendingIndex = new Map();
  const pendingQueue = [];
  // the code-point edges of state s into viable states, restricted to [lo, hi]
  const edgesIn = (s, lo, hi) => {
    const out = [];
    for (const [elo, ehi, t] of states[s].out) {
      if (ehi < lo || elo > hi || !viable[t]) continue;
      out.push([Math.max(elo, lo), Math.min(ehi, hi), t]);
    }
    return out;
  };
  // pending state of code-point state s whose completions are the code points
  // rawLo .. rawLo + size - 1 clipped to valid, with `left` bytes to come;
  // -1 when no completion reaches a viable state. Same future, same state.
  const pendingState = (s, rawLo, size, left, valid) => {
    const iv = clipInterval(rawLo, rawLo + size - 1, valid);
    if (!iv) return -1;
    const edges = edgesIn(s, iv[0], iv[1]);
    if (!edges.length) return -1;
    const key = `${left}|${iv[0] - rawLo}|${iv[1] - rawLo}|` + edges.map((e) => `${e[0] - rawLo}:${e[1] - rawLo}:${e[2]}`).join(",");
    let id = pendingIndex.get(key);
    if (id === undefined) {
      id = S + pendingQueue.length;
      if (id >= maxStates) throw new RegexLimitError(`more than ${maxStates} byte-level states`);
      pendingIndex.set(key, id);
      pendingQueue.push({ s, rawLo, size, left, valid });
    }
    return id;
  };
  for (let s = 0; s < S; s += 1) {
    const row = new Int32Array(256).fill(-1);
    for (const [lo, hi, t] of states[s].out) {
      if (!viable[t] || lo > 0x7f) continue;
      for (let b = lo; b <= Math.min(hi, 0x7f); b += 1) row[b] = t;
    }
    for (let b = 0xc2; b <= 0xf4; b += 1) {
      const L = leadInfo(b);
      row[b] = pendingState(s, L.lo, L.size, L.left, L.valid);
    }
    next.push(row);
    finals.push(states[s].final ? 1 : 0);
  }
  for (let q = 0; q < pendingQueue.length; q += 1) {
    const p = pendingQueue[q];
    const row = new Int32Array(256).fill(-1);
    const sub = p.size / 64;
    for (let c = 0x80; c <= 0xbf; c += 1) {
      const lo = p.rawLo + (c - 0x80) * sub;
      if (p.left === 1) {
        // the code point is complete: the code-point edge, if valid and viable
        const iv = clipInterval(lo, lo, p.valid);
        if (!iv) continue;
        for (const [elo, ehi, t] of states[p.s].out) {
          if (elo <= lo && ehi >= lo) { if (viable[t]) row[c] = t; break; }
        }
      } else {
        row[c] = pendingState(p.s, lo, sub, p.left - 1, p.valid);
      }
    }
    next.push(row);
    finals.push(0);
  }
  return { next, finals };
}

// Moore minimisation of a complete-or-partial byte table (-1 is its own
// class); returns the quotient with the initial state first.
function minimize(next, finals, initial) {
  // only the states reachable from the initial one
  const reach = new Uint8Array(next.length);
  const stack = [initial];
  reach[initial] = 1;
  while (stack.length) {
    const s = stack.pop();
    for (let b = 0; b < 256; b += 1) {
      const t = next[s][b];
      if (t >= 0 && !reach[t]) { reach[t] = 1; stack.push(t); }
    }
  }
  const keep = [];
  const newId = new Int32Array(next.length).fill(-1);
  for (let s = 0; s < next.length; s += 1) if (reach[s]) { newId[s] = keep.length; keep.push(s); }
  next = keep.map((s) => next[s].map((t) => (t < 0 ? -1 : newId[t])));
  finals = keep.map((s) => finals[s]);
  initial = newId[initial];
  const n = next.length;
  let cls = Int32Array.from(finals);
  let count = 2;
  for (;;) {
    const index = new Map();
    const nc = new Int32Array(n);
    for (let s = 0; s < n; s += 1) {
      const row = next[s];
      let key = String(cls[s]);
      for (let b = 0; b < 256; b += 1) key += "," + (row[b] < 0 ? -1 : cls[row[b]]);
      let id = index.get(key);
      if (id === undefined) { id = index.size; index.set(key, id); }
      nc[s] = id;
    }
    const stable = index.size === count;
    cls = nc;
    count = index.size;
    if (stable) break;
  }
  // renumber: the initial state's class first, the rest in order of first use
  const order = new Int32Array(count).fill(-1);
  let k = 0;
  order[cls[initial]] = k++;
  for (let s = 0; s < n; s += 1) if (order[cls[s]] < 0) order[cls[s]] = k++;
  const outNext = new Int32Array(count * 256).fill(-1);
  const outFinals = new Uint8Array(count);
  const done = new Uint8Array(count);
  for (let s = 0; s < n; s += 1) {
    const c = order[cls[s]];
    if (done[c]) continue;
    done[c] = 1;
    outFinals[c] = finals[s];
    for (let b = 0; b < 256; b += 1) {
      const t = next[s][b];
      outNext[c * 256 + b] = t < 0 ? -1 : order[cls[t]];
    }
  }
  return { stateCount: count, next: outNext, finals: outFinals, initial: 0 };
}

/* The code-point DFA of a pattern and its viable states: { states: [{final,
 * out: [[lo, hi, to]]}], viable: Uint8Array }, state 0 initial. */
function compileRegexToCodePointDfa(source, options) {
  const maxStates = (options && options.maxStates) || 1000000;
  const ast = parseRegex(source);
  const nfa = new Nfa(Math.max(maxStates * 8, 400000), options && options.maxStates);
  const [start, end] = nfa.build(ast);
  const states = subsetConstruction(nfa, start, end, maxStates);
  return { states, viable: viableStates(states) };
}

/* The byte-level DFA of a pattern. options.maxStates bounds the NFA's
 * positions (an epsilon-free automaton's nodes), the code-point DFA and the
 * byte table (the reference bounds its automata at 50 000 nodes for JSON
 * grammars, constraints.ts:9,196-212). Throws Error
 * with the reason; the caller adds the "Unsupported generation constraint"
 * prefix. */
function compileRegexToByteDfa(source, options) {
  const maxStates = (options && options.maxStates) || 1000000;
  const { states, viable } = compileRegexToCodePointDfa(source, options);
  if (!states.some((st) => st.final)) throw new Error("constraint accepts no output");
  const table = buildByteTable(states, viable, Math.max(maxStates, 32767) * 4);
  return minimize(table.next, table.finals, 0);
}

module.exports = { compileRegexToByteDfa, compileRegexToCodePointDfa, parseRegex, RegexLimitError, normalize, complement };
