"use strict";
/*
 * Constrained decoding over byte-level DFA tables (src/runtime/constraints.ts):
 *   CompiledGenerationConstraint  accepting / legalTokenIds / acceptToken /
 *                                 acceptBytes / validateFinal (:32-113)
 *   maskConstraintLogits          (:159-173)
 *   selectConstrainedToken        (src/runtime/gemma-session.ts:1305-1329)
 * The engine works on byte-level DFA tables: next[state * 256 + byte] (-1:
 * no edge), finals[state], an initial state. Viable states (co-reachable to a
 * final state, constraints.ts:300-322) are derived by the library. regex,
 * json, json-object and json-schema constraints are compiled into such tables
 * (constraint-compiler.js, regex-dfa.js); "byte-dfa" takes tables as given.
 */
const { Engine } = require("./engine");
const { compileConstraintTables } = require("./constraint-compiler");
const { engineFor, sampleToken } = require("./sampling");

const { EOS_TOKEN_IDS } = require("./token-bytes");

class ByteLevelDfa {
  constructor(spec) {
    const n = spec.stateCount === undefined ? spec.finals.length : spec.stateCount;
    if (!Number.isInteger(n) || n <= 0) throw new RangeError("a DFA needs at least one state");
    this.stateCount = n;
    this.next = Int32Array.from(spec.next);
    if (this.next.length !== n * 256) throw new RangeError("next must hold stateCount * 256 entries");
    this.finals = Uint8Array.from(spec.finals, (f) => (f ? 1 : 0));
    if (this.finals.length !== n) throw new RangeError("finals must hold stateCount entries");
    this.initial = spec.initial === undefined ? 0 : spec.initial;
  }
}

class CompiledGenerationConstraint {
  /* dfa: ByteLevelDfa; validateOutput(text) runs in validateFinal; engine:
   * an Engine whose vocab size matches the tries used (default: the shared
   * single-row engine of the trie's vocab size). */
  constructor(dfa, validateOutput, engine) {
    this.dfa = dfa instanceof ByteLevelDfa ? dfa : new ByteLevelDfa(dfa);
    this.validateOutput = validateOutput || (() => {});
    this.engine = engine || null;
    this.state = this.dfa.initial;
    this.legalCache = new WeakMap();
  }

  engineForTrie(trie) {
    const e = this.engine || engineFor(trie.vocabularySize);
    e.useVocab(trie);
    e.useDfa(this.dfa);
    return e;
  }

  get accepting() {
    return this.dfa.finals[this.state] === 1;
  }

  legalTokenIds(trie) {
    let perState = this.legalCache.get(trie);
    if (!perState) {
      perState = new Map();
      this.legalCache.set(trie, perState);
    }
    const cached = perState.get(this.state);
    if (cached) return cached;
    const ids = Object.freeze(Array.from(this.engineForTrie(trie).legalTokenIds(this.state)));
    perState.set(this.state, ids);
    return ids;
  }

  acceptToken(tokenBytes) {
    const e = this.engine || engineFor(1);
    e.useDfa(this.dfa);
    this.state = e.dfaAdvanceBytes(this.state, Uint8Array.from(tokenBytes));
  }

  acceptBytes(bytes) {
    this.acceptToken(bytes);
  }

  validateFinal(text) {
    if (!this.accepting) throw new Error("Generated output ended before the constraint accepted it");
    this.validateOutput(text);
  }
}

/* compileGenerationConstraint (constraints.ts:115-157): regex, json,
 * json-object and json-schema constraints compiled to byte-level tables, or
 * "byte-dfa" tables as given. */
function compileGenerationConstraint(constraint) {
  if (constraint && constraint.type === "byte-dfa") {
    return new CompiledGenerationConstraint(new ByteLevelDfa(constraint), constraint.validateOutput);
  }
  const tables = compileConstraintTables(constraint);
  return new CompiledGenerationConstraint(new ByteLevelDfa(tables.dfa), tables.validateOutput);
}

function maskConstraintLogits(rawLogits, legalTokenIds, terminationTokenIds) {
  const raw = rawLogits instanceof Float32Array ? rawLogits : Float32Array.from(rawLogits);
  if (raw.length === 0) return new Float32Array(0);
  return engineFor(1).maskLogits(raw, legalTokenIds, terminationTokenIds);
}

/* selectConstrainedToken (gemma-session.ts:1305-1329): legal ids of the
 * constraint's state plus extra legal ids, minus termination ids (EOS and
 * stop ids, legal only while the constraint accepts); a dead end throws;
 * otherwise the masked row is sampled as sampleToken does. */
function selectConstrainedToken(args) {
  const termination = new Set(EOS_TOKEN_IDS.concat(Array.from(args.customStopTokens || [])));
  const legal = Array.from(new Set(args.constraint.legalTokenIds(args.trie).concat(args.additionalLegalTokens || [])))
    .filter((id) => !termination.has(id));
  const legalTermination = args.constraint.accepting ? Array.from(termination) : [];
  if (legal.length === 0 && legalTermination.length === 0) {
    throw new Error("Generation constraint reached a tokenization dead end");
  }
  const masked = maskConstraintLogits(args.logits, legal, legalTermination);
  return sampleToken(masked, args.history, args.config, () => args.random.next());
}

module.exports = {
  EOS_TOKEN_IDS,
  ByteLevelDfa,
  CompiledGenerationConstraint,
  compileGenerationConstraint,
  maskConstraintLogits,
  selectConstrainedToken,
  Engine,
};
