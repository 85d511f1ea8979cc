"use strict";
/*
 * compileGenerationConstraint's front end (src/runtime/constraints.ts:115-157,
 * 175-184, 324-519): each constraint type becomes a regular expression over
 * code points, which regex-dfa.js turns into a byte-level DFA, and a check of
 * the finished text for validateFinal.
 *   regex        the pattern itself; the final text must match it whole
 *                (new RegExp(pattern, "u"), :175-184)
 *   json         whitespace, a JSON value nested at most maxDepth deep,
 *                whitespace; the text must parse (:121-126)
 *   json-object  the same with an object at the root (:127-135)
 *   json-schema  the closed schema subset the reference accepts (:335-519):
 *                const / enum / oneOf / anyOf / type / anchored string
 *                patterns / objects with additionalProperties false and
 *                every property required / arrays with items and
 *                minItems..maxItems (0..64)
 * The grammars (the JSON string, number and integer forms, whitespace modes,
 * the depth-bounded value / array / object recursion, the schema-to-pattern
 * rules and their error messages) follow the reference's, so that the same
 * outputs are legal. The reference validates schema outputs with ajv, which
 * is not available here: validateFinal checks the same subset of keywords
 * itself (oneOf: exactly one alternative, as JSON Schema defines it).
 */
const { compileRegexToByteDfa } = require("./regex-dfa");

const DEFAULT_JSON_DEPTH = 4;
const MAX_JSON_DEPTH = 8;
const MAX_SCHEMA_PROPERTIES = 12;
const JSON_GRAMMAR_MAX_NODES = 50000;
const JSON_STRING = String.raw`"(?:[^"\\\x00-\x1F]|\\["\\/bfnrt]|\\u[0-9A-Fa-f]{4})*"`;
const JSON_NUMBER = String.raw`-?(?:0|[1-9][0-9]*)(?:\.[0-9]+)?(?:[eE][+-]?[0-9]+)?`;
const JSON_INTEGER = String.raw`-?(?:0|[1-9][0-9]*)`;

function messageOf(error) {
  return error instanceof Error ? error.message : String(error);
}

function depthOf(value) {
  const depth = value === undefined ? DEFAULT_JSON_DEPTH : value;
  if (!Number.isInteger(depth) || depth < 1 || depth > MAX_JSON_DEPTH) {
    throw new Error(`JSON constraint maxDepth must be an integer between 1 and ${MAX_JSON_DEPTH}`);
  }
  return depth;
}

function whitespaceOf(mode) {
  switch (mode) {
    case "none": return "";
    case "compact": return " *";
    case "any": return "[\\x20\\x09\\x0A\\x0D]*";
    default: throw new Error(`Unsupported JSON whitespace mode: ${String(mode)}`);
  }
}

function anyOf(patterns) {
  return patterns.length === 1 ? patterns[0] : `(?:${patterns.join("|")})`;
}

// members of an object: "{" ws (string ws ":" ws value (ws "," ws ...)*)? ws "}"
function objectOf(value, ws) {
  const member = `${JSON_STRING}${ws}:${ws}${value}`;
  return `\\{${ws}(?:${member}(?:${ws},${ws}${member})*)?${ws}\\}`;
}

function valueOf(depth, ws) {
  const primitive = `(?:${JSON_STRING}|${JSON_NUMBER}|true|false|null)`;
  if (depth <= 0) return primitive;
  const child = valueOf(depth - 1, ws);
  const array = `\\[${ws}(?:${child}(?:${ws},${ws}${child})*)?${ws}\\]`;
  return `(?:${primitive}|${array}|${objectOf(child, ws)})`;
}

// ------------------------------------------------------------ JSON Schema
const SCHEMA_KEYWORDS = new Set([
  "$schema", "title", "description", "default", "examples",
  "type", "const", "enum", "oneOf", "anyOf", "pattern",
  "properties", "required", "additionalProperties",
  "items", "minItems", "maxItems",
]);

function escapeRegex(text) {
  return text.replace(/[\\^$.*+?()[\]{}|/]/g, "\\$&");
}

function literalOf(value) {
  const text = JSON.stringify(value);
  if (text === undefined) throw new Error("JSON Schema const/enum value is not JSON-serializable");
  return escapeRegex(text);
}

function countOf(value, name) {
  if (!Number.isInteger(value) || value < 0 || value > 64) {
    throw new Error(`JSON Schema ${name} must be an integer between 0 and 64`);
  }
  return value;
}

function listOf(item, ws, count) {
  const parts = [];
  for (let k = 0; k < count; k += 1) parts.push((k ? `${ws},${ws}` : "") + item);
  return parts.join("");
}

function stringPatternOf(schema) {
  if (schema.pattern === undefined) return JSON_STRING;
  if (typeof schema.pattern !== "string") throw new Error("JSON Schema string pattern must be a string");
  if (!schema.pattern.startsWith("^") || !schema.pattern.endsWith("$")) {
    throw new Error("JSON Schema string pattern must be anchored with ^ and $");
  }
  let expression;
  try {
    expression = new RegExp(schema.pattern, "u");
  } catch (error) {
    throw new Error(`Invalid JSON Schema string pattern: ${messageOf(error)}`);
  }
  if (["\"", "\\", "\n", "\r", "\t"].some((c) => expression.test(c))) {
    throw new Error("JSON Schema string pattern cannot admit JSON escapes or control characters");
  }
  return `"${schema.pattern.slice(1, -1)}"`;
}

function arrayPatternOf(schema, maxDepth, ws, depth) {
  if (!schema.items || typeof schema.items !== "object" || Array.isArray(schema.items)) {
    throw new Error("JSON Schema arrays require one object-valued items schema");
  }
  const min = schema.minItems === undefined ? 0 : countOf(schema.minItems, "minItems");
  const max = schema.maxItems === undefined ? null : countOf(schema.maxItems, "maxItems");
  if (max !== null && max < min) throw new Error("JSON Schema maxItems is below minItems");
  const item = schemaPatternOf(schema.items, maxDepth, ws, depth + 1);
  let body;
  if (max !== null) {
    const options = [];
    for (let n = min; n <= max; n += 1) options.push(listOf(item, ws, n));
    body = anyOf(options);
  } else if (min > 0) {
    body = `${listOf(item, ws, min)}(?:${ws},${ws}${item})*`;
  } else {
    body = `(?:${item}(?:${ws},${ws}${item})*)?`;
  }
  return `\\[${ws}${body}${ws}\\]`;
}

function objectPatternOf(schema, maxDepth, ws, depth) {
  if (schema.additionalProperties !== false) {
    throw new Error("JSON Schema objects require additionalProperties: false");
  }
  const properties = schema.properties;
  if (!properties || typeof properties !== "object" || Array.isArray(properties)) {
    throw new Error("JSON Schema objects require a properties object");
  }
  const entries = Object.entries(properties);
  if (entries.length > MAX_SCHEMA_PROPERTIES) {
    throw new Error(`JSON Schema objects support at most ${MAX_SCHEMA_PROPERTIES} properties`);
  }
  const required = schema.required;
  if (!Array.isArray(required) || required.some((key) => typeof key !== "string")) {
    throw new Error("JSON Schema objects require a string-valued required array");
  }
  const requiredSet = new Set(required);
  if (requiredSet.size !== entries.length || entries.some(([key]) => !requiredSet.has(key))) {
    throw new Error("JSON Schema constrained objects require every declared property");
  }
  const members = entries.map(([key, value]) =>
    `${literalOf(key)}${ws}:${ws}${schemaPatternOf(value, maxDepth, ws, depth + 1)}`);
  return `\\{${ws}${members.join(`${ws},${ws}`)}${ws}\\}`;
}

function schemaPatternOf(schema, maxDepth, ws, depth) {
  if (!schema || typeof schema !== "object" || Array.isArray(schema)) {
    throw new Error("JSON Schema constraint must be an object schema");
  }
  const unsupported = Object.keys(schema).filter((key) => !SCHEMA_KEYWORDS.has(key));
  if (unsupported.length > 0) throw new Error(`Unsupported JSON Schema keywords: ${unsupported.join(", ")}`);
  if ("const" in schema) return literalOf(schema.const);
  if (Array.isArray(schema.enum)) {
    if (schema.enum.length === 0) throw new Error("JSON Schema enum must not be empty");
    return anyOf(schema.enum.map(literalOf));
  }
  const alternatives = schema.oneOf !== undefined ? schema.oneOf : schema.anyOf;
  if (Array.isArray(alternatives)) {
    if (alternatives.length === 0) throw new Error("JSON Schema alternatives must not be empty");
    return anyOf(alternatives.map((item) => schemaPatternOf(item, maxDepth, ws, depth)));
  }
  if (depth > maxDepth) throw new Error(`JSON Schema exceeds maxDepth ${maxDepth}`);
  const types = Array.isArray(schema.type) ? schema.type : [schema.type];
  if (types.length === 0 || types[0] === undefined) {
    throw new Error("JSON Schema constraint requires type, const, enum, oneOf, or anyOf");
  }
  return anyOf(types.map((type) => {
    switch (type) {
      case "string": return stringPatternOf(schema);
      case "number": return JSON_NUMBER;
      case "integer": return JSON_INTEGER;
      case "boolean": return "(?:true|false)";
      case "null": return "null";
      case "array": return arrayPatternOf(schema, maxDepth, ws, depth);
      case "object": return objectPatternOf(schema, maxDepth, ws, depth);
      default: throw new Error(`Unsupported JSON Schema type: ${String(type)}`);
    }
  }));
}

// ------------------------------------------------- schema output checking
function jsonEqual(a, b) {
  if (a === b) return true;
  if (typeof a !== typeof b || a === null || b === null || typeof a !== "object") return false;
  if (Array.isArray(a) !== Array.isArray(b)) return false;
  if (Array.isArray(a)) return a.length === b.length && a.every((x, k) => jsonEqual(x, b[k]));
  const ka = Object.keys(a);
  const kb = Object.keys(b);
  return ka.length === kb.length && ka.every((k) => Object.prototype.hasOwnProperty.call(b, k) && jsonEqual(a[k], b[k]));
}

function typeMatches(type, value) {
  switch (type) {
    case "string": return typeof value === "string";
    case "number": return typeof value === "number";
    case "integer": return typeof value === "number" && Number.isInteger(value);
    case "boolean": return typeof value === "boolean";
    case "null": return value === null;
    case "array": return Array.isArray(value);
    case "object": return value !== null && typeof value === "object" && !Array.isArray(value);
    default: return false;
  }
}

// every failed keyword of value against schema, as "path message" strings
function schemaErrors(schema, value, path, out) {
  if ("const" in schema && !jsonEqual(schema.const, value)) out.push(`${path} must be equal to constant`);
  if (Array.isArray(schema.enum) && !schema.enum.some((x) => jsonEqual(x, value))) {
    out.push(`${path} must be equal to one of the allowed values`);
  }
  if (Array.isArray(schema.anyOf) && !schema.anyOf.some((s) => schemaErrors(s, value, path, []).length === 0)) {
    out.push(`${path} must match a schema in anyOf`);
  }
  if (Array.isArray(schema.oneOf)) {
    const n = schema.oneOf.filter((s) => schemaErrors(s, value, path, []).length === 0).length;
    if (n !== 1) out.push(`${path} must match exactly one schema in oneOf`);
  }
  if (schema.type !== undefined) {
    const types = Array.isArray(schema.type) ? schema.type : [schema.type];
    if (!types.some((t) => typeMatches(t, value))) out.push(`${path} must be ${types.join(",")}`);
  }
  if (typeof value === "string" && typeof schema.pattern === "string" && !new RegExp(schema.pattern, "u").test(value)) {
    out.push(`${path} must match pattern "${schema.pattern}"`);
  }
  if (Array.isArray(value)) {
    if (schema.minItems !== undefined && value.length < schema.minItems) {
      out.push(`${path} must NOT have fewer than ${schema.minItems} items`);
    }
    if (schema.maxItems !== undefined && value.length > schema.maxItems) {
      out.push(`${path} must NOT have more than ${schema.maxItems} items`);
    }
    if (schema.items && typeof schema.items === "object") {
      value.forEach((x, k) => schemaErrors(schema.items, x, `${path}/${k}`, out));
    }
  }
  if (value !== null && typeof value === "object" && !Array.isArray(value)) {
    const props = schema.properties && typeof schema.properties === "object" ? schema.properties : {};
    if (Array.isArray(schema.required)) {
      for (const key of schema.required) {
        if (!Object.prototype.hasOwnProperty.call(value, key)) out.push(`${path} must have required property '${key}'`);
      }
    }
    if (schema.additionalProperties === false) {
      for (const key of Object.keys(value)) {
        if (!Object.prototype.hasOwnProperty.call(props, key)) out.push(`${path} must NOT have additional properties`);
      }
    }
    for (const [key, sub] of Object.entries(props)) {
      if (Object.prototype.hasOwnProperty.call(value, key) && sub && typeof sub === "object") {
        schemaErrors(sub, value[key], `${path}/${key}`, out);
      }
    }
  }
  return out;
}

// ------------------------------------------------------------- front end
/* A constraint's byte-level DFA and its final-text check:
 * { dfa: {stateCount, next, finals, initial}, validateOutput(text) }. Every
 * failure is thrown as the reference throws it: pattern and option errors
 * with their own message from the JSON front ends, and, for what the
 * automaton cannot express, "Unsupported generation constraint: <reason>"
 * (constraints.ts:217-219). */
function compileConstraintTables(constraint) {
  if (!constraint || typeof constraint !== "object") throw new Error("Unsupported generation constraint: not an object");
  const build = (source, maxNodes) => {
    try {
      return compileRegexToByteDfa(source, maxNodes ? { maxStates: maxNodes } : undefined);
    } catch (error) {
      throw new Error(`Unsupported generation constraint: ${messageOf(error)}`);
    }
  };
  if (constraint.type === "regex") {
    const pattern = constraint.pattern;
    if (typeof pattern !== "string" || pattern.length === 0) throw new Error("Regex constraint pattern must not be empty");
    const dfa = build(pattern);
    return {
      dfa,
      validateOutput(text) {
        const match = new RegExp(pattern, "u").exec(text);
        if (!match || match.index !== 0 || match[0].length !== text.length) {
          throw new Error("Generated output does not match its regex constraint");
        }
      },
    };
  }
  {
    // every other type takes the schema route, as the reference's does
    const maxDepth = depthOf(constraint.maxDepth);
    const ws = whitespaceOf(constraint.whitespace === undefined ? "compact" : constraint.whitespace);
    if (constraint.type === "json") {
      return {
        dfa: build(`${ws}${valueOf(maxDepth, ws)}${ws}`, JSON_GRAMMAR_MAX_NODES),
        validateOutput(text) { JSON.parse(text); },
      };
    }
    if (constraint.type === "json-object") {
      return {
        dfa: build(`${ws}${objectOf(valueOf(Math.max(0, maxDepth - 1), ws), ws)}${ws}`, JSON_GRAMMAR_MAX_NODES),
        validateOutput(text) {
          const value = JSON.parse(text);
          if (!value || typeof value !== "object" || Array.isArray(value)) {
            throw new Error("Generated JSON must be an object");
          }
        },
      };
    }
    const schema = constraint.schema;
    const source = `${ws}${schemaPatternOf(schema, maxDepth, ws, 0)}${ws}`;
    const dfa = build(source, JSON_GRAMMAR_MAX_NODES);
    return {
      dfa,
      validateOutput(text) {
        const value = JSON.parse(text);
        const errors = schemaErrors(schema, value, "data", []);
        if (errors.length) throw new Error(`Generated JSON does not satisfy its schema: ${errors.join("; ")}`);
      },
    };
  }
}

module.exports = {
  compileConstraintTables,
  schemaErrors,
  DEFAULT_JSON_DEPTH,
  MAX_JSON_DEPTH,
  JSON_STRING,
  JSON_NUMBER,
  JSON_INTEGER,
};
