"use strict";
/*
 * The decode loop around the sampling stage (src/runtime/gemma-session.ts:
 * 404-440, 659-782, 1305-1345): what each generated position samples, and
 * how the history, the RNG, the constraint and the reasoning channel move.
 *
 * Per position, in the reference's order (:671-704):
 *   - a forced reasoning-prefix token ([START_CHANNEL, ...encodeText(
 *     "thought\n")] with requireReasoning), no draw;
 *   - inside a required reasoning channel: END_CHANNEL once 64 content
 *     tokens are out, else a draw over the text tokens (END_CHANNEL allowed
 *     from 16 content tokens on; maskReasoningLogits, :1331-1345);
 *   - with an active constraint: selectConstrainedToken (legal ids, extra
 *     START_CHANNEL while the channel may still open, termination ids while
 *     accepting; :1305-1329);
 *   - a draw over the raw logits unless the row is GPU-greedy (T 0, no
 *     penalties: usesGemmaGpuGreedy), whose token is the model's argmax
 *     prediction.
 * An end token (EOS 1, 50, 106) or a stop id ends the loop before the token
 * is kept (:710-717). The token then updates the channel state, goes through
 * the constraint (acceptToken of its bytes; a token without bytes throws
 * "Constraint selected non-text token <id>"), joins the output and the
 * history, which starts as the prompt (:666, :741). One SeededRandom(seed)
 * serves the whole request and draws once per non-greedy sample, so the
 * draw count, not the position, is the RNG index (forced tokens take none).
 * Logits come from the caller's model (the network is not part of this
 * engine); sampling runs on the GPU through sampleToken /
 * selectConstrainedToken / tokenLogProbability.
 */
const { resolveGemmaGenerationConfig, usesGemmaGpuGreedy } = require("./generation-config");
const { SeededRandom, sampleToken, tokenLogProbability } = require("./sampling");
const { compileGenerationConstraint, maskConstraintLogits, selectConstrainedToken } = require("./constraints");
const { TokenByteTrie } = require("./token-byte-trie");
const { EOS_TOKEN_IDS, GEMMA_START_CHANNEL_TOKEN_ID, GEMMA_END_CHANNEL_TOKEN_ID } = require("./token-bytes");

const GEMMA_REQUIRED_REASONING_TOKENS = 16;      // gemma-session.ts:124
const GEMMA_MAX_REQUIRED_REASONING_TOKENS = 64;  // :125

/* The text tokens of a vocabulary (tokenBytes not null), and the reasoning
 * mask over them: logits of other ids -inf, END_CHANNEL kept when allowed. */
class ReasoningMask {
  constructor(tokenizer, vocabularySize) {
    const ids = [];
    for (let id = 0; id < vocabularySize; id += 1) if (tokenizer.tokenBytes(id) !== null) ids.push(id);
    this.textIds = ids;
  }
  apply(rawLogits, allowEndChannel) {
    const keep = allowEndChannel ? this.textIds.concat([GEMMA_END_CHANNEL_TOKEN_ID]) : this.textIds;
    return maskConstraintLogits(rawLogits, keep, []);
  }
}

function requiredLogits(output) {
  if (!output || !output.logits) throw new Error("Gemma model output is missing logits");
  return output.logits;
}

/* The text of the answer: the UTF-8 of the generated tokens' bytes outside
 * the reasoning channel (START_CHANNEL .. END_CHANNEL). A tokenizer with
 * decodeAnswer(tokenIds) decides instead. */
function answerText(tokenizer, tokenIds) {
  if (typeof tokenizer.decodeAnswer === "function") return tokenizer.decodeAnswer(tokenIds);
  const parts = [];
  let inChannel = false;
  for (const id of tokenIds) {
    if (id === GEMMA_START_CHANNEL_TOKEN_ID) { inChannel = true; continue; }
    if (id === GEMMA_END_CHANNEL_TOKEN_ID) { inChannel = false; continue; }
    if (inChannel) continue;
    const b = tokenizer.tokenBytes(id);
    if (b) parts.push(Buffer.from(b));
  }
  return Buffer.concat(parts).toString("utf8");
}

/*
 * generate(args) -> Promise<result>
 *   args.promptTokenIds  the prompt (the history's start)
 *   args.model           { first: output, evaluateToken(token, outputMode): output | Promise }
 *                        output = { logits?: Float32Array, prediction?: { token } }; first is
 *                        the output after the prompt. outputMode is "logits" or "greedy"
 *                        (the reference's GPU-greedy readback, which may give only prediction)
 *   args.tokenizer       { vocabularySize, tokenBytes(id), encodeText?(text), decodeAnswer?(ids) }
 *   args.options         GemmaGenerationOptions: decoding fields, constraint,
 *                        requireReasoning, captureTokenLogProbabilities, onToken
 *   args.thinking        the input enables thinking (usesGemmaThinking)
 * result: { tokenIds, stoppedOnEndToken, stoppedOnStopToken, draws,
 *           tokenLogProbabilities, reasoningLogProbability, answerLogProbability,
 *           reasoningTokenCount, answerTokenCount, text }
 */
async function generate(args) {
  const options = Object.assign({}, args.options || {});
  const { constraint, onToken } = options;
  const requireReasoning = options.requireReasoning === true;
  const captureTokenLogProbabilities = options.captureTokenLogProbabilities === true;
  delete options.constraint;
  delete options.onToken;
  delete options.requireReasoning;
  delete options.captureTokenLogProbabilities;
  delete options.signal;
  const config = resolveGemmaGenerationConfig(options);
  const thinking = args.thinking === true;
  if (requireReasoning && !thinking) throw new Error("Required reasoning needs enableThinking");
  const tokenizer = args.tokenizer;
  const compiled = constraint
    ? (typeof constraint.legalTokenIds === "function" ? constraint : compileGenerationConstraint(constraint))
    : null;
  const trie = compiled ? (args.trie || new TokenByteTrie(tokenizer)) : null;
  let constraintActive = compiled !== null;
  let allowReasoningChannel = thinking;
  let inReasoningChannel = false;
  let reasoningContentTokens = 0;
  let forcedReasoningPrefix = [];
  if (requireReasoning) {
    if (typeof tokenizer.encodeText !== "function") throw new Error("requireReasoning needs tokenizer.encodeText");
    forcedReasoningPrefix = [GEMMA_START_CHANNEL_TOKEN_ID].concat(Array.from(tokenizer.encodeText("thought\n")));
  }
  const outputMode = compiled || requireReasoning || captureTokenLogProbabilities || !usesGemmaGpuGreedy(config)
    ? "logits" : "greedy";
  const maxNewTokens = config.maxNewTokens;
  const reasoningMask = requireReasoning ? new ReasoningMask(tokenizer, tokenizer.vocabularySize) : null;

  let output = args.model.first;
  const generated = [];
  const logProbabilities = [];
  let reasoningLogProbability = 0;
  let answerLogProbability = 0;
  let reasoningTokenCount = 0;
  let answerTokenCount = 0;
  const history = Array.from(args.promptTokenIds || []);
  const random = new SeededRandom(config.seed);
  const draw = () => random.next();
  const customStopTokens = new Set(config.stopTokenIds);
  const endTokens = new Set(tokenizer.endTokenIds || EOS_TOKEN_IDS);
  let stoppedOnEndToken = false;
  let stoppedOnStopToken = false;
  for (let index = 0; index < maxNewTokens; index += 1) {
    let token = output && output.prediction ? output.prediction.token : 0;
    if (outputMode === "greedy" && !(output && output.prediction)) {
      throw new Error("Gemma greedy mode produced no prediction");
    }
    if (index < forcedReasoningPrefix.length) {
      token = forcedReasoningPrefix[index];
    } else if (requireReasoning && inReasoningChannel) {
      if (reasoningContentTokens >= GEMMA_MAX_REQUIRED_REASONING_TOKENS) {
        token = GEMMA_END_CHANNEL_TOKEN_ID;
      } else {
        const logits = reasoningMask.apply(requiredLogits(output),
          reasoningContentTokens >= GEMMA_REQUIRED_REASONING_TOKENS);
        token = sampleToken(logits, history, config, draw);
      }
    } else if (compiled && constraintActive) {
      token = selectConstrainedToken({
        logits: requiredLogits(output),
        history,
        config,
        random,
        constraint: compiled,
        trie,
        customStopTokens,
        additionalLegalTokens: allowReasoningChannel ? [GEMMA_START_CHANNEL_TOKEN_ID] : [],
      });
    } else if (requireReasoning || !usesGemmaGpuGreedy(config) || (compiled && !constraintActive)) {
      token = sampleToken(requiredLogits(output), history, config, draw);
    }
    if (endTokens.has(token)) {
      stoppedOnEndToken = true;
      break;
    }
    if (customStopTokens.has(token)) {
      stoppedOnStopToken = true;
      break;
    }
    const logProbability = captureTokenLogProbabilities ? tokenLogProbability(requiredLogits(output), token) : null;
    const startsReasoningChannel = allowReasoningChannel && token === GEMMA_START_CHANNEL_TOKEN_ID;
    allowReasoningChannel = false;
    if (startsReasoningChannel) {
      constraintActive = false;
      inReasoningChannel = true;
    } else if (compiled && constraintActive) {
      const bytes = tokenizer.tokenBytes(token);
      if (!bytes) throw new Error(`Constraint selected non-text token ${token}`);
      compiled.acceptToken(bytes);
    }
    generated.push(token);
    if (logProbability !== null) {
      logProbabilities.push(logProbability);
      if (inReasoningChannel && token !== GEMMA_END_CHANNEL_TOKEN_ID) {
        reasoningLogProbability += logProbability;
        reasoningTokenCount += 1;
      } else if (!startsReasoningChannel && token !== GEMMA_END_CHANNEL_TOKEN_ID) {
        answerLogProbability += logProbability;
        answerTokenCount += 1;
      }
    }
    history.push(token);
    if (inReasoningChannel && token === GEMMA_END_CHANNEL_TOKEN_ID) {
      inReasoningChannel = false;
      if (compiled) constraintActive = true;
    } else if (inReasoningChannel && index >= forcedReasoningPrefix.length) {
      reasoningContentTokens += 1;
    }
    if (onToken) await onToken(token, generated.slice());
    if (index + 1 < maxNewTokens) output = await args.model.evaluateToken(token, outputMode);
  }
  if (compiled && !compiled.accepting) {
    throw new Error("Max tokens reached before the generation constraint completed; increase maxNewTokens");
  }
  const text = answerText(tokenizer, generated);
  if (compiled) compiled.validateFinal(text);
  return {
    tokenIds: generated,
    stoppedOnEndToken,
    stoppedOnStopToken,
    draws: random.draws,
    tokenLogProbabilities: logProbabilities,
    reasoningLogProbability,
    answerLogProbability,
    reasoningTokenCount,
    answerTokenCount,
    text,
  };
}

module.exports = {
  generate,
  answerText,
  ReasoningMask,
  GEMMA_REQUIRED_REASONING_TOKENS,
  GEMMA_MAX_REQUIRED_REASONING_TOKENS,
};
