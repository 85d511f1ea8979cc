"""The token byte table carried into the GPU masker at the Gemma vocabulary
size (src/runtime/gemma-tokenizer.ts:346-360, src/runtime/token-byte-trie.ts:20-40,
src/runtime/constraints.ts:56-92).

A synthetic tokenizer.json of 262144 ids (the real Gemma file is a missing
blob in the reference) holds what the reference's byte rule distinguishes:
special added tokens (EOS 1 / 50 / 106, channel 100 / 101, <unusedN>),
byte-fallback pieces "<0xHH>", pieces with "▁" (SentencePiece spaces),
multi-byte text (2-, 3- and 4-byte UTF-8), different pieces with the same
bytes ("▁x" and " x"), lower-case "<0xhh>" text, and ids no piece names.
Node (token-bytes.js) and Python (vocab.py) each load it and write the GSVB
file; the two files must be byte-identical. The table read back goes through
gs_set_vocab; regex and JSON constraints compiled by the Node compiler go
through gs_set_dfa; gs_build_masks' masks for the states along a document
are compared with the oracle's definitional walk over the same table, and
rows sampled under those masks (termination ids legal only when accepting)
with the oracle on logits masked by the oracle's masks."""
import json
import os
import subprocess

import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE_DIR = os.path.join(ROOT, "gemma-webgpu-engine_amd", "node")
V = 262144
EOS = (1, 50, 106)

# segments pieces are built from: ASCII letters, digits, JSON punctuation,
# the SentencePiece space, and 2-, 3- and 4-byte UTF-8 characters
_SEGMENTS = (list("abcdefghijklmnopqrstuvwxyz") + list("0123456789") + list('{}[]:,"-.+e') +
             ["▁", "▁", "é", "ü", "ñ", "ש", "ל", "中", "文", "😀", "🙂", "\\n", "true", "null", "fals"])
# "<0xhh>" pieces whose lower-case hex differs from every byte-fallback piece
_LOWER_HEX = [f"<0x{b:02x}>" for b in range(256) if f"{b:02x}" != f"{b:02X}"]


def gemma_like_tokenizer(path, seed=2024):
    rng = np.random.default_rng(seed)
    vocab = {"<pad>": 0, "<bos>": 2, "<unk>": 3}
    added = [{"id": 1, "content": "<eos>", "special": True},
             {"id": 2, "content": "<bos>", "special": True},
             {"id": 50, "content": "<end_of_turn>", "special": True},
             {"id": 100, "content": "<|channel>", "special": True},
             {"id": 101, "content": "<channel|>", "special": True},
             {"id": 106, "content": "<turn|>", "special": True}]
    specials = {1, 2, 50, 100, 101, 106}
    for i in range(4, 300):
        if i not in specials:
            added.append({"id": i, "content": f"<unused{i}>", "special": True})
    for b in range(256):
        vocab[f"<0x{b:02X}>"] = 300 + b
    seen = set(vocab)
    nxt = 556
    while nxt < V:
        if nxt % 997 == 0:           # an id no piece names
            nxt += 1
            continue
        n = int(rng.integers(1, 7))
        piece = "".join(_SEGMENTS[int(k)] for k in rng.integers(0, len(_SEGMENTS), n))
        if nxt % 613 == 0 and piece.startswith("▁"):
            piece = " " + piece[1:]   # the same bytes as a "▁" piece may have
        if nxt % 877 == 0 and nxt // 877 < len(_LOWER_HEX):
            piece = _LOWER_HEX[nxt // 877]  # lower-case hex: text, not a byte
        if piece in seen:
            continue
        seen.add(piece)
        vocab[piece] = nxt
        nxt += 1
    doc = {"model": {"type": "BPE", "vocab": vocab}, "added_tokens": added}
    with open(path, "w", encoding="utf-8") as f:
        json.dump(doc, f, ensure_ascii=False)


_NODE_SCRIPT = r"""
const tb = require(process.argv[1] + "/token-bytes.js");
const { compileGenerationConstraint } = require(process.argv[1] + "/constraints.js");
const [tokPath, gsvbPath, dfaPath] = process.argv.slice(2);
const table = tb.loadTokenizerJson(tokPath);
tb.writeTokenByteTable(gsvbPath, table);
const out = {};
const specs = {
  regex: { type: "regex", pattern: "(?:[a-z]+|é|ü|中文|😀| )+(?:[0-9]+)?" },
  json: { type: "json", maxDepth: 3, whitespace: "compact" },
};
for (const [name, spec] of Object.entries(specs)) {
  const c = compileGenerationConstraint(spec);
  out[name] = { next: Array.from(c.dfa.next), finals: Array.from(c.dfa.finals), initial: c.dfa.initial,
                states: c.dfa.stateCount };
}
require("fs").writeFileSync(dfaPath, JSON.stringify(out));
"""

_DOCS = {
    "regex": "café über 中文 \U0001F600 abc 123",
    "json": '{"k": [1, "a\\néש\U0001F600", null], "x": -23.5e+1, "y": {"b": true}}',
}


@pytest.fixture(scope="module")
def loaded(tmp_path_factory, node, oracle):
    from gsample import vocab as gv

    d = tmp_path_factory.mktemp("tok")
    tok, js_gsvb, py_gsvb, dfa_json = (str(d / n) for n in ("tokenizer.json", "js.gsvb", "py.gsvb", "dfa.json"))
    gemma_like_tokenizer(tok)
    subprocess.run([node, "-e", _NODE_SCRIPT, NODE_DIR, tok, js_gsvb, dfa_json], check=True, timeout=300)
    table = gv.load_tokenizer_json(tok)
    gv.write_token_byte_table(py_gsvb, table)
    with open(js_gsvb, "rb") as a, open(py_gsvb, "rb") as b:
        assert a.read() == b.read(), "Node and Python GSVB files differ"
    back = gv.read_token_byte_table(js_gsvb)
    assert back == table
    with open(dfa_json) as f:
        dfas = json.load(f)
    return gv.vocab_bytes(back), back, dfas


def test_byte_rule_known_answers(loaded):
    """createTokenByteTable's rule on pieces of each kind (gemma-tokenizer.ts:346-360)."""
    csr, table, _ = loaded
    assert len(table) == V and csr.vocabulary_size == V
    for i in (1, 2, 50, 100, 101, 106, 4, 299):
        assert table[i] is None, i                      # special added tokens
    assert table[0] == b"<pad>" and table[3] == b"<unk>"  # in the vocab, not special
    assert table[300 + 0x0A] == b"\n" and table[300 + 0xC3] == b"\xc3" and table[300 + 0xFF] == b"\xff"
    assert table[997] is None and table[997 * 7] is None  # ids no piece names
    texts = [b for b in table[556:] if b]
    assert any(b.startswith(b" ") for b in texts)
    assert any("😀".encode() in b for b in texts) and any("中".encode() in b for b in texts)
    assert not any("▁".encode() in b for b in texts)     # every SentencePiece space became " "


@pytest.mark.parametrize("kind", ["regex", "json"])
def test_masks_and_samples_over_the_loaded_table(sampler, oracle, loaded, kind):
    import torch

    import gsample as gs
    csr, table, dfas = loaded
    spec = dfas[kind]
    S = spec["states"]
    nxt = np.asarray(spec["next"], np.int32).reshape(S, 256)
    finals = np.asarray(spec["finals"], np.uint8)
    viable = oracle.viable_states(nxt, finals)
    # the states along a document the constraint accepts (every byte boundary)
    doc = _DOCS[kind].encode("utf-8")
    states, s = [spec["initial"]], spec["initial"]
    for b in doc:
        s = int(nxt[s, b])
        assert s >= 0 and viable[s], "the document leaves the constraint"
        states.append(s)
    assert finals[s], "the document does not end in an accepting state"
    uniq = sorted(set(states))
    sampler.set_vocab(csr.offsets, csr.data)
    sampler.set_dfa(nxt, finals)
    got = sampler.build_masks(uniq)
    words = got.cpu().numpy().view(np.uint32)
    ref = [oracle.dfa_legal_mask(nxt, viable, csr.offsets, csr.data, st) for st in uniq]
    legal_counts = []
    for i, st in enumerate(uniq):
        assert np.array_equal(words[i], ref[i]), f"{kind} state {st}: GPU mask differs from the oracle's"
        legal_counts.append(int(oracle.mask_bits_to_ids(ref[i], V).size))
    assert max(legal_counts) > 100, legal_counts
    for i, st in enumerate(uniq):           # no special, unnamed or empty id is ever legal
        ids = oracle.mask_bits_to_ids(ref[i], V)
        assert all(table[t] for t in ids[:2000])
    # rows sampled under those masks, EOS ids as termination (legal only when accepting)
    rows = uniq[:16]
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, (len(rows), V)).astype(np.float32)
    cfg = gs.DecodingConfig(temperature=1.0, topK=0, topP=0.95, repetitionWindow=0)
    conf = np.stack([gs.runtime.row_config(cfg, seed=r, mask_slot=r, accepting=bool(finals[st]))
                     for r, st in enumerate(rows)])
    forced = gs.constraint.forced_ids_csr(len(rows), EOS)
    out = sampler.sample(torch.from_numpy(x).cuda(), conf, forced=forced, mask_table=got[: len(rows)])
    ocfg = Decoding(temperature=1.0, topK=0, topP=0.95, minP=0.0, typicalP=1.0, repetitionPenalty=1.0,
                    repetitionWindow=0, frequencyPenalty=0.0, presencePenalty=0.0)
    for r, st in enumerate(rows):
        legal = oracle.mask_bits_to_ids(ref[r], V)
        masked = oracle.mask_logits(x[r], legal, list(EOS) if finals[st] else [])
        t, tr = oracle.sample_token(masked, [], ocfg, oracle.draw(r, 0))
        assert int(out.tokens[r]) == t, (kind, r, int(out.tokens[r]), t, int(out.flags[r]))
        assert not out.flags[r] & gs.GS_FLAG_INDEX_CHECK
        if out.flags[r] & gs.GS_FLAG_EXACT_PATH:
            assert out.probabilities[r] == tr.probability
        else:
            assert abs(out.probabilities[r] - tr.probability) <= 4e-7 * tr.probability
