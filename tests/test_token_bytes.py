"""The token byte table (src/runtime/gemma-tokenizer.ts:346-360) and its
on-disk form, without a GPU: a synthetic tokenizer.json with byte-fallback
pieces, SentencePiece spaces, multi-byte text, special and ordinary added
tokens and holes in the id range; known answers from the reference's rule,
the Python and Node implementations producing the same table and the same
file, and the file round trip. The real Gemma tokenizer.json is not in this
tree (the reference ships it as a missing blob)."""
import json
import os
import shutil
import subprocess

import pytest

from gsample import vocab as gv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def synthetic_tokenizer(path, unigram=False):
    pieces = {"<pad>": 0, "<eos>": 1, "<bos>": 2, "<unk>": 3}
    for b in range(256):
        pieces[f"<0x{b:02X}>"] = 4 + b
    words = ["▁the", "▁▁", "é", "▁café", "שלום", "😀", "<0xff>", "<0x0A>x", "▁", "a▁b▁", "<0xZZ>"]
    for k, w in enumerate(words):
        pieces[w] = 300 + k
    doc = {"model": {}, "added_tokens": [
        {"id": 1, "content": "<eos>", "special": True},
        {"id": 50, "content": "<end_of_turn>", "special": True},
        {"id": 100, "content": "<|channel>", "special": True},
        {"id": 400, "content": "<custom>", "special": False},
    ]}
    if unigram:
        size = 401
        vocab = [[f"<unused{k}>", 0.0] for k in range(size)]
        for p, i in pieces.items():
            vocab[i] = [p, -1.0]
        doc["model"] = {"type": "Unigram", "vocab": vocab}
    else:
        doc["model"] = {"type": "BPE", "vocab": pieces}
    with open(path, "w", encoding="utf-8") as f:
        json.dump(doc, f, ensure_ascii=False)
    return pieces


def test_known_answers(tmp_path):
    p = tmp_path / "tokenizer.json"
    synthetic_tokenizer(p)
    t = gv.load_tokenizer_json(str(p))
    assert len(t) == 401                      # largest id 400, plus one
    assert t[1] is None and t[50] is None and t[100] is None  # special
    assert t[0] == b"<pad>" and t[2] == b"<bos>"             # not special in this file: their text
    assert t[4 + 0x0A] == b"\n" and t[4 + 0xFF] == b"\xff"    # byte fallback
    assert t[300] == b" the" and t[301] == b"  " and t[308] == b" "
    assert t[302] == "é".encode() and t[303] == " café".encode()
    assert t[304] == "שלום".encode() and t[305] == "😀".encode()
    assert t[306] == b"<0xff>"                # lower-case hex is text
    assert t[307] == b"<0x0A>x" and t[310] == b"<0xZZ>"
    assert t[309] == b"a b "
    assert t[311] is None and t[399] is None  # ids the vocabulary does not name
    assert t[400] == b"<custom>"             # an ordinary added token


def test_unigram_list_gives_the_same_table(tmp_path):
    a, b = tmp_path / "bpe.json", tmp_path / "uni.json"
    synthetic_tokenizer(a)
    synthetic_tokenizer(b, unigram=True)
    ta, tb = gv.load_tokenizer_json(str(a)), gv.load_tokenizer_json(str(b))
    same = [i for i in range(len(ta)) if ta[i] is not None]
    assert all(ta[i] == tb[i] for i in same)
    assert tb[311] == b"<unused311>"         # named in the Unigram list


def test_file_round_trip_and_csr(tmp_path):
    p = tmp_path / "tokenizer.json"
    synthetic_tokenizer(p)
    t = gv.load_tokenizer_json(str(p))
    f = tmp_path / "vocab.gsvb"
    gv.write_token_byte_table(str(f), t)
    assert gv.read_token_byte_table(str(f)) == t
    csr = gv.vocab_bytes(t)
    assert csr.vocabulary_size == len(t)
    assert csr.token_bytes(300) == b" the" and csr.token_bytes(1) is None
    bad = tmp_path / "bad.gsvb"
    bad.write_bytes(f.read_bytes()[:-1])
    with pytest.raises(ValueError, match="size does not match"):
        gv.read_token_byte_table(str(bad))


def test_node_and_python_agree(tmp_path):
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    p = tmp_path / "tokenizer.json"
    synthetic_tokenizer(p)
    f_py, f_js = tmp_path / "py.gsvb", tmp_path / "js.gsvb"
    gv.write_token_byte_table(str(f_py), gv.load_tokenizer_json(str(p)))
    script = (
        "const tb = require(process.argv[1]);"
        "const t = tb.loadTokenizerJson(process.argv[2]);"
        "tb.writeTokenByteTable(process.argv[3], t);"
        "const back = tb.readTokenByteTable(process.argv[4]);"
        "if (back.length !== t.length || back.some((b, i) => (b === null) !== (t[i] === null) ||"
        " (b && Buffer.compare(Buffer.from(b), Buffer.from(t[i])) !== 0))) throw new Error('mismatch');"
    )
    mod = os.path.join(ROOT, "gemma-webgpu-engine_amd", "node", "token-bytes.js")
    subprocess.run([node, "-e", script, mod, str(p), str(f_js), str(f_py)], check=True, timeout=60)
    assert f_js.read_bytes() == f_py.read_bytes()
