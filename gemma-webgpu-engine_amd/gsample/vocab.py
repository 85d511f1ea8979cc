"""The Gemma token byte table and its on-disk form (the Python side of
node/token-bytes.js; the two read and write the same files).

create_token_byte_table follows createTokenByteTable
(src/runtime/gemma-tokenizer.ts:346-360): vocabulary size = largest id + 1;
special ids and ids the vocabulary does not name are None; a byte-fallback
piece "<0xHH>" (upper-case hex) is that one byte; any other piece is the
UTF-8 of its text with every "▁" (the SentencePiece space) turned into
" ". read_tokenizer_json reads a Hugging Face tokenizer.json: the model's
vocab (piece -> id, or a Unigram list whose index is the id) plus
added_tokens, the special ids being the added tokens marked special.

On disk ("GSVB" version 1, little-endian): magic, u32 version, u32 V,
u32 flags (0), u64 total bytes, u8 present[V], u32 offsets[V + 1], bytes.
"""
from __future__ import annotations

import json
import re
import struct
from typing import Dict, Iterable, List, Optional, Tuple

import numpy as np

from .constraint import VocabBytes

_BYTE_FALLBACK = re.compile(r"^<0x([0-9A-F]{2})>$")
_MAGIC = b"GSVB"


def create_token_byte_table(vocabulary: Dict[str, int], special_ids: Iterable[int]) -> List[Optional[bytes]]:
    size = max(vocabulary.values(), default=-1) + 1
    table: List[Optional[bytes]] = [None] * size
    special = set(special_ids)
    for piece, tid in vocabulary.items():
        if tid in special:
            continue
        m = _BYTE_FALLBACK.match(piece)
        table[tid] = bytes([int(m.group(1), 16)]) if m else piece.replace("▁", " ").encode("utf-8")
    return table


def read_tokenizer_json(path: str) -> Tuple[Dict[str, int], List[int]]:
    with open(path, "r", encoding="utf-8") as f:
        doc = json.load(f)
    vocab = (doc.get("model") or {}).get("vocab")
    vocabulary: Dict[str, int] = {}
    if isinstance(vocab, list):
        for tid, entry in enumerate(vocab):
            vocabulary[entry[0]] = tid
    elif isinstance(vocab, dict):
        vocabulary.update(vocab)
    else:
        raise ValueError("tokenizer.json has no model vocab")
    special = []
    for t in doc.get("added_tokens") or []:
        vocabulary[t["content"]] = t["id"]
        if t.get("special"):
            special.append(t["id"])
    return vocabulary, special


def load_tokenizer_json(path: str) -> List[Optional[bytes]]:
    vocabulary, special = read_tokenizer_json(path)
    return create_token_byte_table(vocabulary, special)


def write_token_byte_table(path: str, table: List[Optional[bytes]]) -> None:
    V = len(table)
    present = bytes(1 if b is not None else 0 for b in table)
    offsets = np.zeros(V + 1, dtype="<u4")
    chunks = []
    at = 0
    for i, b in enumerate(table):
        offsets[i] = at
        if b:
            chunks.append(b)
            at += len(b)
    offsets[V] = at
    with open(path, "wb") as f:
        f.write(_MAGIC + struct.pack("<IIIQ", 1, V, 0, at))
        f.write(present)
        f.write(offsets.tobytes())
        f.write(b"".join(chunks))


def read_token_byte_table(path: str) -> List[Optional[bytes]]:
    with open(path, "rb") as f:
        buf = f.read()
    if len(buf) < 24 or buf[:4] != _MAGIC:
        raise ValueError("not a GSVB token byte table")
    version, V, _flags, total = struct.unpack_from("<IIIQ", buf, 4)
    if version != 1:
        raise ValueError(f"unsupported GSVB version {version}")
    p_at, o_at = 24, 24 + V
    b_at = o_at + 4 * (V + 1)
    if len(buf) != b_at + total:
        raise ValueError("GSVB size does not match its header")
    offsets = np.frombuffer(buf, dtype="<u4", count=V + 1, offset=o_at)
    return [bytes(buf[b_at + int(offsets[i]):b_at + int(offsets[i + 1])]) if buf[p_at + i] else None
            for i in range(V)]


def vocab_bytes(table: List[Optional[bytes]]) -> VocabBytes:
    """The CSR the engine's gs_set_vocab takes."""
    return VocabBytes.from_tokens(table)
