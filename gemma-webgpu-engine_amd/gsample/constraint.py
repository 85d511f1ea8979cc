"""Constraint side of the sampler: token-byte table, byte-level DFA and the
compiled-constraint object the decode loop drives.

Replaces TokenByteTrie (src/runtime/token-byte-trie.ts:16-40) with a CSR of
token byte strings, and CompiledGenerationConstraint
(src/runtime/constraints.ts:32-113) with a byte-level DFA whose legal-token
sets are bitmasks built on the GPU and cached per DFA state, as the reference
caches legalTokenIds per DFA node (constraints.ts:56-69).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np

from .runtime import GS_FORCED_EXTRA, GS_FORCED_TERMINATION, GSampleError, Sampler

GEMMA_END_TOKEN_IDS = (1, 50, 106)         # src/runtime/gemma-tokenizer.ts:17
GEMMA_START_CHANNEL_TOKEN_ID = 100         # src/runtime/gemma-tokenizer.ts:18


class VocabBytes:
    """Token id -> UTF-8 bytes as a CSR (offsets[V+1], data). None / b"" = no bytes."""

    def __init__(self, offsets: np.ndarray, data: np.ndarray):
        self.offsets = np.ascontiguousarray(offsets, dtype=np.int64)
        self.data = np.ascontiguousarray(data, dtype=np.uint8)

    @property
    def vocabulary_size(self) -> int:
        return int(self.offsets.size - 1)

    @classmethod
    def from_tokens(cls, tokens: Sequence[Optional[bytes]]) -> "VocabBytes":
        offsets = np.zeros(len(tokens) + 1, dtype=np.int64)
        chunks = []
        for i, t in enumerate(tokens):
            b = b"" if t is None else (t.encode("utf-8") if isinstance(t, str) else bytes(t))
            chunks.append(b)
            offsets[i + 1] = offsets[i] + len(b)
        data = np.frombuffer(b"".join(chunks), dtype=np.uint8).copy() if offsets[-1] else np.zeros(0, np.uint8)
        return cls(offsets, data)

    def token_bytes(self, token_id: int) -> Optional[bytes]:
        a, b = int(self.offsets[token_id]), int(self.offsets[token_id + 1])
        return bytes(self.data[a:b]) if b > a else None


class ByteDfa:
    """A DFA over bytes: next[s][b] (-1 = no edge), finals[s], initial state."""

    def __init__(self, next_table: np.ndarray, finals: np.ndarray, initial: int = 0):
        self.next = np.ascontiguousarray(next_table, dtype=np.int32)
        self.finals = np.ascontiguousarray(finals, dtype=np.uint8)
        self.initial = int(initial)
        if self.next.ndim != 2 or self.next.shape[1] != 256:
            raise ValueError("next table must be [states][256]")

    @property
    def n_states(self) -> int:
        return int(self.next.shape[0])


def mask_constraint_logits(raw_logits, legal_token_ids, termination_token_ids) -> np.ndarray:
    """maskConstraintLogits (src/runtime/constraints.ts:159-173): -inf except the
    legal and termination ids (f32, like the reference's Float32Array)."""
    raw = np.asarray(raw_logits, dtype=np.float32)
    out = np.full(raw.shape, -np.inf, dtype=np.float32)
    for ids in (legal_token_ids, termination_token_ids):
        for t in ids:
            if 0 <= t < raw.size:
                out[t] = raw[t]
    return out


class CompiledByteConstraint:
    """Per-request constraint state over a byte DFA, driving the GPU masker."""

    def __init__(self, sampler: Sampler, vocab: VocabBytes, dfa: ByteDfa):
        if vocab.vocabulary_size != sampler.vocab:
            raise GSampleError(1, "vocab size differs from the sampler's")
        self.sampler = sampler
        self.vocab = vocab
        self.dfa = dfa
        sampler.set_vocab(vocab.offsets, vocab.data)
        sampler.set_dfa(dfa.next, dfa.finals)
        self.state = dfa.initial
        self._mask_cache: Dict[int, object] = {}

    @property
    def accepting(self) -> bool:
        return self.sampler.dfa_accepting(self.state)

    def masks_for(self, states: Sequence[int]):
        """Mask table rows for `states` (cached per state); returns (table, slots)."""
        torch = self.sampler.torch
        missing = sorted({int(s) for s in states if int(s) not in self._mask_cache})
        if missing:
            table = self.sampler.build_masks(missing)
            for i, s in enumerate(missing):
                self._mask_cache[s] = table[i]
        uniq = sorted({int(s) for s in states})
        table = torch.stack([self._mask_cache[s] for s in uniq])
        slot_of = {s: i for i, s in enumerate(uniq)}
        return table, [slot_of[int(s)] for s in states]

    def legal_token_ids(self) -> List[int]:
        """legalTokenIds (constraints.ts:56-92) for the current state, ascending."""
        table, _ = self.masks_for([self.state])
        bits = table[0].cpu().numpy().view(np.uint32)
        ids = np.nonzero(np.unpackbits(bits.view(np.uint8), bitorder="little")[: self.sampler.vocab])[0]
        return [int(i) for i in ids]

    def accept_token(self, token_bytes: bytes):
        """acceptToken (constraints.ts:94-103)."""
        s = self.state
        for b in token_bytes:
            nxt = int(self.dfa.next[s, b])
            if nxt < 0 or not self._viable(nxt):
                raise GSampleError(5, "Selected token violates the generation constraint")
            s = nxt
        self.state = s

    def accept_token_id(self, token_id: int):
        self.state = int(self.sampler.dfa_advance([self.state], [token_id])[0])

    def _viable(self, s: int) -> bool:
        if not hasattr(self, "_viable_set"):
            # reverse reachability from finals (constraints.ts:300-322)
            n = self.dfa.n_states
            preds = [[] for _ in range(n)]
            for a in range(n):
                for t in set(int(x) for x in self.dfa.next[a] if x >= 0):
                    preds[t].append(a)
            viable = set(int(i) for i in np.nonzero(self.dfa.finals)[0])
            stack = list(viable)
            while stack:
                for p in preds[stack.pop()]:
                    if p not in viable:
                        viable.add(p)
                        stack.append(p)
            self._viable_set = viable
        return s in self._viable_set


def forced_ids_csr(rows: int, termination_ids: Sequence[int], extra_ids: Sequence[int] = ()):
    """Per-row forced ids of constrained rows, as (offsets, ids, kinds): the
    termination ids (EOS + custom stop ids; legal only when the constraint is
    accepting) and the extra legal ids (gemma-session.ts:1312-1323)."""
    ids = [int(t) for t in termination_ids] + [int(e) for e in extra_ids]
    kinds = [GS_FORCED_TERMINATION] * len(termination_ids) + [GS_FORCED_EXTRA] * len(extra_ids)
    offsets = np.arange(rows + 1, dtype=np.int64) * len(ids)
    if not ids:
        return offsets, np.zeros(1, np.int32), np.zeros(1, np.uint8)
    return offsets, np.tile(np.asarray(ids, np.int32), rows), np.tile(np.asarray(kinds, np.uint8), rows)
