"""The oracle's constraint functions against the reference's known answers.

The reference compiles regexes to code-point DFAs with refa (absent here);
each pattern of tests/constraints.spec.ts:27-70 is small enough to write down
as the byte-level DFA that accepts the same byte strings, so the reference's
expected legal sets, acceptance states and masks pin the oracle's legalTokenIds
(constraints.ts:56-92), findViableStates (:300-322) and maskConstraintLogits
(:159-173)."""
import numpy as np


def byte_dfa(n_states, edges, finals):
    nxt = np.full((n_states, 256), -1, dtype=np.int32)
    for s, b, t in edges:
        nxt[s, b] = t
    f = np.zeros(n_states, dtype=np.uint8)
    f[list(finals)] = 1
    return nxt, f


def csr(words):
    data = [bytes(w) if w is not None else b"" for w in words]
    offsets = np.zeros(len(data) + 1, dtype=np.int64)
    offsets[1:] = np.cumsum([len(d) for d in data])
    return offsets, np.frombuffer(b"".join(data), dtype=np.uint8).copy()


def legal(oracle, nxt, f, words, state):
    offsets, data = csr(words)
    viable = oracle.viable_states(nxt, f)
    return oracle.mask_bits_to_ids(oracle.dfa_legal_mask(nxt, viable, offsets, data, state), len(words)).tolist()


def walk(nxt, state, token_bytes):
    for b in token_bytes:
        state = int(nxt[state, b])
        if state < 0:
            return -1
    return state


def test_full_match_regex_trie_pruning(oracle):  # constraints.spec.ts:27-39, pattern a(?:b|c)
    words = [None, b"a", b"b", b"c", b"ab", b"ac", b"x"]
    nxt, f = byte_dfa(3, [(0, ord("a"), 1), (1, ord("b"), 2), (1, ord("c"), 2)], [2])
    assert legal(oracle, nxt, f, words, 0) == [1, 4, 5]
    s = walk(nxt, 0, b"a")
    assert not f[s]
    assert legal(oracle, nxt, f, words, s) == [2, 3]
    s = walk(nxt, s, b"b")
    assert f[s]


def test_utf8_state_across_token_boundaries(oracle):  # constraints.spec.ts:41-57, pattern U+0623
    arabic = "أ".encode("utf-8")
    words = [None, arabic[:1], arabic[1:], arabic, b"\xff"]
    nxt, f = byte_dfa(3, [(0, arabic[0], 1), (1, arabic[1], 2)], [2])
    assert legal(oracle, nxt, f, words, 0) == [1, 3]
    s = walk(nxt, 0, arabic[:1])
    assert not f[s]
    assert legal(oracle, nxt, f, words, s) == [2]
    assert f[walk(nxt, s, arabic[1:])]


def test_incomplete_utf8_prefixes_rejected(oracle):  # constraints.spec.ts:59-70, pattern \{
    words = [None, b"\xef", b"\xbf", b"\xbd", b"{"]
    nxt, f = byte_dfa(2, [(0, ord("{"), 1)], [1])
    assert legal(oracle, nxt, f, words, 0) == [4]


def test_non_viable_states_prune_tokens(oracle):
    """A state that cannot reach a final state makes every token through it
    illegal (isViableConstraintState, constraints.ts:253-265)."""
    words = [b"a", b"ab", b"b", b"ba"]
    # 0 -a-> 1 (final), 0 -b-> 2 (no way to a final state), 2 -a-> 2
    nxt, f = byte_dfa(3, [(0, ord("a"), 1), (0, ord("b"), 2), (2, ord("a"), 2)], [1])
    assert oracle.viable_states(nxt, f).tolist() == [1, 1, 0]
    assert legal(oracle, nxt, f, words, 0) == [0]


def test_mask_logits_known_answer(oracle):  # constraints.spec.ts:158-161
    masked = oracle.mask_logits([1, 2, 3, 4], [1, 3], [0])
    assert masked.tolist() == [1.0, 2.0, float("-inf"), 4.0]
