"""Seeded synthetic inputs for the sampling-stage workloads.

Every row is generated from its own seed (numpy Philox keyed by
(workload seed, row)), so any subset of rows can be rebuilt independently of
the batch, and buffers are identical on every machine.

  single_row     1 x 262144 f32 ~ N(0, 3^2); T 0.8, topK 40, topP 0.95, seed 42
  penalties      256 x 262144 f32 ~ N(0, 3^2); 512-id Zipf(1.1) histories,
                 repetition 1.1, presence 0.5, frequency 0.3, window 512;
                 T 0.7, topK 50, topP 0.9; row r draws with seed r
  constrained    128 x 262144 f32 ~ N(0, 3^2); a vocab of random printable byte
                 strings (1-12 bytes) and a 64-state byte DFA with ~3% of tokens
                 legal per state; start state per row; greedy and topP 0.95 (T 1)
  heavy_tail     1024 x 262144 bf16 = RNE(8 ln(rank^-1.1) + N(0, 0.5^2)),
                 vocab permuted per row; topP 0.9 only, T 1, seed = row
  lmhead         H 64 x 2048 bf16 ~ N(0,1), W 262144 x 2048 bf16 ~ N(0, 0.02^2),
                 softcap 30, 256-id histories (window 256), the constrained
                 workload's DFA, topK 64, topP 0.95, T 1, seed = row
  multinomial    256 x 262144 f32 ~ N(0, 3^2); T 0.8 with topK 0, topP 1: the
                 generate() defaults with a temperature (a full-vocabulary draw)
  topk_deep      256 x 262144 f32 ~ N(0, 3^2); T 0.8, topK 200, topP 0.95
  typical        256 x 262144 f32 ~ N(0, 3^2); T 0.8, topK 40, typicalP 0.9
  penalties_constrained
                 256 x 262144 f32 ~ N(0, 3^2); the penalties workload's
                 histories and options (window 512, T 0.7, topK 50, topP 0.9)
                 on logits masked by the constrained workload's 64-state DFA
                 (start state per row): top-k / top-p + penalties + grammar
                 mask in one batch
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from .config import DecodingConfig

V = 262144


def rng(seed: int, row: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(key=[int(seed) & 0xFFFFFFFFFFFFFFFF, int(row)]))


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((b >> 16) & 1) + 0x7FFF
    return ((b + r) >> 16).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)


def zipf_ids(g: np.random.Generator, n: int, s: float = 1.1, vocab: int = V) -> np.ndarray:
    """n ids from Zipf(s) over ranks 1..vocab (rank r -> id r-1)."""
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, g.random(n), side="right"), vocab - 1).astype(np.int32)


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8)).hexdigest()


@dataclass
class Workload:
    name: str
    rows: int
    logits: Optional[np.ndarray]          # [rows][V] f32, or bf16 bits as uint16
    dtype: str                            # "f32" | "bf16"
    configs: List[DecodingConfig]
    seeds: List[int]
    histories: Optional[List[np.ndarray]] = None
    states: Optional[np.ndarray] = None   # DFA start state per row
    extra: dict = field(default_factory=dict)


def normal_logits(seed: int, rows: List[int], sigma: float = 3.0, vocab: int = V) -> np.ndarray:
    out = np.empty((len(rows), vocab), dtype=np.float32)
    for i, r in enumerate(rows):
        out[i] = rng(seed, r).normal(0.0, sigma, vocab).astype(np.float32)
    return out


def single_row(vocab: int = V) -> Workload:
    cfg = DecodingConfig(temperature=0.8, topK=40, topP=0.95, minP=0.0, typicalP=1.0, repetitionPenalty=1.0,
                         repetitionWindow=0, frequencyPenalty=0.0, presencePenalty=0.0, seed=42)
    return Workload("single_row", 1, normal_logits(1, [0], vocab=vocab), "f32", [cfg], [42])


PENALTY_CONFIG = DecodingConfig(temperature=0.7, topK=50, topP=0.9, minP=0.0, typicalP=1.0, repetitionPenalty=1.1,
                                repetitionWindow=512, frequencyPenalty=0.3, presencePenalty=0.5)


def penalties(rows: Optional[List[int]] = None, n_rows: int = 256, vocab: int = V) -> Workload:
    rows = list(range(n_rows)) if rows is None else rows
    logits = normal_logits(2, rows, vocab=vocab)
    hist = [zipf_ids(rng(3, r), 512, vocab=vocab) for r in rows]
    cfgs = [PENALTY_CONFIG.merged(seed=r) for r in rows]
    return Workload("penalties", len(rows), logits, "f32", cfgs, list(rows), histories=hist)


def synthetic_vocab(seed: int = 4, vocab: int = V):
    """V random strings of 1-12 bytes in 0x20..0x7E, as (offsets, data)."""
    g = rng(seed, 0)
    lengths = g.integers(1, 13, vocab)
    offsets = np.zeros(vocab + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(lengths)
    data = g.integers(0x20, 0x7F, int(offsets[-1])).astype(np.uint8)
    return offsets, data


def synthetic_dfa(seed: int = 5, n_states: int = 64, edges_per_state: int = 25):
    """A random byte DFA: each state has `edges_per_state` printable bytes with
    edges to random states; states 0..3 are final. With 25 of 95 printable
    bytes defined, about 3% of 1-12-byte random strings stay legal."""
    g = rng(seed, 0)
    nxt = np.full((n_states, 256), -1, dtype=np.int32)
    for s in range(n_states):
        chars = g.choice(np.arange(0x20, 0x7F), size=edges_per_state, replace=False)
        nxt[s, chars] = g.integers(0, n_states, edges_per_state)
    finals = np.zeros(n_states, dtype=np.uint8)
    finals[:4] = 1
    return nxt, finals


def penalties_constrained(rows: Optional[List[int]] = None, n_rows: int = 256, vocab: int = V) -> Workload:
    rows = list(range(n_rows)) if rows is None else rows
    logits = normal_logits(15, rows, vocab=vocab)
    hist = [zipf_ids(rng(16, r), 512, vocab=vocab) for r in rows]
    states = np.array([int(rng(17, r).integers(0, 64)) for r in rows], dtype=np.int32)
    cfgs = [PENALTY_CONFIG.merged(seed=r) for r in rows]
    return Workload("penalties_constrained", len(rows), logits, "f32", cfgs, list(rows), histories=hist,
                    states=states)


CONSTRAINED_TOPP = DecodingConfig(temperature=1.0, topK=0, topP=0.95, minP=0.0, typicalP=1.0, repetitionPenalty=1.0,
                                  repetitionWindow=0, frequencyPenalty=0.0, presencePenalty=0.0)
CONSTRAINED_GREEDY = CONSTRAINED_TOPP.merged(temperature=0.0)


def constrained(rows: Optional[List[int]] = None, n_rows: int = 128, greedy: bool = False, vocab: int = V) -> Workload:
    rows = list(range(n_rows)) if rows is None else rows
    logits = normal_logits(6, rows, vocab=vocab)
    states = np.array([int(rng(7, r).integers(0, 64)) for r in rows], dtype=np.int32)
    base = CONSTRAINED_GREEDY if greedy else CONSTRAINED_TOPP
    cfgs = [base.merged(seed=r) for r in rows]
    return Workload("constrained", len(rows), logits, "f32", cfgs, list(rows), states=states)


HEAVY_TAIL_CONFIG = DecodingConfig(temperature=1.0, topK=0, topP=0.9, minP=0.0, typicalP=1.0, repetitionPenalty=1.0,
                                   repetitionWindow=0, frequencyPenalty=0.0, presencePenalty=0.0)


def heavy_tail(rows: Optional[List[int]] = None, n_rows: int = 1024, vocab: int = V) -> Workload:
    rows = list(range(n_rows)) if rows is None else rows
    base = 8.0 * np.log(np.arange(1, vocab + 1, dtype=np.float64) ** (-1.1))
    out = np.empty((len(rows), vocab), dtype=np.uint16)
    for i, r in enumerate(rows):
        g = rng(8, r)
        x = base + g.normal(0.0, 0.5, vocab)
        perm = g.permutation(vocab)
        out[i, perm] = to_bf16_bits(x.astype(np.float32))
    cfgs = [HEAVY_TAIL_CONFIG.merged(seed=r) for r in rows]
    return Workload("heavy_tail", len(rows), out, "bf16", cfgs, list(rows))


LMHEAD_CONFIG = DecodingConfig(temperature=1.0, topK=64, topP=0.95, minP=0.0, typicalP=1.0, repetitionPenalty=1.1,
                               repetitionWindow=256, frequencyPenalty=0.3, presencePenalty=0.5)


def lmhead_inputs(n_rows: int = 64, width: int = 2048, vocab: int = V, device=None):
    """(hidden, weight) bf16 torch tensors built on `device` from seeded CPU chunks."""
    import torch

    g = torch.Generator().manual_seed(9)
    hidden = torch.randn(n_rows, width, generator=g, dtype=torch.float32).to(torch.bfloat16)
    weight = torch.empty(vocab, width, dtype=torch.bfloat16, device=device)
    step = 16384
    for r0 in range(0, vocab, step):
        gg = torch.Generator().manual_seed(10_000 + r0)
        w = torch.randn(min(step, vocab - r0), width, generator=gg, dtype=torch.float32) * 0.02
        weight[r0:r0 + w.shape[0]] = w.to(torch.bfloat16).to(device)
    return hidden.to(device), weight


def lmhead_histories(n_rows: int = 64, vocab: int = V) -> List[np.ndarray]:
    return [zipf_ids(rng(11, r), 256, vocab=vocab) for r in range(n_rows)]


MULTINOMIAL_CONFIG = DecodingConfig(temperature=0.8, topK=0, topP=1.0, minP=0.0, typicalP=1.0, repetitionPenalty=1.0,
                                    repetitionWindow=0, frequencyPenalty=0.0, presencePenalty=0.0)
TOPK_DEEP_CONFIG = MULTINOMIAL_CONFIG.merged(topK=200, topP=0.95)
TYPICAL_CONFIG = MULTINOMIAL_CONFIG.merged(topK=40, typicalP=0.9)


def _plain(name: str, cfg: DecodingConfig, seed: int, rows: Optional[List[int]], n_rows: int, vocab: int) -> Workload:
    rows = list(range(n_rows)) if rows is None else rows
    logits = normal_logits(seed, rows, vocab=vocab)
    return Workload(name, len(rows), logits, "f32", [cfg.merged(seed=r) for r in rows], list(rows))


def multinomial(rows: Optional[List[int]] = None, n_rows: int = 256, vocab: int = V) -> Workload:
    return _plain("multinomial", MULTINOMIAL_CONFIG, 12, rows, n_rows, vocab)


def topk_deep(rows: Optional[List[int]] = None, n_rows: int = 256, vocab: int = V) -> Workload:
    return _plain("topk_deep", TOPK_DEEP_CONFIG, 13, rows, n_rows, vocab)


def typical(rows: Optional[List[int]] = None, n_rows: int = 256, vocab: int = V) -> Workload:
    return _plain("typical", TYPICAL_CONFIG, 14, rows, n_rows, vocab)
