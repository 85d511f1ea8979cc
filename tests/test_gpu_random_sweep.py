"""Randomised batches against the oracle: seeded draws over vocabulary sizes
(two to 32 chunks, aligned or not), batch sizes (lone rows to 64), f32 and
bf16 logits, the softcap, quantised logits (exact ties), mostly -inf rows, a
few huge logits, penalty windows with out-of-range ids, every filter
(top-k, min-p, typical-p, top-p, full-vocabulary draws, greedy), uniforms at
0 and near 1, and mask tables of one to three slots with 0.1% to 50% legal
ids. Each batch runs with the batch hint (deep draws over many workgroups)
and without it; every row's id must be the oracle's (sampling.ts:18-65,
constraints.ts:159-173), with probabilities as in the other parity tests.
A wider run of the same generator (tens of thousands of batches) found the
typical-p pool that reaches past a row's finite logits."""
import math

import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

PROB_RTOL = 4e-7
VOCABS = [700, 3000, 5000, 8192, 8269, 16384, 20000, 32768, 40000, 65549, 100000, 262144]
ROWS = [1, 2, 3, 4, 5, 8, 17, 32, 64]


def _batch(gs, oracle, seed):
    W = gs.workloads
    rng = np.random.default_rng(seed)
    V = int(rng.choice(VOCABS))
    R = int(rng.choice(ROWS))
    if V >= 100000:
        R = min(R, 17)
    bf16 = rng.random() < 0.25
    cap = 30.0 if rng.random() < 0.15 else 0.0
    xs, hists, cfgs, us = [], [], [], []
    for _ in range(R):
        x = rng.normal(0, rng.uniform(0.3, 5.0), V).astype(np.float32)
        q = rng.random()
        if q < 0.15:
            x = (np.round(x * 4) / 4).astype(np.float32)
        elif q < 0.25:
            x = (np.round(x * 8) / 8).astype(np.float32)
        if rng.random() < 0.1:
            x[rng.random(V) < 0.8] = -np.inf
        if rng.random() < 0.05:
            x[rng.integers(0, V, 3)] = np.float32(rng.uniform(20, 60))
        xs.append(x)
        hists.append(rng.integers(-2, V + 2, int(rng.integers(0, 120))).tolist())
        full = rng.random() < 0.4
        cfgs.append(gs.DecodingConfig(
            temperature=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.0, 1.5])),
            topK=0 if full else int(rng.choice([0, 1, 5, 40, 64, 65, 300, 2000])),
            topP=1.0 if full else float(rng.choice([1.0, 0.95, 0.9, 0.5, 0.1])),
            minP=0.0 if full else float(rng.choice([0.0, 0.0, 0.05, 0.3])),
            typicalP=1.0 if full else float(rng.choice([1.0, 1.0, 1.0, 0.9, 0.3])),
            repetitionPenalty=float(rng.choice([1.0, 1.1, 2.0])),
            repetitionWindow=int(rng.choice([0, 8, 64, 512])),
            frequencyPenalty=float(rng.choice([0.0, 0.3])),
            presencePenalty=float(rng.choice([0.0, 0.5]))))
        us.append(float(rng.random()) if rng.random() < 0.8 else float(rng.choice([0.0, 1 - 2 ** -32, 0.999])))
    X = np.stack(xs)
    bits = None
    if bf16:
        bits = W.to_bf16_bits(X)
        X = W.bf16_bits_to_f32(bits).reshape(R, V)
    vals = [oracle.softcap(X[r], cap) if cap > 0 else X[r] for r in range(R)]
    words, slots = None, [-1] * R
    if rng.random() < 0.3:
        n_slots = int(rng.integers(1, 4))
        words = np.zeros((n_slots, (V + 31) // 32), np.uint32)
        legal_sets = []
        for k in range(n_slots):
            frac = float(rng.choice([0.001, 0.01, 0.03, 0.2, 0.5]))
            legal = np.unique(np.concatenate([rng.choice(V, max(1, int(V * frac)), replace=False),
                                              [int(rng.integers(0, V))]]))
            np.bitwise_or.at(words[k], legal >> 5, np.left_shift(np.uint32(1), (legal & 31).astype(np.uint32)))
            legal_sets.append(legal.astype(np.int32))
        slots = [int(rng.integers(-1, n_slots)) for _ in range(R)]
        vals = [oracle.mask_logits(vals[r], legal_sets[slots[r]], []) if slots[r] >= 0 else vals[r]
                for r in range(R)]
    return V, R, X, bits, cap, vals, hists, cfgs, us, words, slots


def _ocfg(c):
    return Decoding(temperature=c.temperature, topK=c.topK, topP=c.topP, minP=c.minP, typicalP=c.typicalP,
                    repetitionPenalty=c.repetitionPenalty, repetitionWindow=c.repetitionWindow,
                    frequencyPenalty=c.frequencyPenalty, presencePenalty=c.presencePenalty)


def test_random_sweep_matches_oracle(oracle):
    import torch

    import gsample as gs

    samplers = {}
    bad = []
    n_rows = 0
    try:
        for seed in range(300):
            V, R, X, bits, cap, vals, hists, cfgs, us, words, slots = _batch(gs, oracle, 900000 + seed)
            if V not in samplers:
                samplers[V] = gs.Sampler(vocab_size=V, max_rows=64)
            s = samplers[V]
            dev = (torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16) if bits is not None
                   else torch.from_numpy(X).cuda())
            table = torch.from_numpy(words.view(np.int32)).cuda() if words is not None else None
            conf = np.stack([gs.runtime.row_config(c, uniform=u, softcap_value=cap, mask_slot=m)
                             for c, u, m in zip(cfgs, us, slots)])
            outs = {"hint": s.sample(dev, conf, histories=hists, mask_table=table, raise_on_failure=False),
                    "no hint": s.sample(dev, conf, histories=hists, mask_table=table, raise_on_failure=False,
                                        hints=0)}
            for r in range(R):
                t, tr = oracle.sample_token(vals[r], hists[r], _ocfg(cfgs[r]), us[r])
                p = tr.probability if t >= 0 else 0.0
                for tag, out in outs.items():
                    tok, fl, pr = int(out.tokens[r]), int(out.flags[r]), float(out.probabilities[r])
                    if t < 0:
                        ok = bool(fl & gs.GS_FLAG_EMPTY_CANDIDATES)
                    else:
                        ok = tok == t and not fl & gs.GS_FLAG_INDEX_CHECK
                        if ok and cfgs[r].temperature > 0:
                            if fl & gs.GS_FLAG_EXACT_PATH:
                                ok = pr == p or (math.isnan(p) and math.isnan(pr))
                            else:
                                ok = abs(pr - p) <= PROB_RTOL * abs(p)
                    if not ok:
                        bad.append(f"seed {900000 + seed} V {V} row {r} slot {slots[r]} {tag}: {tok} (flags {fl}, "
                                   f"p {pr}) != {t} (p {p}); {cfgs[r]} u {us[r]}")
            n_rows += R
    finally:
        for s in samplers.values():
            s.close()
    assert not bad, "\n".join(bad[:20])
    assert n_rows > 2000, n_rows
