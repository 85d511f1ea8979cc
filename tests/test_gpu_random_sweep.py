"""Randomised batches against the oracle: seeded draws over vocabulary sizes
(two to 32 chunks, aligned or not), batch sizes (lone rows to 64), f32 and
bf16 logits, the softcap, quantised logits (exact ties), mostly -inf rows, a
few huge logits, penalty windows with out-of-range ids, every filter
(top-k, min-p, typical-p, top-p, full-vocabulary draws, greedy), uniforms at
0 and near 1 or seeded draws at a draw index, forced exact replays, and mask
tables of one to three slots with 0.1% to 50% legal ids, with termination and
extra ids on some (gemma-session.ts:1305-1329, dead ends included), and rows
padded past V with NaN and +inf that no kernel may read. Each batch
runs with the batch hint (deep draws over many workgroups) and without it;
every row's id must be the oracle's (sampling.ts:18-65,
constraints.ts:159-173), with probabilities as in the other parity tests. A
wider run of the same generator (tens of thousands of batches) found the
typical-p pool that reaches past a row's finite logits."""
import math

import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

PROB_RTOL = 4e-7
VOCABS = [700, 3000, 5000, 8192, 8269, 16384, 20000, 32768, 40000, 65549, 100000, 262144]
ROWS = [1, 2, 3, 4, 5, 8, 17, 32, 64]


def _batch(gs, oracle, seed, extreme=False, typical=False):
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
        sigma = float(rng.choice([1e-3, 0.3, 5.0, 50.0, 3e3])) if extreme else rng.uniform(0.3, 5.0)
        x = rng.normal(0, sigma, V).astype(np.float32)
        q = rng.random() * (0.5 if typical else 1.0)
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
        full = rng.random() < 0.4 and not typical
        if typical:
            # typical-p on every row, half the rows on a 1/4 or 1/8 grid: exact
            # and mirrored surprise ties (sampling.ts:49-55)
            cfgs.append(gs.DecodingConfig(
                temperature=float(rng.choice([0.3, 0.7, 1.0, 1.5, 3.0])),
                topK=int(rng.choice([0, 3, 10, 40, 64, 100, 128, 300])),
                topP=float(rng.choice([1.0, 1.0, 0.95, 0.5])),
                minP=float(rng.choice([0.0, 0.0, 0.0, 0.05])),
                typicalP=float(rng.choice([0.05, 0.2, 0.5, 0.8, 0.95, 0.999])),
                repetitionPenalty=float(rng.choice([1.0, 1.1])),
                repetitionWindow=int(rng.choice([0, 64]))))
            us.append(float(rng.random()) if rng.random() < 0.8 else float(rng.choice([0.0, 1 - 2 ** -32, 0.999])))
            continue
        if extreme:
            # the far ends of every option the reference accepts (decoding.ts:31-55)
            cfgs.append(gs.DecodingConfig(
                temperature=float(rng.choice([0.0, 1e-3, 0.05, 0.7, 20.0, 1e3])),
                topK=0 if full else int(rng.choice([0, 1, 2, 63, 64, 4096, 4097, 100000])),
                topP=1.0 if full else float(rng.choice([1.0, 0.999999999, 0.5, 1e-9])),
                minP=0.0 if full else float(rng.choice([0.0, 1e-9, 0.5, 0.99])),
                typicalP=1.0 if full else float(rng.choice([1.0, 1.0, 0.999, 0.01])),
                repetitionPenalty=float(rng.choice([1.0, 0.5, 5.0])),
                repetitionWindow=int(rng.choice([0, 1, 1000])),
                frequencyPenalty=float(rng.choice([0.0, 10.0, 0.001])),
                presencePenalty=float(rng.choice([0.0, 10.0, 1e-6]))))
            us.append(float(rng.random()) if rng.random() < 0.8 else float(rng.choice([0.0, 1 - 2 ** -32, 0.999])))
            continue
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
    words, slots, forced = None, [-1] * R, None
    accepting, dead = [False] * R, [False] * R
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
        if rng.random() < 0.5:
            # forced ids (gemma-session.ts:1305-1329): termination ids, legal only when the
            # constraint is accepting, and extra legal ids, some of them termination ids too
            f_ids, f_kinds, f_off = [], [], [0]
            for r in range(R):
                if slots[r] >= 0:
                    term = rng.integers(0, V, int(rng.integers(0, 4))).tolist()
                    extra = rng.integers(0, V, int(rng.integers(0, 5))).tolist()
                    if term and rng.random() < 0.3:
                        extra.append(term[0])
                    if rng.random() < 0.3:
                        term.append(int(legal_sets[slots[r]][0]))
                    accepting[r] = bool(rng.random() < 0.5)
                    f_ids += term + extra
                    f_kinds += [gs.runtime.GS_FORCED_TERMINATION] * len(term) + [gs.runtime.GS_FORCED_EXTRA] * len(extra)
                    tset = set(term)
                    legal = [t for t in set(legal_sets[slots[r]].tolist()) | set(extra) if t not in tset]
                    lterm = sorted(tset) if accepting[r] else []
                    dead[r] = not legal and not lterm
                    vals[r] = oracle.mask_logits(vals[r], legal, lterm)
                f_off.append(len(f_ids))
            forced = (np.asarray(f_off, np.int64), np.asarray(f_ids or [0], np.int32),
                      np.asarray(f_kinds or [0], np.uint8))
        else:
            vals = [oracle.mask_logits(vals[r], legal_sets[slots[r]], []) if slots[r] >= 0 else vals[r]
                    for r in range(R)]
    # seeded draws (SeededRandom(seed) at a draw index) on some rows, forced exact replays on a few
    seeded = [rng.random() < 0.3 for _ in range(R)]
    seeds = [int(rng.integers(0, 2 ** 32)) for _ in range(R)]
    didx = [int(rng.integers(0, 50)) for _ in range(R)]
    fexact = [rng.random() < 0.05 for _ in range(R)]
    confs = []
    for r in range(R):
        if seeded[r]:
            us[r] = float(oracle.draw(seeds[r], didx[r]))
        confs.append(gs.runtime.row_config(cfgs[r], uniform=None if seeded[r] else us[r],
                                           seed=seeds[r] if seeded[r] else None, draw_index=didx[r] if seeded[r] else 0,
                                           softcap_value=cap, mask_slot=slots[r], accepting=accepting[r],
                                           force_exact=fexact[r]))
    # padded rows on some batches (a row stride past V; NaN and +inf in the padding, which no kernel
    # may read)
    pad = int(rng.choice([1, 3, 64])) if rng.random() < 0.2 else 0
    return V, R, X, bits, vals, hists, cfgs, us, words, forced, dead, np.stack(confs), pad


def _device_rows(torch, X, bits, pad):
    """The batch's logits on the device, in rows of V + pad elements when pad > 0."""
    R, V = X.shape
    if bits is not None:
        if not pad:
            return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
        buf = np.zeros((R, V + pad), np.uint16)
        buf[:, V:] = np.where(np.arange(pad) % 2 == 0, 0x7FC0, 0x7F80).astype(np.uint16)
        buf[:, :V] = bits
        return torch.from_numpy(buf.view(np.int16)).cuda().view(torch.bfloat16)[:, :V]
    if not pad:
        return torch.from_numpy(X).cuda()
    buf = np.zeros((R, V + pad), np.float32)
    buf[:, V:] = np.where(np.arange(pad) % 2 == 0, np.nan, np.inf).astype(np.float32)
    buf[:, :V] = X
    return torch.from_numpy(buf).cuda()[:, :V]


def _ocfg(c):
    return Decoding(temperature=c.temperature, topK=c.topK, topP=c.topP, minP=c.minP, typicalP=c.typicalP,
                    repetitionPenalty=c.repetitionPenalty, repetitionWindow=c.repetitionWindow,
                    frequencyPenalty=c.frequencyPenalty, presencePenalty=c.presencePenalty)


@pytest.mark.parametrize("extreme,typical,n_batches,seed0",
                         [(False, False, 300, 900000), (True, False, 100, 950000), (False, True, 150, 1200000)])
def test_random_sweep_matches_oracle(oracle, extreme, typical, n_batches, seed0):
    """300 batches of the settings above; 100 more at the far ends of every
    option: temperatures 1e-3 to 1e3, logit spreads 1e-3 to 3e3, topK up to
    100000, topP 1e-9 and 1 - 1e-9, minP 0.99, typicalP 0.01, repetition
    penalties 0.5 and 5, presence and frequency penalties of 10, windows of 1
    and 1000 ids; 150 with typical-p (0.05 to 0.999) on every row and half the
    rows' logits on a grid, so that surprises tie, exactly or mirrored about
    the entropy."""
    import torch

    import gsample as gs

    samplers = {}
    bad = []
    n_rows = 0
    try:
        for seed in range(seed0, seed0 + n_batches):
            V, R, X, bits, vals, hists, cfgs, us, words, forced, dead, conf, pad = _batch(gs, oracle, seed, extreme, typical)
            if V not in samplers:
                samplers[V] = gs.Sampler(vocab_size=V, max_rows=64)
            s = samplers[V]
            dev = _device_rows(torch, X, bits, pad)
            table = torch.from_numpy(words.view(np.int32)).cuda() if words is not None else None
            outs = {"hint": s.sample(dev, conf, histories=hists, forced=forced, mask_table=table,
                                     raise_on_failure=False),
                    "no hint": s.sample(dev, conf, histories=hists, forced=forced, mask_table=table,
                                        raise_on_failure=False, hints=0)}
            for r in range(R):
                if dead[r]:
                    # no legal id and no legal termination id: the reference throws
                    for tag, out in outs.items():
                        if not int(out.flags[r]) & gs.GS_FLAG_DEAD_END:
                            bad.append(f"seed {seed} row {r} {tag}: flags {int(out.flags[r])}, no dead end")
                    continue
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
                        bad.append(f"seed {seed} V {V} row {r} slot {int(conf[r]['mask_slot'])} {tag}: {tok} (flags {fl}, "
                                   f"p {pr}) != {t} (p {p}); {cfgs[r]} u {us[r]}")
            n_rows += R
    finally:
        for s in samplers.values():
            s.close()
    assert not bad, "\n".join(bad[:20])
    assert n_rows > 6 * n_batches, n_rows
