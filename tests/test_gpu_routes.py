"""GPU parity of the option settings that used to fall onto the exact replay:
a full-vocabulary draw (topK 0, topP 1: the generate() defaults with a
temperature), top-k above 64, and typical-p with top-k up to 64. Ids are
bit-exact against the oracle (sampling.ts:18-65); probabilities identical on
exact-path rows and within PROB_RTOL relative on one-pass rows."""
import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

PROB_RTOL = 4e-7
V = 262144


def _gs():
    import gsample

    return gsample


def to_oracle_cfg(c):
    return Decoding(temperature=c.temperature, topK=c.topK, topP=c.topP, minP=c.minP, typicalP=c.typicalP,
                    repetitionPenalty=c.repetitionPenalty, repetitionWindow=c.repetitionWindow,
                    frequencyPenalty=c.frequencyPenalty, presencePenalty=c.presencePenalty)


def check(gs, oracle, label, out, xs, hists, cfgs, us):
    exact = 0
    for r in range(len(cfgs)):
        t, tr = oracle.sample_token(xs[r], hists[r] if hists else [], to_oracle_cfg(cfgs[r]), us[r])
        assert int(out.tokens[r]) == t, f"{label} row {r}: {int(out.tokens[r])} != {t} (flags {int(out.flags[r])})"
        assert not out.flags[r] & gs.GS_FLAG_INDEX_CHECK, (label, r, int(out.flags[r]))
        p = 1.0 if cfgs[r].temperature == 0 else tr.probability
        if out.flags[r] & gs.GS_FLAG_EXACT_PATH:
            exact += 1
            assert out.probabilities[r] == p, (label, r)
        else:
            assert abs(out.probabilities[r] - p) <= PROB_RTOL * p, (label, r, out.probabilities[r], p)
    return exact


def test_full_vocabulary_draws(sampler, oracle):
    """topK 0, topP 1: the draw walks the whole sorted vocabulary. Draws that
    land inside the complete region of the chunk lists are settled there
    (ctotal is the row's whole mass, 1 within (2V + 2) 2^-53); the rest
    replay exactly. u spans [0, 1) including both ends."""
    import torch

    gs = _gs()
    w = gs.workloads.multinomial(rows=list(range(48)))
    us = [0.0, 1 - 2 ** -32] + [float(u) for u in np.random.default_rng(3).random(46)]
    cfgs = [c.merged(temperature=t) for c, t in zip(w.configs, [0.8, 0.5, 1.0, 0.7] * 12)]
    # with a penalty window on some rows (its ids among the row's largest logits)
    hists = [np.argsort(-w.logits[r])[:30].tolist() if r % 3 == 0 else [] for r in range(48)]
    cfgs = [c.merged(repetitionPenalty=1.2, repetitionWindow=64) if r % 3 == 0 else c for r, c in enumerate(cfgs)]
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf, histories=hists)
    exact = check(gs, oracle, "full draw", out, w.logits, hists, cfgs, us)
    assert exact < 24, exact  # most draws settle on the one-pass path


def test_full_vocabulary_draw_boundary(sampler, oracle):
    """u placed on a prefix-sum boundary of the sorted probabilities (within
    1e-12 of it): the one-pass draw cannot decide it and the row replays
    exactly, with the oracle's id."""
    import torch

    gs = _gs()
    rng = np.random.default_rng(19)
    x = rng.normal(0, 3, V).astype(np.float32)
    T = 0.8
    v = np.sort(x.astype(np.float64) / T)[::-1]
    e = np.exp(v - v[0])
    cum = np.cumsum(e / e.sum())
    us, xs = [], []
    for i in (0, 3, 40):
        for d in (-1e-12, 1e-12):
            us.append(float(cum[i] + d))
            xs.append(x)
    cfg = gs.DecodingConfig(temperature=T, topK=0, topP=1.0, repetitionWindow=0)
    cfgs = [cfg] * len(us)
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(np.stack(xs)).cuda(), conf)
    check(gs, oracle, "draw boundary", out, xs, None, cfgs, us)
    assert np.all(out.flags & gs.GS_FLAG_EXACT_PATH), out.flags


def test_full_vocabulary_draws_bf16_and_softcap(sampler, oracle):
    """Full-vocabulary draws whose cursors sit deep in the tail (u near 1),
    so that most rows take the deep draw: bf16 rows (its gather reads eight
    logits per 16-byte piece), and f32 and bf16 rows with softcap 30 (the
    capped loop), each against the oracle on the same values, once with the
    deep draws spread over many workgroups and once on each row's own."""
    import torch

    gs = _gs()
    n = 16
    w = gs.workloads.multinomial(rows=list(range(n)))
    us = [1 - 2 ** -32, 0.9999, 0.999, 0.995, 0.99, 0.98, 0.97, 0.95] * 2
    temps = [1.0, 0.9, 1.0, 0.8] * 4
    cfgs = [c.merged(temperature=t) for c, t in zip(w.configs, temps)]
    bits = gs.workloads.to_bf16_bits(w.logits)
    xb = gs.workloads.bf16_bits_to_f32(bits).reshape(n, V)
    dev_b = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    deep = 0
    for label, dev, xin, cap in (("bf16", dev_b, xb, 0.0), ("f32 softcap", torch.from_numpy(w.logits).cuda(),
                                                         w.logits, 30.0), ("bf16 softcap", dev_b, xb, 30.0)):
        conf = np.stack([gs.runtime.row_config(c, uniform=u, softcap_value=cap) for c, u in zip(cfgs, us)])
        vals = [oracle.softcap(xin[r], cap) if cap > 0 else xin[r] for r in range(n)]
        # the deep draw over many workgroups (the batch hint), then on each
        # row's own workgroup (no hint): the same ids
        outs = [sampler.sample(dev, conf), sampler.sample(dev, conf, hints=0)]
        for tag, out in zip(("multi", "single"), outs):
            check(gs, oracle, f"{label} {tag}", out, vals, None, cfgs, us)
            deep += int(np.sum((out.flags & gs.GS_FLAG_EXACT_PATH) == 0))
        assert np.array_equal(outs[0].tokens, outs[1].tokens)
    assert deep > 0


def test_lone_row_deep_draws(sampler, oracle):
    """Small calls (interactive decoding) whose cursor sits deep in the tail:
    one-row calls keep the deep draw on the row's own workgroup, and a
    four-row call of the same rows spreads it over many workgroups (a part per
    chunk for each row); penalty-window ids below the region floor on some
    rows. The same ids as the oracle either way."""
    import torch

    gs = _gs()
    w = gs.workloads.multinomial(rows=list(range(6)))
    us = [1 - 2 ** -32, 0.9999, 0.999, 0.9995, 0.99995, 0.9999]
    temps = [1.0, 0.8, 1.0, 0.9, 1.0, 0.8]
    deep = 0
    for r in range(6):
        cfg = w.configs[r].merged(temperature=temps[r])
        hist = None
        if r % 2:
            # window ids from the tail (ranks 5000..50000), lowered by the penalty
            order = np.argsort(-w.logits[r])
            hist = [order[5000:50000:1500].tolist()]
            cfg = cfg.merged(repetitionPenalty=1.3, repetitionWindow=64)
        conf = np.stack([gs.runtime.row_config(cfg, uniform=us[r])])
        x = torch.from_numpy(w.logits[r:r + 1]).cuda()
        out = sampler.sample(x, conf, histories=hist)
        check(gs, oracle, f"lone row {r}", out, [w.logits[r]], hist, [cfg], [us[r]])
        deep += int((out.flags[0] & gs.GS_FLAG_EXACT_PATH) == 0)
        # the row four times in one call: the multi-workgroup deep draw
        out4 = sampler.sample(torch.from_numpy(np.repeat(w.logits[r:r + 1], 4, axis=0)).cuda(),
                              np.concatenate([conf] * 4), histories=hist * 4 if hist else None)
        for k in range(4):
            assert int(out4.tokens[k]) == int(out.tokens[0]), (r, k)
            assert abs(out4.probabilities[k] - out.probabilities[0]) <= PROB_RTOL * out.probabilities[0]
    assert deep > 0


@pytest.mark.parametrize("Vs", [8269, 20000, 32768])
def test_small_region_full_draws(oracle, Vs):
    """Full-vocabulary draws on vocabularies of two to four chunks, whose
    complete region (64 list entries per chunk) holds at most 256 entries:
    the finish's prefix ranking returns early for them, and cursors past the
    region go to the deep draw. Over many workgroups (the batch hint), on each
    row's own (no hint) and as lone rows, penalty windows on some rows: the
    oracle's ids every time."""
    import torch

    gs = _gs()
    rng = np.random.default_rng(Vs)
    n = 24
    rows, cfgs, us, hists = [], [], [], []
    for r in range(n):
        x = rng.normal(0, [0.5, 1.0, 2.0][r % 3], Vs).astype(np.float32)
        rows.append(x)
        cfg = gs.DecodingConfig(temperature=[0.7, 1.0, 1.3][(r // 3) % 3], topK=0, topP=1.0, minP=0.0,
                                typicalP=1.0, repetitionWindow=0)
        hist = []
        if r % 4 == 1:
            hist = rng.integers(0, Vs, 8).tolist()
            cfg = cfg.merged(repetitionPenalty=2.0, repetitionWindow=8)
        cfgs.append(cfg)
        hists.append(hist)
        us.append(float(rng.uniform(0.3, 0.999)))
    s = gs.Sampler(vocab_size=Vs, max_rows=n)
    try:
        conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
        x = torch.from_numpy(np.stack(rows)).cuda()
        multi = s.sample(x, conf, histories=hists)
        single = s.sample(x, conf, histories=hists, hints=0)
        lone = [s.sample(x[r:r + 1], conf[r:r + 1], histories=[hists[r]]) for r in range(0, n, 5)]
    finally:
        s.close()
    check(gs, oracle, f"V={Vs} multi", multi, rows, hists, cfgs, us)
    check(gs, oracle, f"V={Vs} single", single, rows, hists, cfgs, us)
    assert np.array_equal(multi.tokens, single.tokens)
    for k, r in enumerate(range(0, n, 5)):
        assert int(lone[k].tokens[0]) == int(multi.tokens[r]), (Vs, r)
    # most rows are deep draws (one pass over the row), not exact replays
    assert int(np.sum((multi.flags & gs.GS_FLAG_EXACT_PATH) == 0)) >= n // 2, multi.flags


@pytest.mark.parametrize("Vs", [3000, 40000])
def test_typical_p_pool_past_finite_logits(oracle, Vs):
    """typical-p with top-k on rows holding fewer finite logits than topK (a
    mask with few legal ids, or mostly -inf logits): the reference's pool is
    still the first topK entries of its list, so entries of probability 0
    join it and their p ln p turns the entropy NaN (sampling.ts:44,49-55),
    which leaves the pool in list order for the typicalP cut. With min-p those
    entries leave the pool first. The oracle's ids (the same as V8's) on every
    row, constrained and not."""
    import torch

    gs = _gs()
    rng = np.random.default_rng(Vs + 1)
    n_legal = [1, 4, 33, 63, 64, 200]
    words = np.zeros((len(n_legal), (Vs + 31) // 32), np.uint32)
    legal_sets = []
    for k, m in enumerate(n_legal):
        legal = np.sort(rng.choice(Vs, m, replace=False)).astype(np.int32)
        np.bitwise_or.at(words[k], legal >> 5, np.left_shift(np.uint32(1), (legal & 31).astype(np.uint32)))
        legal_sets.append(legal)
    rows, cfgs, us, slots, vals = [], [], [], [], []
    for r in range(36):
        x = rng.normal(0, [0.5, 2.0, 4.0][r % 3], Vs).astype(np.float32)
        slot = r % 7 - 1  # -1: unconstrained
        if slot < 0 and r % 2:
            x[rng.random(Vs) < 0.99] = -np.inf  # about 30 (V 3000) or 400 finite logits
        rows.append(x)
        slots.append(slot)
        vals.append(oracle.mask_logits(x, legal_sets[slot], []) if slot >= 0 else x)
        cfgs.append(gs.DecodingConfig(temperature=[0.7, 1.0, 1.5][r % 3], topK=[64, 40, 5, 64][r % 4],
                                      typicalP=[0.3, 0.9, 0.6][(r // 3) % 3], topP=[1.0, 0.95][r % 2],
                                      minP=0.05 if r % 5 == 4 else 0.0, repetitionWindow=0))
        us.append(float(rng.random()))
    s = gs.Sampler(vocab_size=Vs, max_rows=64)
    try:
        conf = np.stack([gs.runtime.row_config(c, uniform=u, mask_slot=m) for c, u, m in zip(cfgs, us, slots)])
        table = torch.from_numpy(words.view(np.int32)).cuda()
        out = s.sample(torch.from_numpy(np.stack(rows)).cuda(), conf, mask_table=table)
    finally:
        s.close()
    check(gs, oracle, f"typical past finite V={Vs}", out, vals, None, cfgs, us)


def test_topk_above_64(sampler, oracle):
    """topK 65 .. 2000 keep 64 entries per chunk; the finish ranks the
    complete region (block-wide) and cuts it at K."""
    import torch

    gs = _gs()
    w = gs.workloads.topk_deep(rows=list(range(24)))
    ks = [65, 100, 200, 500, 1000, 2000] * 4
    ps = [1.0, 0.95, 0.9, 0.5] * 6
    cfgs = [c.merged(topK=k, topP=p, minP=0.01 if r % 5 == 0 else 0.0) for r, (c, k, p) in
            enumerate(zip(w.configs, ks, ps))]
    us = [float(u) for u in np.random.default_rng(4).random(24)]
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf)
    exact = check(gs, oracle, "topk>64", out, w.logits, None, cfgs, us)
    assert exact <= 4, exact


def test_pools_past_64_with_window_ids(sampler, oracle):
    """Top-p pools of hundreds of candidates, and top-k ones of 300 and 1500:
    the finish ranks only the prefix of the candidate list that holds the pool
    (a key histogram with each bin's mass picks where ranking may stop), so
    window ids ranked inside the pool, around its end and below it (raised by
    a repetition penalty below 1, lowered by one above it) must land where the
    reference puts them; min-p rows beside them."""
    import torch

    gs = _gs()
    rows = 24
    g = np.random.default_rng(11)
    xs = g.normal(0, 3, (rows, V)).astype(np.float32)
    hists, cfgs = [], []
    for r in range(rows):
        order = np.argsort(-xs[r], kind="stable")
        hists.append(order[g.integers(0, 3000, 300)].tolist())
        cfgs.append(gs.DecodingConfig(
            temperature=[1.0, 0.8, 0.9, 1.0, 0.8, 1.0][r % 6], topK=[0, 0, 0, 1500, 300, 0][r % 6],
            topP=[0.5, 0.8, 0.75, 0.95, 0.8, 0.95][r % 6], minP=0.001 if r % 6 == 5 or r % 4 == 0 else 0.0,
            typicalP=1.0,
            repetitionPenalty=[1.05, 0.9, 1.0, 1.2][r % 4], repetitionWindow=512,
            frequencyPenalty=0.05 if r % 2 else 0.0, presencePenalty=0.2 if r % 4 == 2 else 0.0))
    us = [float(u) for u in g.random(rows)]
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(xs).cuda(), conf, histories=hists)
    exact = check(gs, oracle, "pools>64", out, xs, hists, cfgs, us)
    assert exact <= 4, exact


def test_typical_p_with_top_k(sampler, oracle):
    """typicalP with topK <= 64: entropy, the surprise order, its leading
    mass and the kept set back in list order, in one wave; with min-p, top-p
    and penalties alongside."""
    import torch

    gs = _gs()
    w = gs.workloads.typical(rows=list(range(32)))
    rng = np.random.default_rng(6)
    cfgs = []
    for r, c in enumerate(w.configs):
        cfgs.append(c.merged(topK=int(rng.choice([5, 20, 40, 64])), typicalP=float(rng.choice([0.9, 0.5, 0.3, 0.99])),
                             topP=float(rng.choice([1.0, 0.95, 0.8])), minP=float(rng.choice([0.0, 0.0, 0.02])),
                             temperature=float(rng.choice([0.6, 0.8, 1.0, 1.5]))))
    hists = [rng.integers(0, V, 100).tolist() for _ in range(32)]
    cfgs = [c.merged(repetitionPenalty=1.1, repetitionWindow=100) if r % 4 == 0 else c for r, c in enumerate(cfgs)]
    us = [float(u) for u in rng.random(32)]
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf, histories=hists)
    exact = check(gs, oracle, "typical", out, w.logits, hists, cfgs, us)
    assert exact <= 4, exact


def test_typical_workload_matches_oracle(sampler, oracle):
    """The typical workload's 256 rows (topK 40, typicalP 0.9) against the
    oracle. Row 180 holds two items on the same side of the entropy whose
    surprises lie within the normaliser's margin of each other: their order
    does not depend on the normaliser (a common shift of every signed
    surprise), so the row is settled without the binary64 recompute."""
    import torch

    gs = _gs()
    w = gs.workloads.typical()
    conf = np.stack([gs.runtime.row_config(c, seed=sd) for c, sd in zip(w.configs, w.seeds)])
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf)
    us = [oracle.draw(sd, 0) for sd in w.seeds]
    exact = check(gs, oracle, "typical workload", out, w.logits, None, w.configs, us)
    assert exact == 0, exact


def test_typical_p_ties_and_small_pools(oracle):
    """typical-p on small vocabularies with repeated values (equal surprises,
    stable order) and a pool of one, against the oracle."""
    import torch

    gs = _gs()
    Vs = 5000
    rng = np.random.default_rng(8)
    rows, cfgs, us = [], [], []
    for r in range(24):
        x = rng.normal(0, 2, Vs).astype(np.float32)
        if r % 2 == 0:
            x = (np.round(x * 2) / 2).astype(np.float32)
        rows.append(x)
        cfgs.append(gs.DecodingConfig(temperature=1.0, topK=int(rng.choice([1, 3, 16, 64])),
                                      typicalP=float(rng.choice([0.2, 0.6, 0.95])), topP=1.0, minP=0.0,
                                      repetitionWindow=0))
        us.append(float(rng.random()))
    s = gs.Sampler(vocab_size=Vs, max_rows=32)
    try:
        conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
        out = s.sample(torch.from_numpy(np.stack(rows)).cuda(), conf)
    finally:
        s.close()
    check(gs, oracle, "typical small", out, rows, None, cfgs, us)
