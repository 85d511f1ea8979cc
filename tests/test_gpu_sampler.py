"""GPU parity of the batched sampler (gs_sample through the C ABI) against the
oracle: token ids bit-exact on every row; probabilities identical on rows the
exact path resolved and within PROB_RTOL relative on one-pass rows.

One-pass rows take their softmax normaliser from the chunk scan, which sums
binary32 terms from the hardware exp2 (relative error of a chunk sum at most
3.9e-7; the derivation is in gs_scan.hip), so one-pass probabilities carry up
to that relative error (PROB_RTOL adds the binary64 roundings); rows whose
top-p cut fell within that bound recompute the normaliser in binary64
(4.2e-10 per term). The path's stated bound is 1e-6 relative."""
import math

import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

PROB_RTOL = 4e-7


def _gs():
    import gsample

    return gsample


def to_oracle_cfg(c):
    return Decoding(temperature=c.temperature, topK=c.topK, topP=c.topP, minP=c.minP, typicalP=c.typicalP,
                    repetitionPenalty=c.repetitionPenalty, repetitionWindow=c.repetitionWindow,
                    frequencyPenalty=c.frequencyPenalty, presencePenalty=c.presencePenalty)


def assert_rows_match(out, expected, flags_ok=None, label=""):
    gs = _gs()
    for i, (t, p) in enumerate(expected):
        assert out.tokens[i] == t, f"{label} row {i}: token {out.tokens[i]} != {t} (flags {out.flags[i]})"
        assert not out.flags[i] & gs.GS_FLAG_INDEX_CHECK, (label, i, int(out.flags[i]))
        if out.flags[i] & gs.GS_FLAG_EXACT_PATH:
            assert out.probabilities[i] == p or (math.isnan(p) and math.isnan(out.probabilities[i])), (label, i)
        else:
            assert abs(out.probabilities[i] - p) <= PROB_RTOL * abs(p), (label, i, out.probabilities[i], p)


# ------------------------------------------------------------ reference tests


def test_reference_known_answers_on_gpu():
    """tests/sampling.spec.ts:13-139 through the drop-in sample_token."""
    gs = _gs()
    D = gs.DEFAULT_DECODING_CONFIG
    assert gs.sample_token([0.2, 4, 1], [], D.merged(temperature=0), lambda: 0.5) == 1
    assert gs.sample_token([0.2, 4, 1], [], D.merged(topK=1), lambda: 0.99) == 1
    cfg = D.merged(topK=0, topP=1)
    r1, r2 = gs.SeededRandom(71), gs.SeededRandom(71)
    a = [gs.sample_token([1, 1, 1], [], cfg, r1.next) for _ in range(20)]
    b = [gs.sample_token([1, 1, 1], [], cfg, r2.next) for _ in range(20)]
    assert a == b
    assert gs.sample_token([2, 1.5], [0], D.merged(temperature=0, repetitionPenalty=2), lambda: 0) == 1
    assert gs.sample_token([2, 1.5], [0], D.merged(temperature=0, repetitionPenalty=2, repetitionWindow=0),
                           lambda: 0) == 0
    pf = D.merged(temperature=0, repetitionPenalty=1, repetitionWindow=2, presencePenalty=0.1, frequencyPenalty=0.3)
    assert gs.sample_token([2, 1.5], [0, 0], pf, lambda: 0) == 1
    assert gs.sample_token([2, 2.1], [0, 1], pf.merged(repetitionWindow=1, presencePenalty=0.5, frequencyPenalty=0),
                           lambda: 0) == 0
    l3 = [math.log(0.6), math.log(0.3), math.log(0.1)]
    assert gs.sample_token(l3, [], D.merged(temperature=1, topK=0, topP=1, typicalP=1, minP=0.6), lambda: 0.99) == 0
    assert gs.sample_token(l3, [], D.merged(temperature=1, topK=0, topP=0.5, minP=0, typicalP=1), lambda: 0.99) == 0
    lt = [math.log(0.45), math.log(0.4), math.log(0.15)]
    assert gs.sample_token(lt, [], D.merged(temperature=1, topK=0, topP=1, minP=0, typicalP=0.3), lambda: 0.5) == 1
    assert gs.token_log_probability(l3, 0) == pytest.approx(math.log(0.6), abs=1e-6)
    assert gs.token_log_probability(l3, 2) == pytest.approx(math.log(0.1), abs=1e-6)
    with pytest.raises(gs.GSampleError, match="outside logits length"):
        gs.token_log_probability(l3, 3)


def test_random_never_called_for_greedy():
    gs = _gs()
    calls = []

    def rnd():
        calls.append(1)
        return 0.5

    gs.sample_token([0.1, 0.2], [], gs.DEFAULT_DECODING_CONFIG.merged(temperature=0), rnd)
    assert calls == []
    gs.sample_token([0.1, 0.2], [], gs.DEFAULT_DECODING_CONFIG, rnd)
    assert calls == [1]


# ------------------------------------------------------- random small vocabs


def _random_batch(seed, rows, V):
    rng = np.random.default_rng(seed)
    gs = _gs()
    logits = np.empty((rows, V), dtype=np.float32)
    hists, cfgs, us = [], [], []
    for r in range(rows):
        x = rng.normal(0, rng.uniform(0.5, 4), V).astype(np.float32)
        if rng.random() < 0.3:
            x = (np.round(x * 4) / 4).astype(np.float32)
        if rng.random() < 0.15:
            x[rng.random(V) < 0.8] = -np.inf
        logits[r] = x
        hists.append(rng.integers(-2, V + 2, int(rng.integers(0, 80))).tolist())
        cfgs.append(gs.DecodingConfig(
            temperature=float(rng.choice([0.0, 0.5, 0.8, 1.0, 1.7])),
            topK=int(rng.choice([0, 1, 5, 40, 64, 300])),
            topP=float(rng.choice([1.0, 0.95, 0.5, 0.9, 0.1])),
            minP=float(rng.choice([0.0, 0.0, 0.05, 0.3])),
            typicalP=float(rng.choice([1.0, 1.0, 1.0, 0.9, 0.3])),
            repetitionPenalty=float(rng.choice([1.0, 1.1, 2.0])),
            repetitionWindow=int(rng.choice([0, 8, 64])),
            frequencyPenalty=float(rng.choice([0.0, 0.3])),
            presencePenalty=float(rng.choice([0.0, 0.5]))))
        us.append(float(rng.random()))
    return logits, hists, cfgs, us


# (False, 8269, 2) holds full-vocabulary draws (row 6 among them) whose cursor
# lies past a region of under 256 entries: the finish's prefix ranking returns
# early for them, and every thread reads the region mass it leaves in LDS only
# after a barrier (without it a wave could read the word before it was written
# and leave the workgroup's barriers out of step).
@pytest.mark.parametrize("force_exact,V,seed", [
    (False, 3000, 1),
    (False, 8192 + 77, 2),
    (False, 40000, 3),
    (True, 3000, 1),
    (True, 8192 + 77, 2),
    (True, 40000, 3),
])
def test_random_batches_match_oracle(oracle, V, seed, force_exact):
    import torch

    gs = _gs()
    rows = 96
    logits, hists, cfgs, us = _random_batch(seed, rows, V)
    s = gs.Sampler(vocab_size=V, max_rows=rows)
    try:
        conf = np.stack([gs.runtime.row_config(c, uniform=u, force_exact=force_exact) for c, u in zip(cfgs, us)])
        out = s.sample(torch.from_numpy(logits).cuda(), conf, histories=hists, raise_on_failure=False)
    finally:
        s.close()
    expected = []
    for r in range(rows):
        t, tr = oracle.sample_token(logits[r], hists[r], to_oracle_cfg(cfgs[r]), us[r])
        expected.append((t, tr.probability if t >= 0 else 0.0))
    for r, (t, p) in enumerate(expected):
        if t < 0:
            assert out.flags[r] & gs.GS_FLAG_EMPTY_CANDIDATES
            expected[r] = (int(out.tokens[r]), float(out.probabilities[r]))
    assert_rows_match(out, expected, label=f"V={V}")
    if force_exact:
        for r in range(rows):
            if cfgs[r].temperature > 0:
                assert out.flags[r] & gs.GS_FLAG_EXACT_PATH


# ------------------------------------------------------------- full-size rows


def test_exact_rows_beyond_the_context_slots(oracle):
    """A finish workgroup replays an exact-path row itself when the row has a
    scratch slot of its own (row < slots); the rows past the slots wait in the
    device queue for the exact kernel, which the call launches only for batches
    with more rows than slots. At V = 2^21 a context keeps 170 slots, so in a
    180-row batch with rows 166-179 forced onto the exact path rows 166-169 are
    replayed in place and rows 170-179 by the exact kernel: both give the
    oracle's ids and bit-exact probabilities."""
    import torch

    gs = _gs()
    V, rows = 1 << 21, 180
    slots = 12 * 2**30 // (36 * V)  # 170 slots of 36 * 2^21 bytes in the 12 GiB budget
    rng = np.random.default_rng(17)
    logits = rng.standard_normal((rows, V), dtype=np.float32) * np.float32(2.5)
    forced = list(range(slots - 4, rows))
    cfg_forced = gs.DecodingConfig(temperature=0.8, topK=40, topP=0.9)
    cfg_greedy = gs.DecodingConfig(temperature=0.0)
    us = [float(u) for u in rng.random(rows)]
    conf = np.stack([gs.runtime.row_config(cfg_forced if r in forced else cfg_greedy, uniform=us[r],
                                           force_exact=r in forced) for r in range(rows)])
    s = gs.Sampler(vocab_size=V, max_rows=rows)
    try:
        x = torch.from_numpy(logits).cuda()
        s.timing_begin(2)
        out = s.sample(x, conf)
        out_small = s.sample(x[:slots], conf[:slots])
        stages = s.timing_end()
    finally:
        s.close()
    assert stages["exact"][1] == 1, stages  # launched for the 180-row batch only
    for r in range(rows):
        if r in forced:
            t, tr = oracle.sample_token(logits[r], [], to_oracle_cfg(cfg_forced), us[r])
            assert out.flags[r] & gs.GS_FLAG_EXACT_PATH, r
            assert int(out.tokens[r]) == t and out.probabilities[r] == tr.probability, (r, int(out.tokens[r]), t)
        else:
            assert int(out.tokens[r]) == int(np.argmax(logits[r])), r
    assert list(out_small.tokens) == list(out.tokens[:slots])


def test_topk_deeper_than_chunk_lists(sampler, oracle):
    """Top-k rows list at most 16 entries' worth of depth per chunk; rows whose
    top K crowd into one chunk (here the 60 largest logits, one per lane of
    one chunk) leave fewer than K candidates above the lists' threshold, and
    must still come out as the oracle's ids (by the block-wide or exact
    path)."""
    import torch

    gs = _gs()
    V = 262144
    rng = np.random.default_rng(5)
    rows, cfgs = [], []
    for k, start in ((50, 0), (64, 8192 * 7), (40, 8192 * 31)):
        x = rng.normal(0, 1, V).astype(np.float32)
        ids = start + 4 * np.arange(60)  # thread t's first element, t = 0..59
        x[ids] = 8.0 + rng.normal(0, 0.3, ids.size).astype(np.float32)
        rows.append(x)
        cfgs.append(gs.DecodingConfig(temperature=1.0, topK=k, topP=0.97, repetitionPenalty=1.0, repetitionWindow=0))
    us = [0.11, 0.5, 0.93]
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(np.stack(rows)).cuda(), conf)
    exp = []
    for x, c, u in zip(rows, cfgs, us):
        t, tr = oracle.sample_token(x, [], to_oracle_cfg(c), u)
        exp.append((t, tr.probability))
    assert_rows_match(out, exp, label="crowded_topk")


def test_hardware_exp2_bound(sampler):
    """The chunk scan evaluates every normaliser term with v_exp_f32 and its
    error bound (3.9e-7 per chunk sum) assumes the instruction is within 1e-7
    relative of 2^y over [-150, 2^-10]: checked here at every binary32 y of
    that range whose result is normal, on the device the kernels run on."""
    err, y = sampler.check_exp2(-150.0, 2.0 ** -10)
    assert 0 < err <= 1e-7, (err, y)


def test_topp_cut_inside_scan_normaliser_bound(sampler, oracle):
    """Top-p cuts placed within the scan normaliser's bound (3.9e-7 relative)
    of topP: beyond 4e-9 the finish kernel settles them with its binary64
    recomputation of the normaliser (one-pass rows, no exact replay), inside
    it the exact replay does; either way the ids are the oracle's. Two rows
    shapes: a cut inside the top 50 (the one-wave filters) and a cut near 280
    candidates deep (the block-wide filters)."""
    import torch

    gs = _gs()
    V = 262144
    rng = np.random.default_rng(11)
    # 40 raised logits (about 96% of the mass) spread over the chunks
    peaked = rng.normal(0, 1, V).astype(np.float32)
    top = (np.arange(32)[:, None] * 8192 + 100 + np.arange(2)[None, :]).reshape(-1)[:40]
    peaked[top] = 12.0 + rng.normal(0, 1, top.size).astype(np.float32)
    deep = rng.normal(0, 1, V).astype(np.float32)
    raised = (np.arange(32)[:, None] * 8192 + np.arange(10)[None, :]).reshape(-1)
    deep[raised] = 12.0 + rng.normal(0, 0.5, raised.size).astype(np.float32)
    xs, cfgs, exact = [], [], []
    for x, k in ((peaked, 50), (deep, 0)):
        probe = gs.DecodingConfig(temperature=1.0, topK=k, topP=0.9, repetitionPenalty=1.0, repetitionWindow=0)
        _, tr = oracle.sample_token(x, [], to_oracle_cfg(probe), 0.5)
        cum = tr.cumulative_at_cut
        assert 0.9 <= cum < 1.0, cum
        for rel, want_exact in ((-1e-8, False), (1e-8, False), (-3e-7, False), (2e-7, False), (-1e-11, True)):
            xs.append(x)
            cfgs.append(probe.merged(topP=cum * (1.0 + rel)))
            exact.append(want_exact)
    us = [0.37 + 0.05 * i for i in range(len(xs))]
    conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out = sampler.sample(torch.from_numpy(np.stack(xs)).cuda(), conf)
    expected = []
    for x, c, u in zip(xs, cfgs, us):
        t, tr = oracle.sample_token(x, [], to_oracle_cfg(c), u)
        expected.append((t, tr.probability))
    assert_rows_match(out, expected, label="topp_near")
    for r, want_exact in enumerate(exact):
        assert bool(out.flags[r] & gs.GS_FLAG_EXACT_PATH) == want_exact, (r, int(out.flags[r]))
        assert out.flags[r] & gs.GS_FLAG_TOPP_TIE, (r, int(out.flags[r]))



def test_constrained_topp_cut_inside_scan_normaliser_bound(sampler, oracle):
    """Constrained rows (about 3% of ids legal, the first and last ids among
    them) whose top-p cut lies within the scan normaliser's bound: the
    binary64 recomputation visits only the legal ids, by the mask words' set
    bits. Ids and probabilities are the oracle's; the cuts beyond 4e-9 stay
    on the one-pass path, the one inside it takes the exact replay."""
    import torch

    gs = _gs()
    V = 262144
    rng = np.random.default_rng(23)
    x = rng.normal(0, 3, V).astype(np.float32)
    legal = np.union1d(rng.choice(V, V // 32, replace=False), [0, V - 2, V - 1])
    words = np.zeros(V // 32, np.uint32)
    np.bitwise_or.at(words, legal >> 5, np.left_shift(np.uint32(1), (legal & 31).astype(np.uint32)))
    assert np.array_equal(oracle.mask_bits_to_ids(words, V), legal)
    masked = oracle.mask_logits(x, legal, [])
    probe = gs.DecodingConfig(temperature=1.0, topK=0, topP=0.95, repetitionPenalty=1.0, repetitionWindow=0)
    _, tr = oracle.sample_token(masked, [], to_oracle_cfg(probe), 0.5)
    cum = tr.cumulative_at_cut
    assert 0.95 <= cum < 1.0, cum
    rels = ((-1e-8, False), (1e-8, False), (-3e-7, False), (2e-7, False), (-1e-11, True))
    cfgs = [probe.merged(topP=cum * (1.0 + rel)) for rel, _ in rels]
    us = [0.41 + 0.1 * i for i in range(len(rels))]
    conf = np.stack([gs.runtime.row_config(c, uniform=u, mask_slot=0) for c, u in zip(cfgs, us)])
    masks = torch.from_numpy(words.view(np.int32)[None].copy()).cuda()
    out = sampler.sample(torch.from_numpy(np.stack([x] * len(rels))).cuda(), conf, mask_table=masks)
    expected = []
    for c, u in zip(cfgs, us):
        t, trc = oracle.sample_token(masked, [], to_oracle_cfg(c), u)
        expected.append((t, trc.probability))
    assert_rows_match(out, expected, label="constrained topp_near")
    for r, (_, want_exact) in enumerate(rels):
        assert bool(out.flags[r] & gs.GS_FLAG_EXACT_PATH) == want_exact, (r, int(out.flags[r]))
        assert out.flags[r] & gs.GS_FLAG_TOPP_TIE, (r, int(out.flags[r]))


def test_single_row_config(sampler, oracle):
    import torch

    gs = _gs()
    w = gs.workloads.single_row()
    conf = gs.runtime.row_config(w.configs[0], seed=42).reshape(1)
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf)
    t, tr = oracle.sample_token(w.logits[0], [], to_oracle_cfg(w.configs[0]), oracle.draw(42, 0))
    assert_rows_match(out, [(t, tr.probability)], label="single_row")


def test_penalties_batch(sampler, oracle):
    import torch

    gs = _gs()
    w = gs.workloads.penalties()
    conf = np.stack([gs.runtime.row_config(c, seed=s) for c, s in zip(w.configs, w.seeds)])
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf, histories=w.histories)
    pick = list(range(0, 256, 8))
    exp = []
    for r in pick:
        t, tr = oracle.sample_token(w.logits[r], w.histories[r], to_oracle_cfg(w.configs[r]), oracle.draw(w.seeds[r], 0))
        exp.append((t, tr.probability))
    sub = gs.runtime.SampleOutput(out.tokens[pick], out.probabilities[pick], out.flags[pick])
    assert_rows_match(sub, exp, label="penalties")
    # every row was settled by the one-pass path (no margin within 1e-10)
    assert not np.any(out.flags & gs.GS_FLAG_EXACT_PATH), out.flags


def test_heavy_tail_bf16(sampler, oracle):
    import torch

    gs = _gs()
    rows = list(range(0, 1024, 64))
    w = gs.workloads.heavy_tail(rows=rows)
    conf = np.stack([gs.runtime.row_config(c, seed=s) for c, s in zip(w.configs, w.seeds)])
    x = torch.from_numpy(w.logits.view(np.int16)).cuda().view(torch.bfloat16)
    out = sampler.sample(x, conf)
    exp = []
    for i, r in enumerate(rows):
        f = gs.workloads.bf16_bits_to_f32(w.logits[i])
        t, tr = oracle.sample_token(f, [], to_oracle_cfg(w.configs[i]), oracle.draw(w.seeds[i], 0))
        exp.append((t, tr.probability))
    assert_rows_match(out, exp, label="heavy_tail")


def test_constrained_bf16_mixed_batch(sampler, oracle):
    """bf16 logits with a mask table: constrained rows (about 3% of ids
    legal) and unconstrained rows (no mask slot) in one batch run the bf16
    constrained scan variant through both its masked and its unmasked group
    scan. Ids and probabilities are the oracle's on the same bf16 values."""
    import torch

    gs = _gs()
    V = 262144
    rng = np.random.default_rng(31)
    x32 = rng.normal(0, 3, (6, V)).astype(np.float32)
    u32 = x32.view(np.uint32)
    bits = ((u32 + np.uint32(0x7FFF) + ((u32 >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    legal = np.union1d(rng.choice(V, V // 32, replace=False), [0, V - 1])
    words = np.zeros(V // 32, np.uint32)
    np.bitwise_or.at(words, legal >> 5, np.left_shift(np.uint32(1), (legal & 31).astype(np.uint32)))
    slots = [0, -1, 0, -1, 0, -1]
    base = gs.DecodingConfig(temperature=1.0, topK=0, topP=0.9, repetitionPenalty=1.0, repetitionWindow=0)
    cfgs = [base, base.merged(topK=40, temperature=0.8), base.merged(topP=0.95), base.merged(topK=64),
            base.merged(temperature=0.0), base.merged(temperature=0.0)]
    us = [0.13 + 0.14 * i for i in range(6)]
    conf = np.stack([gs.runtime.row_config(c, uniform=u, mask_slot=m) for c, u, m in zip(cfgs, us, slots)])
    masks = torch.from_numpy(words.view(np.int32)[None].copy()).cuda()
    x = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    out = sampler.sample(x, conf, mask_table=masks)
    expected = []
    for i in range(6):
        f = gs.workloads.bf16_bits_to_f32(bits[i])
        if slots[i] >= 0:
            f = oracle.mask_logits(f, legal, [])
        t, tr = oracle.sample_token(f, [], to_oracle_cfg(cfgs[i]), us[i])
        expected.append((t, tr.probability))
    assert_rows_match(out, expected, label="constrained bf16 mixed")


def test_constrained_masks_and_samples(sampler, oracle, synthetic_constraint):
    import torch

    gs = _gs()
    offsets, data, nxt, finals, ref_masks = synthetic_constraint
    sampler.set_vocab(offsets, data)
    sampler.set_dfa(nxt, finals)
    states = list(range(64))
    table = sampler.build_masks(states).cpu().numpy().view(np.uint32)
    for s in states:
        assert np.array_equal(table[s], ref_masks[s]), s
    frac = np.mean([oracle.mask_bits_to_ids(ref_masks[s], 262144).size for s in states]) / 262144
    assert 0.005 < frac < 0.1
    rows = list(range(0, 128, 8))
    for greedy in (True, False):
        w = gs.workloads.constrained(rows=rows, greedy=greedy)
        masks = torch.from_numpy(table.view(np.int32)).cuda()
        conf = np.stack([gs.runtime.row_config(c, seed=s, mask_slot=int(st))
                         for c, s, st in zip(w.configs, w.seeds, w.states)])
        out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf, mask_table=masks)
        exp = []
        for i in range(len(rows)):
            legal = oracle.mask_bits_to_ids(ref_masks[w.states[i]], 262144)
            masked = oracle.mask_logits(w.logits[i], legal, [])
            t, tr = oracle.sample_token(masked, [], to_oracle_cfg(w.configs[i]), oracle.draw(w.seeds[i], 0))
            exp.append((t, tr.probability))
        assert_rows_match(out, exp, label=f"constrained greedy={greedy}")


# ---------------------------------------------------------------- edge cases


def test_edge_cases(oracle):
    import torch

    gs = _gs()
    V = 10000
    s = gs.Sampler(vocab_size=V, max_rows=16)
    try:
        base = gs.DecodingConfig(temperature=1.0, topK=0, topP=0.9, minP=0, typicalP=1, repetitionPenalty=1,
                                 repetitionWindow=0)
        rows = []
        # all equal logits (one giant tie), greedy and sampled
        rows.append((np.zeros(V, np.float32), [], base, 0.37))
        rows.append((np.zeros(V, np.float32), [], base.merged(temperature=0), 0.0))
        rows.append((np.zeros(V, np.float32), [], base.merged(topK=10), 0.99))
        # -0 and +0 tie by id
        z = np.zeros(V, np.float32)
        z[5] = -0.0
        z[3] = -0.0
        rows.append((z, [], base.merged(temperature=0), 0.0))
        # a single finite logit among -inf
        one = np.full(V, -np.inf, np.float32)
        one[777] = -3.0
        rows.append((one, [], base, 0.5))
        rows.append((one, [], base.merged(topK=5), 0.999))
        # top-k larger than the finite set
        few = np.full(V, -np.inf, np.float32)
        few[[10, 20, 30]] = [1.0, 2.0, 3.0]
        rows.append((few, [], base.merged(topK=50, topP=1.0), 0.75))
        # huge spread: exp underflow in the normaliser
        wide = np.linspace(-2000, 10, V).astype(np.float32)
        rows.append((wide, [], base.merged(topP=0.999999), 0.8))
        # extreme temperatures go to the exact path
        x = np.random.default_rng(0).normal(0, 3, V).astype(np.float32)
        rows.append((x, [], base.merged(temperature=1e-250), 0.3))
        rows.append((x, [], base.merged(temperature=1e250), 0.3))
        # penalties on every id of a long window
        rows.append((x, list(range(V)) * 2, base.merged(repetitionPenalty=1.3, repetitionWindow=2000, topK=20), 0.6))
        # u = 0 and u just below 1
        rows.append((x, [], base.merged(topK=40, topP=0.95), 0.0))
        rows.append((x, [], base.merged(topK=40, topP=0.95), 1 - 2 ** -32))
        logits = np.stack([r[0] for r in rows])
        conf = np.stack([gs.runtime.row_config(r[2], uniform=r[3]) for r in rows])
        out = s.sample(torch.from_numpy(logits).cuda(), conf, histories=[r[1] for r in rows])
        exp = []
        for r in rows:
            t, tr = oracle.sample_token(r[0], r[1], to_oracle_cfg(r[2]), r[3])
            exp.append((t, tr.probability))
        assert_rows_match(out, exp, label="edge")
    finally:
        s.close()


def test_dead_end_and_termination_rules():
    """selectConstrainedToken (gemma-session.ts:1305-1329): termination ids only
    when accepting, extra ids legal unless also termination, empty -> dead end."""
    import torch

    gs = _gs()
    V = 4096
    s = gs.Sampler(vocab_size=V, max_rows=8)
    try:
        tokens = [None] * V
        tokens[10], tokens[11], tokens[12] = b"a", b"b", b"ab"
        vocab = gs.VocabBytes.from_tokens(tokens)
        nxt = np.full((3, 256), -1, np.int32)
        nxt[0, ord("a")] = 1
        nxt[1, ord("b")] = 2
        finals = np.array([0, 0, 1], np.uint8)
        s.set_vocab(vocab.offsets, vocab.data)
        s.set_dfa(nxt, finals)
        table = s.build_masks([0, 1, 2])
        assert np.nonzero(np.unpackbits(table[0].cpu().numpy().view(np.uint8), bitorder="little"))[0].tolist() == [10, 12]
        x = np.linspace(0, 1, V).astype(np.float32)
        base = gs.DecodingConfig(temperature=0, topK=0, topP=1, repetitionWindow=0)
        term = [1, 50, 106]
        forced = gs.constraint.forced_ids_csr(3, term, [100])
        conf = np.stack([
            gs.runtime.row_config(base, uniform=0.0, mask_slot=0),                   # legal {10,12,100}
            gs.runtime.row_config(base, uniform=0.0, mask_slot=2, accepting=True),   # only termination + extra
            gs.runtime.row_config(base, uniform=0.0, mask_slot=2, accepting=False),  # only the extra id
        ])
        out = s.sample(torch.from_numpy(np.stack([x, x, x])).cuda(), conf, forced=forced, mask_table=table)
        assert out.tokens.tolist() == [100, 106, 100]
        forced2 = gs.constraint.forced_ids_csr(1, term, [])
        conf2 = gs.runtime.row_config(base, uniform=0.0, mask_slot=2, accepting=False).reshape(1)
        with pytest.raises(gs.GSampleError, match="tokenization dead end"):
            s.sample(torch.from_numpy(x[None]).cuda(), conf2, forced=forced2, mask_table=table)
    finally:
        s.close()


def test_token_log_probability_rows(sampler):
    import torch

    x = np.random.default_rng(9).normal(0, 3, (4, 262144)).astype(np.float32)
    toks = [0, 5, 262143, 1234]
    got = sampler.token_log_probability(torch.from_numpy(x).cuda(), toks)
    for r in range(4):
        v = x[r].astype(np.float64)
        ref = v[toks[r]] - v.max() - np.log(np.exp(v - v.max()).sum())
        assert got[r] == pytest.approx(ref, abs=1e-12)
