"""GPU parity at full batch shapes and for the per-row final-logit softcap.

* The per-row softcap (gs_row_config.softcap): the scan caps every logit,
  the finish caps the specials it gathers and the logits of its binary64
  normaliser recompute, and the exact replay caps every logit. The oracle
  samples the same capped binary32 values (oracle.softcap, itself pinned to
  the binary64 closed form in test_oracle_known_answers.py).
* The heavy-tailed bf16 batch at its full 1024 rows (two scan groups per
  row, rows past the context's exact slots) and the constrained batch at its
  full 128 rows (the constrained scan variant's own grid), compared with the
  oracle on rows spread over the whole batch.

Ids are bit-exact; probabilities are identical on exact-path rows and within
PROB_RTOL relative on one-pass rows (the scan normaliser's bound, 3.9e-7,
plus binary64 roundings)."""
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


def check_row(gs, label, r, token, prob, flags, t, p):
    assert int(token) == t, f"{label} row {r}: token {int(token)} != {t} (flags {int(flags)})"
    assert not flags & gs.GS_FLAG_INDEX_CHECK, (label, r, int(flags))
    if flags & gs.GS_FLAG_EXACT_PATH:
        assert prob == p, (label, r, prob, p)
    else:
        assert abs(prob - p) <= PROB_RTOL * abs(p), (label, r, prob, p)


def test_softcap_rows_f32_and_bf16(sampler, oracle):
    """softcap 30 on rows whose logits reach well into tanh's bend (N(0, 15^2)):
    top-k with penalties (window ids among the capped logits), top-p only,
    greedy, forced-exact rows, and a top-p cut placed inside the scan
    normaliser's bound (settled by the binary64 recompute, which caps again),
    in f32 and in bf16."""
    import torch

    gs = _gs()
    rng = np.random.default_rng(41)
    cap = 30.0
    n = 8
    x32 = rng.normal(0, 15, (n, V)).astype(np.float32)
    # window ids: the largest logits of the row and random ones
    hists = []
    for r in range(n):
        top = np.argsort(-x32[r])[:40]
        hists.append(np.concatenate([top, rng.integers(0, V, 200), top[:10]]).astype(np.int32).tolist())
    base = gs.DecodingConfig(temperature=0.9, topK=50, topP=0.9, minP=0.0, typicalP=1.0, repetitionPenalty=1.2,
                             repetitionWindow=256, frequencyPenalty=0.2, presencePenalty=0.4)
    cfgs = [base, base.merged(topK=0, topP=0.8), base.merged(temperature=0.0), base,
            base.merged(topK=64, minP=0.02), base.merged(topK=0, topP=0.95, repetitionWindow=0), base, base]
    force = [False, False, False, True, False, False, False, True]
    us = [0.05 + 0.11 * i for i in range(n)]
    outs = {}
    for dtype in ("f32", "bf16"):
        if dtype == "f32":
            xin = x32
            dev = torch.from_numpy(x32).cuda()
        else:
            bits = gs.workloads.to_bf16_bits(x32)
            xin = gs.workloads.bf16_bits_to_f32(bits).reshape(n, V)
            dev = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
        # rows 6 and 7: a top-p cut 1e-8 relative inside the scan normaliser's bound
        probe = base.merged(topK=0, topP=0.9)
        _, tr = oracle.sample_token(oracle.softcap(xin[6], cap), hists[6], to_oracle_cfg(probe), 0.5)
        cfgs[6] = cfgs[7] = probe.merged(topP=tr.cumulative_at_cut * (1 - 1e-8))
        conf = np.stack([gs.runtime.row_config(c, uniform=u, softcap_value=cap, force_exact=f)
                         for c, u, f in zip(cfgs, us, force)])
        out = outs[dtype] = sampler.sample(dev, conf, histories=hists)
        for r in range(n):
            capped = oracle.softcap(xin[r], cap)
            t, tr = oracle.sample_token(capped, hists[r], to_oracle_cfg(cfgs[r]), us[r])
            check_row(gs, f"softcap {dtype}", r, out.tokens[r], out.probabilities[r], out.flags[r], t,
                      1.0 if cfgs[r].temperature == 0 else tr.probability)
            if force[r] and cfgs[r].temperature > 0:
                assert out.flags[r] & gs.GS_FLAG_EXACT_PATH, r
        # the cut inside the bound stays on the one-pass path (recomputed normaliser)
        assert not out.flags[6] & gs.GS_FLAG_EXACT_PATH, int(out.flags[6])
        assert out.flags[6] & gs.GS_FLAG_TOPP_TIE, int(out.flags[6])
    # the cap changes the answers: without it the same rows sample differently
    plain = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
    out_plain = sampler.sample(torch.from_numpy(x32).cuda(), plain, histories=hists)
    assert np.any(out_plain.probabilities != outs["f32"].probabilities)


def test_heavy_tail_full_batch(sampler, oracle):
    """The full 1024-row heavy-tailed bf16 batch in one launch: 64 rows spread
    over it (every 16th, so rows on both sides of the exact-slot count and in
    both scan generations) against the oracle."""
    import torch

    gs = _gs()
    w = gs.workloads.heavy_tail()
    conf = np.stack([gs.runtime.row_config(c, seed=s) for c, s in zip(w.configs, w.seeds)])
    x = torch.from_numpy(w.logits.view(np.int16)).cuda().view(torch.bfloat16)
    out = sampler.sample(x, conf)
    assert not np.any(out.tokens < 0)
    for r in range(0, 1024, 16):
        f = gs.workloads.bf16_bits_to_f32(w.logits[r])
        t, tr = oracle.sample_token(f, [], to_oracle_cfg(w.configs[r]), oracle.draw(w.seeds[r], 0))
        check_row(gs, "heavy_tail full", r, out.tokens[r], out.probabilities[r], out.flags[r], t, tr.probability)


@pytest.mark.parametrize("greedy", [False, True])
def test_constrained_full_batch(sampler, oracle, synthetic_constraint, greedy):
    """The full 128-row constrained batch (64-state DFA masks, the constrained
    scan variant's grid). The GPU's mask table is compared with the oracle's
    masks for all 64 states first (constraints.ts:56-92,253-265,300-322);
    then every other row is sampled against the oracle on logits masked with
    the oracle's own masks."""
    import torch

    gs = _gs()
    offsets, data, nxt, finals, ref_masks = synthetic_constraint
    sampler.set_vocab(offsets, data)
    sampler.set_dfa(nxt, finals)
    table = sampler.build_masks(list(range(64)))
    words = table.cpu().numpy().view(np.uint32)
    for s in range(64):
        assert np.array_equal(words[s], ref_masks[s]), f"state {s}: GPU mask differs from the oracle's"
    w = gs.workloads.constrained(greedy=greedy)
    conf = np.stack([gs.runtime.row_config(c, seed=s, mask_slot=int(st))
                     for c, s, st in zip(w.configs, w.seeds, w.states)])
    out = sampler.sample(torch.from_numpy(w.logits).cuda(), conf, mask_table=table)
    for r in range(0, 128, 2):
        legal = oracle.mask_bits_to_ids(ref_masks[w.states[r]], V)
        masked = oracle.mask_logits(w.logits[r], legal, [])
        t, tr = oracle.sample_token(masked, [], to_oracle_cfg(w.configs[r]), oracle.draw(w.seeds[r], 0))
        check_row(gs, f"constrained full greedy={greedy}", r, out.tokens[r], out.probabilities[r], out.flags[r],
                  t, 1.0 if greedy else tr.probability)


def test_long_penalty_windows(oracle):
    """Windows with thousands of distinct ids (sampling.ts:21-30 counts any
    window): 8192 and 20000 distinct ids, repeated ids among them, on a
    top-k row, a top-p row, a typical-p row (the exact route) and a greedy
    row. Rows with more distinct ids than the one-pass finish evaluates are
    replayed exactly, which counts window ids per vocabulary id."""
    import torch

    gs = _gs()
    Vs = 65536
    rng = np.random.default_rng(57)
    x = rng.normal(0, 3, (5, Vs)).astype(np.float32)
    hists = []
    for n_distinct in (8192, 20000, 8192, 30000, 1500):
        ids = rng.choice(Vs, n_distinct, replace=False)
        rep = rng.choice(ids, n_distinct // 3)
        h = np.concatenate([ids, rep])
        rng.shuffle(h)
        hists.append(h.astype(np.int32).tolist())
    base = gs.DecodingConfig(temperature=0.8, topK=40, topP=0.95, repetitionPenalty=1.3, frequencyPenalty=0.2,
                             presencePenalty=0.3, repetitionWindow=40000)
    cfgs = [base, base.merged(topK=0, topP=0.9), base.merged(topK=0, topP=1.0, typicalP=0.9),
            base.merged(temperature=0.0), base.merged(repetitionWindow=1800)]
    us = [0.21, 0.43, 0.65, 0.0, 0.87]
    s = gs.Sampler(vocab_size=Vs, max_rows=8)
    try:
        conf = np.stack([gs.runtime.row_config(c, uniform=u) for c, u in zip(cfgs, us)])
        out = s.sample(torch.from_numpy(x).cuda(), conf, histories=hists)
    finally:
        s.close()
    for r in range(5):
        t, tr = oracle.sample_token(x[r], hists[r], to_oracle_cfg(cfgs[r]), us[r])
        check_row(gs, "long windows", r, out.tokens[r], out.probabilities[r], out.flags[r], t,
                  1.0 if cfgs[r].temperature == 0 else tr.probability)
    for r in (0, 1):
        assert out.flags[r] & gs.GS_FLAG_EXACT_PATH, (r, int(out.flags[r]))


def test_mask_slot_outside_the_table_is_an_error():
    """A constrained row whose mask_slot lies past the batch's mask table is
    never sampled unmasked: the device entry point flags the row and the
    synchronous call raises."""
    import torch

    gs = _gs()
    Vs = 4096
    s = gs.Sampler(vocab_size=Vs, max_rows=4)
    try:
        x = torch.zeros((2, Vs), dtype=torch.float32, device="cuda")
        table = torch.full((1, Vs // 32), -1, dtype=torch.int32, device="cuda")
        cfg = gs.DecodingConfig(temperature=1.0, topK=10, topP=0.9, repetitionWindow=0)
        conf = np.stack([gs.runtime.row_config(cfg, uniform=0.5, mask_slot=0),
                         gs.runtime.row_config(cfg, uniform=0.5, mask_slot=3)])
        out = s.sample(x, conf, mask_table=table, raise_on_failure=False)
        assert out.tokens[0] >= 0 and out.tokens[1] == -1
        assert out.flags[1] & gs.GS_FLAG_INVALID_SLOT
        with pytest.raises(gs.GSampleError, match="mask_slot outside the mask table"):
            s.sample(x, conf, mask_table=table)
    finally:
        s.close()


def test_full_penalty_batch_mixed_routes_repeated(sampler, oracle):
    """256 f32 rows at the full vocabulary (four scan groups per row, one
    generation of workgroups): penalised top-k/top-p rows, greedy rows and
    rows forced onto the exact path in one batch. It is launched three times
    with a two-row batch (another grid) in between: every launch gives
    identical results, and the rows checked (every 8th, the greedy ones
    among them and the forced ones) match the oracle."""
    import torch

    gs = _gs()
    w = gs.workloads.penalties()
    cfgs = list(w.configs)
    greedy = gs.DecodingConfig(temperature=0.0, repetitionPenalty=1.1, repetitionWindow=512,
                               frequencyPenalty=0.3, presencePenalty=0.5)
    for r in range(3, 256, 8):
        cfgs[r] = greedy
    force = {r for r in range(5, 256, 64)}
    conf = np.stack([gs.runtime.row_config(c, seed=s, force_exact=(r in force))
                     for r, (c, s) in enumerate(zip(cfgs, w.seeds))])
    x = torch.from_numpy(w.logits).cuda()
    outs = []
    for rep in range(3):
        outs.append(sampler.sample(x, conf, histories=w.histories))
        small = sampler.sample(x[:2], conf[:2], histories=w.histories[:2])
        assert np.array_equal(small.tokens, outs[0].tokens[:2])
    for o in outs[1:]:
        assert np.array_equal(o.tokens, outs[0].tokens)
        assert np.array_equal(o.probabilities, outs[0].probabilities)
        assert np.array_equal(o.flags, outs[0].flags)
    out = outs[0]
    for r in sorted(set(range(0, 256, 8)) | set(range(3, 256, 64)) | force):
        t, tr = oracle.sample_token(w.logits[r], list(w.histories[r]), to_oracle_cfg(cfgs[r]),
                                    oracle.draw(w.seeds[r], 0))
        check_row(gs, "mixed routes", r, out.tokens[r], out.probabilities[r], out.flags[r], t, tr.probability)
    for r in force:
        assert out.flags[r] & gs.GS_FLAG_EXACT_PATH


def test_results_identical_across_calls(sampler, synthetic_constraint):
    """Every result is the same bit for bit on every call of the same batch:
    the finish sums the specials (window and forced ids, which sit in LDS in
    an order that atomics chose) as integers, and every other sum runs in a
    fixed order. The full penalty batch (512-id windows on every row), a
    constrained batch with windows and forced termination ids, and the
    typical-p and full-draw workloads (the binary64 normaliser recompute and
    the deep draws), each sampled 8 times."""
    import torch

    gs = _gs()
    W = gs.workloads
    batches = []
    w = W.penalties()
    conf = np.stack([gs.runtime.row_config(c, seed=sd) for c, sd in zip(w.configs, w.seeds)])
    batches.append(("penalties", torch.from_numpy(w.logits).cuda(), conf, dict(histories=w.histories)))
    offsets, data, nxt, finals, _ = synthetic_constraint
    sampler.set_vocab(offsets, data)
    sampler.set_dfa(nxt, finals)
    table = sampler.build_masks(list(range(64)))
    w = W.constrained(rows=list(range(0, 128, 2)))
    cfgs = [c.merged(repetitionPenalty=1.3, repetitionWindow=256, presencePenalty=0.4) for c in w.configs]
    hists = W.lmhead_histories(len(cfgs))
    conf = np.stack([gs.runtime.row_config(c, seed=sd, mask_slot=int(st), accepting=bool(finals[st]))
                     for c, sd, st in zip(cfgs, w.seeds, w.states)])
    batches.append(("constrained", torch.from_numpy(w.logits).cuda(), conf,
                    dict(histories=hists, forced=gs.constraint.forced_ids_csr(len(cfgs), (1, 50, 106)),
                         mask_table=table)))
    for name in ("typical", "multinomial"):
        w = getattr(W, name)(rows=list(range(64)))
        cfgs = [c.merged(repetitionPenalty=1.2, repetitionWindow=128) for c in w.configs]
        hists = W.lmhead_histories(64)
        conf = np.stack([gs.runtime.row_config(c, seed=sd) for c, sd in zip(cfgs, w.seeds)])
        batches.append((name, torch.from_numpy(w.logits).cuda(), conf, dict(histories=hists)))
    for name, x, conf, kw in batches:
        first = sampler.sample(x, conf, raise_on_failure=False, **kw)
        for k in range(7):
            out = sampler.sample(x, conf, raise_on_failure=False, **kw)
            assert np.array_equal(out.tokens, first.tokens), (name, k)
            assert np.array_equal(out.flags, first.flags), (name, k)
            same = out.probabilities.view(np.uint64) == first.probabilities.view(np.uint64)
            assert same.all(), (name, k, np.nonzero(~same)[0][:8])
