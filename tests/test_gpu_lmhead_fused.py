"""The fused lm_head + sampler (gs_lmhead_sample with GS_BATCH_FUSED_HEAD): the GEMM's epilogue writes
the chunk statistics that the scan would compute from the logits
(src/webgpu/decode-model.ts:127-150 is the handoff it removes,
src/webgpu/decode-lm-head.ts:262-340 the producer).

* the logits it writes agree with a float64 GEMM of the same bf16 inputs
  within the fp32-accumulation bound (its K order differs from gs_lmhead's
  resident kernel, so the two are not bit-identical);
* every row's token equals the unfused pipeline's (gs_sample over the logits
  the fused call wrote) over a batch mixing every route: greedy, top-k,
  top-p, min-p, typical-p, constrained rows with and without an accepting
  state (forced termination ids), penalties, a forced exact replay, a
  full-vocabulary draw and a row of NaN logits, at 96 rows (a partial second
  64-row block of the GEMM);
* the tokens of the sampled rows equal the oracle's on the same logits."""
import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

V, D = 262144, 2048
EOS = (1, 50, 106)


def _decoding(c):
    return Decoding(temperature=c.temperature, topK=c.topK, topP=c.topP, minP=c.minP, typicalP=c.typicalP,
                    repetitionPenalty=c.repetitionPenalty, repetitionWindow=c.repetitionWindow,
                    frequencyPenalty=c.frequencyPenalty, presencePenalty=c.presencePenalty)


@pytest.fixture(scope="module")
def weight_and_hidden():
    import torch

    import gsample as gs
    hidden, weight = gs.workloads.lmhead_inputs(96, D, V, device=torch.device("cuda", 0))
    return hidden.to("cuda"), weight


def test_fused_logits_match_f64(sampler, weight_and_hidden):
    import torch

    import gsample as gs
    hidden, weight = weight_and_hidden
    m = 70
    h = hidden[:m].contiguous()
    cfg = gs.DecodingConfig(temperature=1.0, topK=40, topP=0.95, repetitionWindow=0)
    conf = np.stack([gs.runtime.row_config(cfg, seed=r) for r in range(m)])
    cols = np.random.default_rng(9).choice(V, 2000, replace=False)
    cols = np.concatenate([cols, [0, 1, 255, 256, 8191, 8192, V - 1]])
    hf = h.to(torch.float32).cpu().numpy().astype(np.float64)
    wf = weight[cols].to(torch.float32).cpu().numpy().astype(np.float64)
    ref = hf @ wf.T
    # fp32 accumulation of D products: |err| <= c sqrt(D) 2^-24 sum|h w|
    bound = 2e-5 * (np.abs(hf) @ np.abs(wf).T) + 1e-30
    for cap in (30.0, 0.0):
        scratch = torch.full((m, V), 5.0, dtype=torch.float32, device=hidden.device)
        sampler.lmhead_sample(h, weight, cap, scratch, conf, fused=True)
        got = scratch[:, cols].cpu().numpy().astype(np.float64)
        if cap > 0:
            exp = cap * np.tanh(ref / cap)
            err_bound = bound + 4 * np.spacing(np.abs(exp).astype(np.float32)).astype(np.float64)
        else:
            exp, err_bound = ref, bound
        err = np.abs(got - exp)
        assert np.all(err <= err_bound), (cap, float((err / err_bound).max()))


def _mixed_batch(gs, rows, states, finals):
    base = gs.DecodingConfig(temperature=1.0, topK=64, topP=0.95, repetitionPenalty=1.1, repetitionWindow=256,
                             frequencyPenalty=0.3, presencePenalty=0.5)
    kinds = [
        ("greedy", base.merged(temperature=0.0), False, {}),
        ("topk5", base.merged(topK=5, temperature=0.8, repetitionWindow=0), False, {}),
        ("topk64_pen", base, False, {}),
        ("topp", base.merged(topK=0, topP=0.9, temperature=0.7), False, {}),
        ("minp", base.merged(topK=0, topP=1.0, minP=0.05, repetitionWindow=0), False, {}),
        ("typical", base.merged(topK=40, typicalP=0.9), False, {}),
        ("c_accepting", base, True, {"accepting": True}),
        ("c_greedy", base.merged(temperature=0.0), True, {"accepting": False}),
        ("exact", base.merged(topK=10), False, {"force_exact": True}),
        ("c_topp", base.merged(topK=0, topP=0.95, repetitionWindow=0), True, {"accepting": False}),
        ("full_draw", base.merged(topK=0, topP=1.0, temperature=0.8, repetitionWindow=0), False, {}),
        ("topk64_t07", base.merged(temperature=0.7), False, {}),
    ]
    conf, meta = [], []
    for r in range(rows):
        name, c, constrained, kw = kinds[r % len(kinds)]
        slot = states[r] if constrained else -1
        kw = dict(kw)
        if constrained and "accepting" in kw:
            kw["accepting"] = bool(finals[states[r]]) if kw["accepting"] else False
        conf.append(gs.runtime.row_config(c, seed=r, mask_slot=slot, **kw))
        meta.append((name, c, constrained, kw.get("accepting", False)))
    return np.stack(conf), meta


def test_fused_matches_unfused_and_oracle(sampler, weight_and_hidden, oracle, synthetic_constraint):
    import torch

    import gsample as gs
    W = gs.workloads
    hidden, weight = weight_and_hidden
    rows = 96
    h = hidden.clone()
    h[50, 7] = float("nan")  # row 50: every logit NaN
    offsets, data, nxt, finals, ref_masks = synthetic_constraint
    sampler.set_vocab(offsets, data)
    sampler.set_dfa(nxt, finals)
    table = sampler.build_masks(list(range(64)))
    states = [int(W.rng(21, r).integers(0, 64)) for r in range(rows)]
    hist = W.lmhead_histories(rows)
    conf, meta = _mixed_batch(gs, rows, states, finals)
    forced = gs.constraint.forced_ids_csr(rows, EOS)

    scratch = torch.empty((rows, V), dtype=torch.float32, device=hidden.device)
    fused = sampler.lmhead_sample(h, weight, 30.0, scratch, conf, histories=hist, forced=forced, mask_table=table,
                                  fused=True)
    assert bool(torch.isnan(scratch[50]).all())
    # the unfused sampler over the logits the fused call wrote
    unfused = sampler.sample(scratch.clone(), conf, histories=hist, forced=forced, mask_table=table,
                             raise_on_failure=False)
    for r in range(rows):
        name = meta[r][0]
        assert int(fused.tokens[r]) == int(unfused.tokens[r]), (r, name, int(fused.tokens[r]),
                                                                int(unfused.tokens[r]), int(fused.flags[r]),
                                                                int(unfused.flags[r]))
        assert not fused.flags[r] & gs.GS_FLAG_INDEX_CHECK
        fp, up = float(fused.probabilities[r]), float(unfused.probabilities[r])
        if np.isfinite(up) and up > 0:
            # two normaliser sums of the same terms grouped differently: each
            # within the scan's 3.9e-7 bound of the exact one
            assert abs(fp - up) <= 8e-7 * up, (r, name, fp, up)
        else:
            assert fp == up or (np.isnan(fp) and np.isnan(up)), (r, name, fp, up)

    logits = scratch.cpu().numpy()
    for r in range(0, rows, 5):
        if r == 50:
            continue
        name, c, constrained, accepting = meta[r]
        x = logits[r]
        if constrained:
            legal = oracle.mask_bits_to_ids(ref_masks[states[r]], V)
            x = oracle.mask_logits(x, legal, list(EOS) if accepting else [])
        t, tr = oracle.sample_token(x, hist[r], _decoding(c), oracle.draw(r, 0))
        assert int(fused.tokens[r]) == t, (r, name, int(fused.tokens[r]), t, int(fused.flags[r]))
