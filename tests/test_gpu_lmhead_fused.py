"""The fused lm_head + sampler (gs_lmhead_sample with GS_BATCH_FUSED_HEAD): the GEMM's epilogue writes
the chunk statistics that the scan would compute from the logits
(src/webgpu/decode-model.ts:127-150 is the handoff it removes,
src/webgpu/decode-lm-head.ts:262-340 the producer).

* the logits it writes equal gs_lmhead's bit for bit (same tiles, same K
  order, same softcap);
* every row's token equals the unfused pipeline's (gs_lmhead, then gs_sample
  over the same logits) over a batch mixing every route: greedy, top-k,
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


def test_fused_logits_equal_lmhead(sampler, weight_and_hidden):
    import torch

    import gsample as gs
    hidden, weight = weight_and_hidden
    m = 70
    h = hidden[:m].contiguous()
    cfg = gs.DecodingConfig(temperature=1.0, topK=40, topP=0.95, repetitionWindow=0)
    conf = np.stack([gs.runtime.row_config(cfg, seed=r) for r in range(m)])
    for cap in (30.0, 0.0):
        ref = sampler.lmhead(h, weight, softcap_value=cap)
        scratch = torch.full((m, V), 5.0, dtype=torch.float32, device=hidden.device)
        sampler.lmhead_sample(h, weight, cap, scratch, conf, fused=True)
        assert torch.equal(scratch, ref), cap


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

    ref_logits = sampler.lmhead(h, weight, softcap_value=30.0)
    unfused = sampler.sample(ref_logits, conf, histories=hist, forced=forced, mask_table=table,
                             raise_on_failure=False)
    scratch = torch.empty((rows, V), dtype=torch.float32, device=hidden.device)
    fused = sampler.lmhead_sample(h, weight, 30.0, scratch, conf, histories=hist, forced=forced, mask_table=table,
                                  fused=True)
    # bit patterns: row 50's NaNs compare unequal as values
    assert torch.equal(scratch.view(torch.int32), ref_logits.view(torch.int32))
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
