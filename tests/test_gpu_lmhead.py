"""GPU parity of the bf16 MFMA lm_head (gs_lmhead) and of the fused
lm_head + sampler call (gs_lmhead_sample) at the 64 x 2048 x 262144 shape.

The reference's producer is an int2 QAT GEMV (src/webgpu/decode-lm-head.ts:
187-340) with no softcap, so the bf16 GEMM and the 30 tanh(x/30) cap have no
reference vectors: they are checked against a float64 CPU GEMM of the same
bf16 inputs, with the fp32-accumulation bound written below. The sampler
half is bit-exact against the oracle on the logits the GPU produced."""
import numpy as np
import pytest

from oracle.oracle import Decoding

pytestmark = pytest.mark.gpu

V, M, D = 262144, 64, 2048
# fp32 accumulation of D products: |err| <= c * sqrt(D) * 2^-24 * sum|h w|;
# 2e-5 * sum|h w| leaves a factor ~7 over sqrt(2048) * 6e-8
GEMM_RTOL_OF_ABS_SUM = 2e-5


def _gs():
    import gsample

    return gsample


def _f64(t):
    import torch

    return t.to(torch.float32).cpu().numpy().astype(np.float64)


@pytest.fixture(scope="module")
def lm_inputs():
    import torch

    gs = _gs()
    hidden, weight = gs.workloads.lmhead_inputs(M, D, V, device=torch.device("cuda", 0))
    return hidden, weight


def test_lmhead_gemm_matches_f64(sampler, lm_inputs):
    hidden, weight = lm_inputs
    cols = np.random.default_rng(5).choice(V, 3000, replace=False)
    cols = np.concatenate([cols, [0, 1, 127, 128, V - 129, V - 1]])
    h = _f64(hidden)
    w = _f64(weight[cols])
    ref = h @ w.T
    bound = GEMM_RTOL_OF_ABS_SUM * (np.abs(h) @ np.abs(w).T) + 1e-30
    for cap in (0.0, 30.0):
        out = sampler.lmhead(hidden, weight, softcap_value=cap)
        got = out[:, cols].cpu().numpy().astype(np.float64)
        if cap > 0:
            exp = cap * np.tanh(ref / cap)
            # tanh is 1-Lipschitz: the GEMM bound carries over, plus a few f32 ulps of the cap's output
            err_bound = bound + 4 * np.spacing(np.abs(exp).astype(np.float32)).astype(np.float64)
        else:
            exp = ref
            err_bound = bound
        err = np.abs(got - exp)
        assert np.all(err <= err_bound), (cap, float((err / err_bound).max()))


def test_lmhead_partial_row_block(sampler, lm_inputs):
    """m_rows below the 64-row MFMA block: rows beyond m are neither read nor written."""
    import torch

    hidden, weight = lm_inputs
    m = 5
    out = torch.full((M, V), 7.0, dtype=torch.float32, device=hidden.device)
    sampler.lmhead(hidden[:m].contiguous(), weight, softcap_value=0.0, out=out)
    full = sampler.lmhead(hidden, weight, softcap_value=0.0)
    assert torch.equal(out[:m], full[:m])
    assert bool((out[m:] == 7.0).all())


def test_lmhead_sample_bit_exact_on_gpu_logits(sampler, lm_inputs, oracle, synthetic_constraint):
    """gs_lmhead_sample over the config-5 pipeline: penalties from 256-id
    histories, the synthetic DFA's masks, topK 64 / topP 0.95, T 1, seed = row.
    Token ids must equal the oracle's on the GPU-produced logits."""
    import torch

    gs = _gs()
    W = gs.workloads
    hidden, weight = lm_inputs
    offsets, data, nxt, finals, ref_masks = synthetic_constraint
    sampler.set_vocab(offsets, data)
    sampler.set_dfa(nxt, finals)
    table = sampler.build_masks(list(range(64)))
    hist = W.lmhead_histories(M)
    states = [int(W.rng(7, r).integers(0, 64)) for r in range(M)]
    cfg = W.LMHEAD_CONFIG
    conf = np.stack([gs.runtime.row_config(cfg, seed=r, mask_slot=states[r]) for r in range(M)])
    scratch = torch.empty((M, V), dtype=torch.float32, device=hidden.device)
    batch, keep = sampler.prepare(scratch, conf, histories=hist, mask_table=table)
    sampler.lmhead_sample_launch(hidden, weight, 30.0, scratch, batch)
    sampler.synchronize()
    res = keep[-1].cpu().numpy().view(np.uint8).reshape(-1)[: M * 16].view(gs.runtime.RESULT_DTYPE)
    logits = scratch.cpu().numpy()
    assert np.all(np.abs(logits) <= 30.0)
    masks = table.cpu().numpy().view(np.uint32)
    for s in sorted(set(states)):
        assert np.array_equal(masks[s], ref_masks[s]), s
    ocfg = Decoding(temperature=cfg.temperature, topK=cfg.topK, topP=cfg.topP, minP=cfg.minP, typicalP=cfg.typicalP,
                    repetitionPenalty=cfg.repetitionPenalty, repetitionWindow=cfg.repetitionWindow,
                    frequencyPenalty=cfg.frequencyPenalty, presencePenalty=cfg.presencePenalty)
    for r in range(0, M, 4):
        legal = oracle.mask_bits_to_ids(ref_masks[states[r]], V)
        masked = oracle.mask_logits(logits[r], legal, [])
        t, tr = oracle.sample_token(masked, hist[r], ocfg, oracle.draw(r, 0))
        assert int(res["token"][r]) == t, (r, int(res["token"][r]), t, int(res["flags"][r]))
        # the scan's normaliser bound (3.9e-7 relative) plus binary64 roundings
        assert abs(res["probability"][r] - tr.probability) <= 4e-7 * tr.probability


@pytest.mark.parametrize("vocab,width,m", [
    (40004, 640, 96),    # K steps split unevenly over the waves; two 64-row blocks
    (40004, 1152, 5),    # a partial row block; V ends inside a 16-row tile
    (40004, 2048, 1),
    (40004, 2112, 70),   # wider than 2048: the staged-H kernel
    (40002, 1152, 64),   # V not a multiple of 4: the staged-H kernel
])
def test_lmhead_shapes_match_f64(vocab, width, m):
    """Widths, row counts and vocabulary sizes off the 64 x 2048 x 262144 shape,
    on both lm_head kernels: every column near V's end and 3000 others against
    a float64 GEMM; rows past m stay untouched."""
    import torch

    gs = _gs()
    s = gs.Sampler(vocab_size=vocab, max_rows=128)
    try:
        dev = torch.device("cuda", 0)
        hidden, weight = gs.workloads.lmhead_inputs(m, width, vocab, device=dev)
        cols = np.random.default_rng(width + m).choice(vocab, 3000, replace=False)
        cols = np.unique(np.concatenate([cols, np.arange(vocab - 40, vocab), np.arange(0, 40)]))
        h = _f64(hidden)
        w = _f64(weight[torch.from_numpy(cols).to(dev)])
        ref = h @ w.T
        bound = GEMM_RTOL_OF_ABS_SUM * (np.abs(h) @ np.abs(w).T) + 1e-30
        for cap in (0.0, 30.0):
            out = torch.full((m + 3, vocab), 7.0, dtype=torch.float32, device=dev)
            s.lmhead(hidden, weight, softcap_value=cap, out=out)
            got = out[:m].cpu().numpy()[:, cols].astype(np.float64)
            exp = cap * np.tanh(ref / cap) if cap > 0 else ref
            err_bound = bound + (4 * np.spacing(np.abs(exp).astype(np.float32)).astype(np.float64) if cap > 0 else 0)
            err = np.abs(got - exp)
            assert np.all(err <= err_bound), (cap, float((err / err_bound).max()))
            assert bool((out[m:] == 7.0).all())
    finally:
        s.close()
