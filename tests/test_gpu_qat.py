"""The int2 QAT LM head (gs_qat_lmhead) on the GPU against the oracle's
cpuQatLinear restatement (oracle/qat_ref.c, src/reference/qat-linear.ts:
78-148): the reference's own known answer (tests/qat-linear-gpu.spec.ts:
1307-1397), then the full Gemma shape (V 262144, width 1536) with random
codes, input and output SRQ, one and several rows of activations, both weight
layouts -- logits equal bit for bit, on the exact integer path and on the
binary64 kernel it leaves rows to -- and the fused head + sampler against the
oracle sampler on the oracle's logits."""
import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu


def _gs():
    import gsample

    return gsample


def test_reference_known_answer():
    import torch

    gs = _gs()
    words = np.full(8 * 96, 0xAAAAAAAA, np.uint32)
    words[96:192] = 0xFFFFFFFF
    words[192:288] = 0x55555555
    scales = np.array([1, 0.5, 0.25, 1, 1, 1, 1, 1], np.float32)
    s = gs.Sampler(vocab_size=8, max_rows=1)
    try:
        x = torch.ones((1, 1536), dtype=torch.float32, device="cuda")
        sc = torch.from_numpy(scales).cuda()
        for layout, w in ((gs.runtime.GS_QAT_ROW_MAJOR, words),
                          (gs.runtime.GS_QAT_BLOCK_MAJOR, oracle.repack_block_major(words, 8, 1536))):
            codes = torch.from_numpy(w.view(np.int32)).cuda()
            out = s.qat_lmhead(x, codes, sc, layout=layout).cpu().numpy()
            assert out[0].tolist() == [0, 768, -384, 0, 0, 0, 0, 0], (layout, out)
    finally:
        s.close()


@pytest.fixture(scope="module")
def gemma_head():
    rng = np.random.default_rng(17)
    V, D = 262144, 1536
    codes = rng.integers(0, 4, V * D, dtype=np.uint8)
    words = oracle.pack_int2_rows(codes, V, D)
    scales = (0.0008 + (np.arange(V) % 29) * 0.000025).astype(np.float32)
    x = rng.normal(0, 1.5, (3, D)).astype(np.float32)
    return V, D, words, scales, x


@pytest.mark.parametrize("in_scale,out_scale", [(0.0, 0.0), (0.03, 0.02)])
def test_gemma_shape_bit_exact(gemma_head, in_scale, out_scale):
    import torch

    gs = _gs()
    V, D, words, scales, x = gemma_head
    # the scales are float tensors in the checkpoint, and float in the C ABI
    in_scale, out_scale = float(np.float32(in_scale)), float(np.float32(out_scale))
    want = np.stack([oracle.qat_linear_int2(x[m], words, scales, D, V, in_scale, out_scale) for m in range(3)])
    s = gs.Sampler(vocab_size=V, max_rows=4)
    try:
        sc = torch.from_numpy(scales).cuda()
        xs = torch.from_numpy(x).cuda()
        row = torch.from_numpy(words.view(np.int32)).cuda()
        block = torch.from_numpy(oracle.repack_block_major(words, V, D).view(np.int32)).cuda()
        for layout, codes in ((gs.runtime.GS_QAT_ROW_MAJOR, row), (gs.runtime.GS_QAT_BLOCK_MAJOR, block)):
            for m in (1, 3):
                got = s.qat_lmhead(xs[:m].contiguous(), codes, sc, layout=layout, input_scale=in_scale,
                                   output_scale=out_scale).cpu().numpy()
                bad = np.nonzero(got.view(np.uint32) != want[:m].view(np.uint32))
                assert bad[0].size == 0, (layout, m, bad[0][:5], bad[1][:5], got[bad][:5], want[:m][bad][:5])
        if out_scale:
            assert len(np.unique(want[0])) <= 256  # the SRQ grid
    finally:
        s.close()


@pytest.mark.parametrize("in_scale", [0.0, 0.03])
def test_integer_path_and_fallback_rows(gemma_head, in_scale):
    """The exact integer path (int8 MFMA on limbs of the activations) takes
    the rows whose products and partial sums are all exact in binary64; a row
    with an activation 2^-100 beside values near 1 (an exponent range past 53
    bits) and a row holding an f32 subnormal are left to the binary64 kernel.
    Five rows (the last operand tile half empty), both layouts: every logit
    equals cpuQatLinear's bit for bit."""
    import torch

    gs = _gs()
    V, D, words, scales, x = gemma_head
    xs = np.concatenate([x, x[:2] * 0.5]).astype(np.float32)
    xs[1, 10] = np.float32(2.0 ** -100)
    xs[3, 5] = np.float32(1e-40)
    assert xs[3, 5] != 0 and xs[3, 5] < np.finfo(np.float32).tiny
    in_scale = float(np.float32(in_scale))
    want = np.stack([oracle.qat_linear_int2(xs[m], words, scales, D, V, in_scale, 0.0) for m in range(5)])
    s = gs.Sampler(vocab_size=V, max_rows=8)
    try:
        sc = torch.from_numpy(scales).cuda()
        xt = torch.from_numpy(xs).cuda()
        row = torch.from_numpy(words.view(np.int32)).cuda()
        block = torch.from_numpy(oracle.repack_block_major(words, V, D).view(np.int32)).cuda()
        for layout, codes in ((gs.runtime.GS_QAT_ROW_MAJOR, row), (gs.runtime.GS_QAT_BLOCK_MAJOR, block)):
            got = s.qat_lmhead(xt, codes, sc, layout=layout, input_scale=in_scale).cpu().numpy()
            bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
            assert bad[0].size == 0, (layout, bad[0][:5], bad[1][:5], got[bad][:5], want[bad][:5])
    finally:
        s.close()


def test_fused_head_and_sampler(gemma_head):
    import torch

    gs = _gs()
    V, D, words, scales, x = gemma_head
    logits = np.stack([oracle.qat_linear_int2(x[m], words, scales, D, V, 0.0, 0.0) for m in range(3)])
    cfg = gs.DecodingConfig(temperature=0.8, topK=40, topP=0.9, repetitionPenalty=1.2, repetitionWindow=32)
    us = [0.1, 0.5, 0.93]
    hists = [list(range(100 * m, 100 * m + 20)) for m in range(3)]
    s = gs.Sampler(vocab_size=V, max_rows=4)
    try:
        conf = np.stack([gs.runtime.row_config(cfg, uniform=u) for u in us])
        scratch = torch.empty((3, V), dtype=torch.float32, device="cuda")
        out = s.qat_lmhead_sample(torch.from_numpy(x).cuda(), torch.from_numpy(words.view(np.int32)).cuda(),
                                  torch.from_numpy(scales).cuda(), scratch, conf, histories=hists)
        assert np.array_equal(scratch.cpu().numpy().view(np.uint32), logits.view(np.uint32))
        ocfg = oracle.Decoding(temperature=0.8, topK=40, topP=0.9, minP=0.0, typicalP=1.0, repetitionPenalty=1.2,
                               repetitionWindow=32, frequencyPenalty=0.0, presencePenalty=0.0)
        for m in range(3):
            t, _ = oracle.sample_token(logits[m], hists[m], ocfg, us[m])
            assert int(out.tokens[m]) == t
    finally:
        s.close()


def test_signed_zero_logits():
    """Rows whose scale is 0 turn a negative dot into -0, and the output SRQ
    keeps a -0 ratio as -0 while ratios in [-1/2, 0) round to +0
    (qat-linear.ts:120-148); activations of -0 beside +0: every logit's bits,
    sign of zero included, equal cpuQatLinear's, on both layouts."""
    import torch

    gs = _gs()
    rng = np.random.default_rng(23)
    V, D = 100, 1536
    codes = rng.integers(0, 4, V * D, dtype=np.uint8)
    words = oracle.pack_int2_rows(codes, V, D)
    scales = rng.uniform(0.0005, 0.005, V).astype(np.float32)
    scales[::7] = 0.0
    x = rng.normal(0, 1.0, (4, D)).astype(np.float32)
    x[1, ::3] = np.float32(-0.0)
    x[2] = np.float32(-0.0)
    s = gs.Sampler(vocab_size=V, max_rows=4)
    try:
        sc = torch.from_numpy(scales).cuda()
        xs = torch.from_numpy(x).cuda()
        row = torch.from_numpy(words.view(np.int32)).cuda()
        block = torch.from_numpy(oracle.repack_block_major(words, V, D).view(np.int32)).cuda()
        for in_s, out_s in ((0.0, 0.02), (0.03, 0.125), (0.0, 0.0)):
            in_s, out_s = float(np.float32(in_s)), float(np.float32(out_s))
            want = np.stack([oracle.qat_linear_int2(x[m], words, scales, D, V, in_s, out_s) for m in range(4)])
            if out_s:
                assert np.any(np.signbit(want) & (want == 0)) and np.any(~np.signbit(want) & (want == 0))
            for layout, cw in ((gs.runtime.GS_QAT_ROW_MAJOR, row), (gs.runtime.GS_QAT_BLOCK_MAJOR, block)):
                got = s.qat_lmhead(xs, cw, sc, layout=layout, input_scale=in_s, output_scale=out_s).cpu().numpy()
                bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
                assert bad[0].size == 0, (in_s, out_s, layout, bad[0][:5], bad[1][:5], got[bad][:5], want[bad][:5])
    finally:
        s.close()
