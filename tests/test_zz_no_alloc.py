"""gs_sample_noalloc, the entry point that allocates nothing, against gs_sample
through the C ABI: two calls in a row (the second with fewer rows and
shorter histories, so the fixed device array still holds the first call's
contents), rows on the one-pass path, greedy rows, constrained rows and
forced-exact rows past the entry point's two exact slots (replayed by the
exact kernel in the same array). Same kernels, so results are bit-identical;
and sizes beyond the array's limits are refused before anything launches."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V = 262144
GS_ERR_UNSUPPORTED = 9


def _inputs(rng, rows, hist_len):
    import gsample as gs

    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    hists = [rng.integers(0, V, hist_len).tolist() for _ in range(rows)]
    base = gs.DecodingConfig(temperature=0.8, topK=40, topP=0.95, repetitionPenalty=1.1, repetitionWindow=hist_len,
                             frequencyPenalty=0.2, presencePenalty=0.3)
    conf = []
    for r in range(rows):
        kind = r % 5
        cfg = base.merged(temperature=0.0) if kind == 1 else base.merged(topK=0, topP=0.9) if kind == 2 else base
        conf.append(gs.runtime.row_config(cfg, seed=1000 + r, mask_slot=0 if kind == 3 else -1,
                                          force_exact=kind == 4))
    return x, hists, np.stack(conf)


def test_noalloc_matches_gs_sample():
    import torch

    import gsample as gs

    lib = gs.runtime.library()
    rng = np.random.default_rng(77)
    legal = np.union1d(rng.choice(V, V // 16, replace=False), [0, V - 1])
    words = np.zeros(V // 32, np.uint32)
    np.bitwise_or.at(words, legal >> 5, np.left_shift(np.uint32(1), (legal & 31).astype(np.uint32)))
    table = torch.from_numpy(words.view(np.int32)[None].copy()).cuda()
    s = gs.Sampler(vocab_size=V, max_rows=64)
    stream = torch.cuda.Stream()
    try:
        for rows, hist_len in ((48, 300), (20, 64)):
            x, hists, conf = _inputs(rng, rows, hist_len)
            dev = torch.from_numpy(x).cuda()
            ref = s.sample(dev, conf, histories=hists, mask_table=table)
            b, keep = s.prepare(dev, conf, histories=hists, mask_table=table)
            res = torch.full((rows, 2), -7.0, dtype=torch.float64, device="cuda")
            b.results = res.data_ptr()
            torch.cuda.synchronize()
            st = lib.gs_sample_noalloc(C.byref(b), V, C.c_void_p(stream.cuda_stream))
            assert st == 0, lib.gs_last_error(None).decode()
            stream.synchronize()
            got = res.cpu().numpy().view(np.uint8).reshape(-1).view(gs.runtime.RESULT_DTYPE)
            assert np.array_equal(got["token"], ref.tokens), rows
            assert np.array_equal(got["flags"], ref.flags), rows
            assert np.array_equal(got["probability"].view(np.uint64), ref.probabilities.view(np.uint64)), rows
            # the forced-exact rows (every fifth) really took the exact path
            assert np.all(got["flags"][4::5] & gs.GS_FLAG_EXACT_PATH)
            del keep
        # beyond the fixed array's limits: refused, nothing launched
        b.rows = 65
        assert lib.gs_sample_noalloc(C.byref(b), V, None) == GS_ERR_UNSUPPORTED
        assert "rows must be 0..64" in lib.gs_last_error(None).decode()
        b.rows = 4
        assert lib.gs_sample_noalloc(C.byref(b), V + 1, None) == GS_ERR_UNSUPPORTED
        assert "vocab_size must be 1..262144" in lib.gs_last_error(None).decode()
    finally:
        s.close()
