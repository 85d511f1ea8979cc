"""The checked build (libgsample_checked.so, compiled with -DGS_CHECKED):
every index the finish and the deep draw read back from LDS or from their
records is range-checked, and a failed check replays the row exactly with
GS_FLAG_INDEX_CHECK instead of writing a result.

A child process loads the checked build (GSAMPLE_CHECKED=1; this process
already holds the normal one) and samples the batches that exercise the
finish's routes: the penalties batch (top-k / top-p, greedy, forced exact
rows), full-vocabulary draws taken by the deep kernels, top-k past 64,
typical-p (also on a logit grid, where surprises tie), the constrained batch,
heavy-tailed bf16 rows and full-vocabulary draws past small regions. No row may carry the flag, and every token,
probability and flag must equal the normal build's on the same inputs.

The checked build also delays wave 0 after every barrier of the finish and
deep kernels and clears their LDS at each workgroup's start, so a read that
races a write by wave 0 sees the cleared word on every run: such a race
changes results here deterministically, where the normal build shows it
once in many runs."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = r"""
import json, os, sys
sys.path[:0] = [sys.argv[1], os.path.join(sys.argv[1], "gemma-webgpu-engine_amd")]
import numpy as np, torch
import gsample as gs
W = gs.workloads
assert gs.runtime.LIB_PATH.endswith(sys.argv[2]), gs.runtime.LIB_PATH
s = gs.Sampler(vocab_size=262144, max_rows=512)
out = {}
def run(name, x, conf, **kw):
    o = s.sample(x, conf, **kw)
    out[name] = [o.tokens.tolist(), o.probabilities.tolist(), o.flags.tolist()]
w = W.penalties()
cfgs = list(w.configs)
for r in range(3, 256, 8):
    cfgs[r] = cfgs[r].merged(temperature=0.0)
conf = np.stack([gs.runtime.row_config(c, seed=sd, force_exact=(r % 64 == 5)) for r, (c, sd) in enumerate(zip(cfgs, w.seeds))])
run("penalties", torch.from_numpy(w.logits).cuda(), conf, histories=w.histories)
for name in ("multinomial", "topk_deep", "typical"):
    w = getattr(W, name)()
    conf = np.stack([gs.runtime.row_config(c, seed=sd) for c, sd in zip(w.configs, w.seeds)])
    run(name, torch.from_numpy(w.logits).cuda(), conf)
offsets, data = W.synthetic_vocab()
nxt, finals = W.synthetic_dfa()
s.set_vocab(offsets, data)
s.set_dfa(nxt, finals)
table = s.build_masks(list(range(64)))
w = W.constrained()
conf = np.stack([gs.runtime.row_config(c, seed=sd, mask_slot=int(st)) for c, sd, st in zip(w.configs, w.seeds, w.states)])
run("constrained", torch.from_numpy(w.logits).cuda(), conf, mask_table=table)
w = W.heavy_tail(n_rows=512)
conf = np.stack([gs.runtime.row_config(c, seed=sd) for c, sd in zip(w.configs, w.seeds)])
run("heavy_tail", torch.from_numpy(w.logits.view(np.int16)).cuda().view(torch.bfloat16), conf)
s.close()
# full-vocabulary draws past regions of at most 128 entries (two chunks)
rng = np.random.default_rng(5)
Vs, n = 8269, 48
s = gs.Sampler(vocab_size=Vs, max_rows=n)
x = torch.from_numpy(rng.normal(0, 1.0, (n, Vs)).astype(np.float32)).cuda()
cfg = gs.DecodingConfig(temperature=1.0, topK=0, topP=1.0, minP=0.0, typicalP=1.0, repetitionPenalty=2.0,
                        repetitionWindow=8)
hist = [rng.integers(0, Vs, 8).tolist() for _ in range(n)]
conf = np.stack([gs.runtime.row_config(cfg, uniform=float(u)) for u in rng.uniform(0.3, 0.99, n)])
run("small_region_multi", x, conf, histories=hist)
run("small_region_single", x, conf, histories=hist, hints=0)
s.close()
# typical-p on every row, logits on a 1/4 grid: exact and mirrored surprise ties
rng = np.random.default_rng(11)
Vt, n = 40000, 64
s = gs.Sampler(vocab_size=Vt, max_rows=n)
xt = torch.from_numpy((np.round(rng.normal(0, 2.0, (n, Vt)) * 4) / 4).astype(np.float32)).cuda()
conf = np.stack([gs.runtime.row_config(gs.DecodingConfig(
    temperature=float(rng.choice([0.7, 1.0, 1.5])), topK=int(rng.choice([0, 10, 64, 128, 300])), topP=1.0,
    minP=0.0, typicalP=float(rng.choice([0.2, 0.5, 0.9, 0.999])), repetitionPenalty=1.0),
    uniform=float(rng.random())) for _ in range(n)])
run("typical_grid", xt, conf)
s.close()
with open(sys.argv[3], "w") as f:
    json.dump(out, f)
"""


def _run(tmp_path, checked):
    name = "libgsample_checked.so" if checked else "libgsample.so"
    path = str(tmp_path / ("checked.json" if checked else "normal.json"))
    env = dict(os.environ, GSAMPLE_CHECKED="1" if checked else "0")
    print(f"child process: {name}", flush=True)
    subprocess.run([sys.executable, "-c", _CHILD, ROOT, name, path], check=True, timeout=600, env=env)
    with open(path) as f:
        return json.load(f)


def test_checked_build_flags_nothing_and_matches(tmp_path):
    import gsample

    checked = _run(tmp_path, True)
    normal = _run(tmp_path, False)
    assert checked.keys() == normal.keys()
    for name in checked:
        tok_c, prob_c, flag_c = (np.asarray(v) for v in checked[name])
        tok_n, prob_n, flag_n = (np.asarray(v) for v in normal[name])
        assert not np.any(flag_c & gsample.GS_FLAG_INDEX_CHECK), (name, np.nonzero(flag_c & gsample.GS_FLAG_INDEX_CHECK))
        assert np.array_equal(tok_c, tok_n), name
        assert np.array_equal(prob_c, prob_n), name
        assert np.array_equal(flag_c, flag_n), name
        assert not np.any(tok_c < 0), name
