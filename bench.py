#!/usr/bin/env python3
"""Throughput of the batched sampling stage on one MI355X.

A step is one gs_sample call (chunk scan -> row finish -> exact replay) over a
batch of synthetic logits already resident in HBM; `value` is sampled rows per
second over the timed steps. The steps rotate over copies of the logits whose
total size is three times the 256 MB Infinity Cache, so no step finds its
logits left in that cache by the step before. The default workload is the batched penalties +
top-k/top-p case: 256 rows x 262144 f32 logits ~ N(0, 3^2), 512-id Zipf(1.1)
histories, repetition 1.1 / presence 0.5 / frequency 0.3 over a 512-id window,
temperature 0.7, topK 50, topP 0.9, row r drawing SeededRandom(r).next().

The same run reports
  roofline      the dominant kernel's algorithmic bytes per launch over its
                mean duration over a second run of the same K steps, each
                kernel launched with start/stop HIP events that stamp its own
                dispatch (gs_timing_begin / gs_timing_end; the events slow a
                step down, so the step rate comes from the first run,
                bracketed by two events only);
  traffic       HBM bytes the dominant kernel moves per launch, taken from the
                PMC summary committed under profiles/ for this workload (a
                line "bench-traffic: workload=<w> kernel=<k> bytes=<B>" that
                scales rocprofv3's FETCH_SIZE + WRITE_SIZE per dispatch by
                what those counters read for a copy of known size); null when
                no such summary exists;
  cpu_baseline  the JavaScript restatement of the reference sampler (and of
                its constraint masking for constrained rows) run by Node over
                bounded samples of the same rows: (i) on one thread, as the
                reference runs; (ii) split over worker_threads, one per host
                core up to --cpu-threads; and a bit-exact comparison of those
                rows' token ids with the GPU's.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "gemma-webgpu-engine_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "sampled rows/sec at vocab 262144, batch 256; achieved HBM GB/s (% of peak)"
HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E, AMD public specification
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
F64_VECTOR_PEAK_TFLOPS = 78.6  # MI355X fp64 (vector and matrix)
V = 262144


def profiled_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload` from the committed PMC
    summaries (profiles/*.md, lines "bench-traffic: workload=.. kernel=.. bytes=..")."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None
    for name in sorted(os.listdir(pdir)):
        if not name.endswith(".md"):
            continue
        with open(os.path.join(pdir, name)) as f:
            for line in f:
                if not line.startswith("bench-traffic:"):
                    continue
                kv = dict(t.split("=", 1) for t in line.split()[1:] if "=" in t)
                if kv.get("workload") == workload and kv.get("kernel") == kernel:
                    return int(kv["bytes"])
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="penalties",
                    choices=["penalties", "single_row", "heavy_tail", "constrained", "lmhead", "lmhead_fused", "qat",
                             "multinomial", "topk_deep", "typical", "penalties_constrained"])
    ap.add_argument("--also", default="penalties_constrained",
                    help="comma-separated workloads measured after the main one and reported beside it under "
                         "'also' (default: penalties_constrained; '' for none); with the main workload only")
    ap.add_argument("--cpu-rows", type=int, default=128,
                    help="rows of the one-thread CPU baseline sample (about 13 s on one core)")
    ap.add_argument("--cpu-threads", type=int, default=16,
                    help="worker threads of the all-cores CPU baseline leg (one per host core, at most this)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", dest="copy_probe", action="store_true", default=True,
                    help="time a plain 256 MiB device copy in the same run (achievable HBM bandwidth, reported "
                         "beside the peak; the reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE); "
                         "on by default")
    ap.add_argument("--no-copy-probe", dest="copy_probe", action="store_false")
    return ap.parse_args()


# ----------------------------------------------------------------- workloads

# Bytes of logits the timed steps rotate through, so that no step reads its
# logits from the 256 MB Infinity Cache a previous step left them in.
ROTATE_BYTES = 3 * (256 << 20)
PLAIN = {"multinomial": "T 0.8, topK 0, topP 1 (a full-vocabulary draw, the generate() defaults with a temperature)",
         "topk_deep": "T 0.8, topK 200, topP 0.95", "typical": "T 0.8, topK 40, typicalP 0.9"}


def rotated(torch, device, host, dtype_in):
    """n >= 1 device copies of the [rows][V] logits whose total size is at
    least ROTATE_BYTES, as one tensor [n][rows][V]."""
    if dtype_in == "bf16":
        t = torch.from_numpy(host.view(np.int16)).to(device).view(torch.bfloat16)
    else:
        t = torch.from_numpy(host).to(device)
    nbytes = t.numel() * t.element_size()
    n = max(2, -(-ROTATE_BYTES // nbytes))
    out = torch.empty((n,) + tuple(t.shape), dtype=t.dtype, device=device)
    out[:] = t
    return out


def build_workload(name, gs, torch, device):
    """Device-resident inputs + one gs_batch per rotated logits copy.

    Returns dict(rows, batches=[(batch, keep)], sampler, desc, scan_bytes_per_row, step_bytes, cpu=..., ...)."""
    W = gs.workloads
    rt = gs.runtime
    out = {"name": name}
    if name in ("penalties", "single_row", "heavy_tail") or name in PLAIN:
        if name == "penalties":
            w = W.penalties()
        elif name == "single_row":
            w = W.single_row()
        elif name == "heavy_tail":
            w = W.heavy_tail()
        else:
            w = getattr(W, name)()
        window = w.configs[0].repetitionWindow if w.histories is not None else 0
        conf = np.stack([rt.row_config(c, seed=s) for c, s in zip(w.configs, w.seeds)])
        s = gs.Sampler(vocab_size=V, max_rows=w.rows)
        copies = rotated(torch, device, w.logits, w.dtype)
        batches = [s.prepare(copies[i], conf, histories=w.histories) for i in range(copies.shape[0])]
        esize = 2 if w.dtype == "bf16" else 4
        per_row = esize * V + 4 * window  # logits + window ids, read once by the scan
        if name == "penalties":
            desc = ("penalties: 256 x 262144 f32 logits ~ N(0, 3^2); 512-id Zipf(1.1) histories, repetition 1.1, "
                    "presence 0.5, frequency 0.3, window 512; T 0.7, topK 50, topP 0.9; row r seeds SeededRandom(r)")
        elif name == "single_row":
            desc = "single_row: 1 x 262144 f32 logits ~ N(0, 3^2); T 0.8, topK 40, topP 0.95, seed 42"
        elif name == "heavy_tail":
            desc = (f"heavy_tail: {w.rows} x {V} bf16 logits 8 ln(rank^-1.1) + N(0, 0.5^2), permuted per row; "
                    "topP 0.9, T 1, seed = row")
        else:
            desc = f"{name}: {w.rows} x {V} f32 logits ~ N(0, 3^2); {PLAIN[name]}; seed = row"
        out.update(rows=w.rows, sampler=s, batches=batches, copies=copies, workload=w, dtype_in=w.dtype,
                   scan_bytes_per_row=per_row, step_bytes=w.rows * (per_row + 8), dominant="scan", desc=desc)
        return out
    if name in ("constrained", "penalties_constrained"):
        w = W.constrained() if name == "constrained" else W.penalties_constrained()
        s = gs.Sampler(vocab_size=V, max_rows=w.rows)
        offsets, data = W.synthetic_vocab()
        nxt, finals = W.synthetic_dfa()
        s.set_vocab(offsets, data)
        s.set_dfa(nxt, finals)
        table = s.build_masks(list(range(64)))
        conf = np.stack([rt.row_config(c, seed=sd, mask_slot=int(st))
                         for c, sd, st in zip(w.configs, w.seeds, w.states)])
        copies = rotated(torch, device, w.logits, "f32")
        batches = [s.prepare(copies[i], conf, histories=w.histories, mask_table=table)
                   for i in range(copies.shape[0])]
        window = w.configs[0].repetitionWindow if w.histories is not None else 0
        per_row = 4 * V + 4 * window + (V // 8)  # logits + window ids + the row's legal-token bitmask
        if name == "constrained":
            desc = (f"constrained: {w.rows} x {V} f32 logits ~ N(0, 3^2); synthetic 1-12-byte vocab, 64-state "
                    "byte DFA (~3% legal), per-row start state; topP 0.95, T 1 (masks built once per state)")
        else:
            desc = (f"penalties_constrained: {w.rows} x {V} f32 logits ~ N(0, 3^2); 512-id Zipf(1.1) histories, "
                    "repetition 1.1, presence 0.5, frequency 0.3, window 512; T 0.7, topK 50, topP 0.9; the "
                    "constrained workload's 64-state byte DFA masks (~3% legal, per-row start state); seed = row")
        out.update(rows=w.rows, sampler=s, batches=batches, copies=copies, workload=w, dtype_in="f32",
                   scan_bytes_per_row=per_row, step_bytes=w.rows * (per_row + 8), dominant="scan",
                   masks=table, dfa=(offsets, data, nxt, finals), desc=desc)
        return out
    if name in ("lmhead", "lmhead_fused"):
        M, D = 64, 2048
        hidden, weight = W.lmhead_inputs(M, D, V, device=device)
        hist = W.lmhead_histories(M)
        cfg = W.LMHEAD_CONFIG
        s = gs.Sampler(vocab_size=V, max_rows=M)
        offsets, data = W.synthetic_vocab()
        nxt, finals = W.synthetic_dfa()
        s.set_vocab(offsets, data)
        s.set_dfa(nxt, finals)
        table = s.build_masks(list(range(64)))
        states = [int(W.rng(7, r).integers(0, 64)) for r in range(M)]
        conf = np.stack([rt.row_config(cfg, seed=r, softcap_value=0.0, mask_slot=states[r]) for r in range(M)])
        scratch = torch.empty((M, V), dtype=torch.float32, device=device)
        batch, keep = s.prepare(scratch, conf, histories=hist, mask_table=table)
        if name == "lmhead_fused":
            # the head's epilogue computes the chunk statistics (GS_BATCH_FUSED_HEAD)
            batch.hints |= rt.GS_BATCH_FUSED_HEAD
            out["kernel"] = "lmhead_scan_kernel"
        keep += [hidden, weight, scratch]
        out.update(rows=M, sampler=s, batches=[(batch, keep)], dtype_in="bf16", hidden=hidden, weight=weight,
                   scratch=scratch, histories=hist, states=states, masks=table, dfa=(offsets, data, nxt, finals),
                   lm_bytes=2 * V * D + 2 * M * D, lm_logits_bytes=4 * M * V, lm_flops=2 * M * D * V,
                   step_bytes=2 * V * D + 2 * M * D + 4 * 256 * M + 8 * M, dominant="lmhead",
                   desc=f"{name}: H {M} x {D} bf16 ~ N(0,1), W {V} x {D} bf16 ~ N(0, 0.02^2), softcap 30, "
                        "256-id histories (window 256), DFA masks, topK 64, topP 0.95, T 1, seed = row")
        return out
    if name == "qat":
        # the reference's own producer: one decode row through the int2 QAT
        # head (V x 1536 2-bit codes, block-major), then the sampler
        M, D = 1, 1536
        rng = np.random.default_rng(5)
        n_words = V * D // 16
        # three copies of the 96 MiB of codes (more than the 256 MB Infinity
        # Cache), step i reading copy i mod 3
        codes = [torch.from_numpy(rng.integers(0, 2 ** 32, n_words, dtype=np.uint64).astype(np.uint32)
                                  .view(np.int32)).to(device) for _ in range(3)]
        scales = torch.from_numpy((0.0008 + (np.arange(V) % 29) * 0.000025).astype(np.float32)).to(device)
        x = torch.from_numpy(rng.normal(0, 1.5, (M, D)).astype(np.float32)).to(device)
        cfg = gs.DecodingConfig(temperature=0.8, topK=40, topP=0.95)
        s = gs.Sampler(vocab_size=V, max_rows=M)
        conf = np.stack([rt.row_config(cfg, seed=42)])
        scratch = torch.empty((M, V), dtype=torch.float32, device=device)
        batch, keep = s.prepare(scratch, conf)
        out.update(rows=M, sampler=s, batches=[(batch, keep)], dtype_in="f32", qat=(x, codes, scales),
                   scratch=scratch, histories=None, states=None,
                   lm_bytes=V * D // 4 + 4 * V + 4 * M * D, lm_logits_bytes=4 * M * V, lm_flops=2 * M * D * V,
                   step_bytes=V * D // 4 + 4 * V + 4 * M * D + 8 * M * V + 16 * M, dominant="lmhead",
                   kernel="qat_tile_kernel", config_obj=cfg,
                   desc=(f"qat: 1 x {D} f32 activation ~ N(0, 1.5^2) through the int2 QAT head, {V} x {D} "
                         "2-bit codes (block-major, 3 rotated copies), row scales 0.0008 + (r mod 29) 2.5e-5, "
                         "output SRQ 0.125; then the sampler, T 0.8, topK 40, topP 0.95, seed 42"))
        return out
    raise SystemExit(f"unknown workload {name}")


def launch_step(wl, i, stream):
    s = wl["sampler"]
    batch = wl["batches"][i % len(wl["batches"])][0]
    if wl["name"] in ("lmhead", "lmhead_fused"):
        s.lmhead_sample_launch(wl["hidden"], wl["weight"], 30.0, wl["scratch"], batch, stream)
    elif wl["name"] == "qat":
        x, codes, scales = wl["qat"]
        s.qat_lmhead_sample_launch(x, codes[i % len(codes)], scales, wl["scratch"], batch,
                                   layout=gs_layout_block_major(), output_scale=0.125, stream=stream)
    else:
        s.launch(batch, stream)


def gs_layout_block_major():
    import gsample

    return gsample.runtime.GS_QAT_BLOCK_MAJOR


# -------------------------------------------------------------- CPU baseline


def _cfg_dict(c):
    return {k: getattr(c, k) for k in ("temperature", "topK", "topP", "minP", "typicalP", "repetitionPenalty",
                                        "repetitionWindow", "frequencyPenalty", "presencePenalty")}


def cpu_inputs(wl):
    """(logits [rows][V] as stored, dtype, configs, seeds, histories, constraint) of the workload
    for the CPU restatement; the lm_head workload's logits are the ones the GPU produced."""
    if wl["name"] in ("lmhead", "lmhead_fused"):
        logits = wl["scratch"].cpu().numpy()
        import gsample

        cfgs = [gsample.workloads.LMHEAD_CONFIG] * wl["rows"]
        return logits, "f32", cfgs, list(range(wl["rows"])), wl["histories"], wl["states"]
    if wl["name"] == "qat":
        return wl["scratch"].cpu().numpy(), "f32", [wl["config_obj"]] * wl["rows"], [42], None, None
    w = wl["workload"]
    return w.logits, wl["dtype_in"], w.configs, w.seeds, w.histories, w.states


def run_node_leg(wl, node, pick, threads, tmp):
    """The JavaScript restatement over rows `pick` on `threads` Node threads."""
    logits, dtype, cfgs, seeds, hists, states = cpu_inputs(wl)
    sub = np.ascontiguousarray(logits[pick])
    sub.tofile(os.path.join(tmp, "logits.bin"))
    spec = {"logits": os.path.join(tmp, "logits.bin"), "dtype": dtype, "rows": len(pick), "vocab": V,
            "pick": list(range(len(pick))), "seeds": [int(seeds[r]) for r in pick], "warmup": 1,
            "threads": threads, "out": os.path.join(tmp, "out.json"),
            "configs": [_cfg_dict(cfgs[r]) for r in pick]}
    if hists is not None:
        hist = [np.asarray(hists[r], np.int32) for r in pick]
        off = np.zeros(len(pick) + 1, np.float64)
        off[1:] = np.cumsum([h.size for h in hist])
        off.tofile(os.path.join(tmp, "hoff.bin"))
        np.concatenate(hist).astype(np.int32).tofile(os.path.join(tmp, "hids.bin"))
        spec["history_offsets"] = os.path.join(tmp, "hoff.bin")
        spec["history_ids"] = os.path.join(tmp, "hids.bin")
    if states is not None:
        offsets, data, nxt, finals = wl["dfa"]
        np.asarray(offsets, np.float64).tofile(os.path.join(tmp, "voff.bin"))
        np.asarray(data, np.uint8).tofile(os.path.join(tmp, "vbytes.bin"))
        np.asarray(nxt, np.int32).tofile(os.path.join(tmp, "next.bin"))
        np.asarray(finals, np.uint8).tofile(os.path.join(tmp, "finals.bin"))
        spec["constraint"] = {"next": os.path.join(tmp, "next.bin"), "finals": os.path.join(tmp, "finals.bin"),
                              "states": int(nxt.shape[0]), "vocab_offsets": os.path.join(tmp, "voff.bin"),
                              "vocab_bytes": os.path.join(tmp, "vbytes.bin"),
                              "row_states": [int(states[r]) for r in pick], "termination": []}
    with open(os.path.join(tmp, "spec.json"), "w") as f:
        json.dump(spec, f)
    runner = os.path.join(ROOT, "oracle", "node_runner.js")
    subprocess.run([node, runner, os.path.join(tmp, "spec.json")], check=True, timeout=900)
    with open(os.path.join(tmp, "out.json")) as f:
        return json.load(f)


def cpu_baseline(wl, tokens, probs, n_rows, threads_cap):
    """Times the reference sampler's JavaScript restatement (with the masking
    restatement for constrained rows) on Node on bounded row samples: (i) one
    thread, as the reference runs; (ii) the rows split over worker threads,
    one per host core up to `threads_cap`. Compares both legs' ids with the
    GPU's on those rows."""
    node = shutil.which("node")
    if not node:
        log("cpu baseline: node is not installed; skipped")
        return None, None
    rows = wl["rows"]
    step = max(1, rows // n_rows)
    pick1 = list(range(0, rows, step))[:n_rows]
    host_cpus = os.cpu_count() or 1
    threads = max(1, min(threads_cap, host_cpus))
    pickn = list(range(min(rows, 256)))
    tmp = tempfile.mkdtemp(prefix="gs_cpu_")
    try:
        log(f"cpu baseline (i): node, 1 thread, {len(pick1)} rows")
        r1 = run_node_leg(wl, node, pick1, 1, tmp)
        log(f"cpu baseline (ii): node, {threads} threads, {len(pickn)} rows")
        rn = run_node_leg(wl, node, pickn, threads, tmp)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    checked, mism, rel = 0, 0, 0.0
    for res, pick in ((r1, pick1), (rn, pickn)):
        for k, r in enumerate(pick):
            checked += 1
            if int(tokens[r]) != int(res["tokens"][k]):
                mism += 1
            p = res["probabilities"][k]
            if p:
                rel = max(rel, abs(probs[r] - p) / abs(p))
    what = "the sampler" if wl["name"] not in ("constrained", "penalties_constrained", "lmhead", "lmhead_fused") else (
        "legal-id walk (cached per state) + maskConstraintLogits + the sampler")
    if wl["name"] in ("lmhead", "lmhead_fused"):
        what += " on the GPU-produced logits (no CPU bf16 GEMM exists in the reference)"
    if wl["name"] == "qat":
        what += " on the GPU-produced logits (the QAT head's CPU leg is timed in qat_cpu)"
    base = {"value": round(len(pick1) / r1["seconds"], 2), "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": (f"{len(pick1)} of the {rows} rows (one in {step}), {r1['seconds']:.2f} s; JavaScript "
                       f"restatement of {what} on Node {r1['node']}, {r1['cpu_model']} ({r1['host_cpus']} host cpus)"),
            "all_cores": {"value": round(len(pickn) / rn["seconds"], 2), "unit": "rows/s", "cores": rn["threads"],
                          "sample": (f"{len(pickn)} rows split over {rn['threads']} worker_threads "
                                     f"(one per host core, at most {threads_cap}), {rn['seconds']:.2f} s")}}
    parity = {"rows_checked": checked, "token_mismatches": mism, "max_prob_rel_diff": rel}
    return base, parity


def qat_cpu_leg(wl):
    """The QAT head's CPU leg: the C restatement of cpuQatLinear (oracle/qat_ref.c,
    one thread, binary64 as the reference's JavaScript) on the step's activation and
    the codes copy the last timed step read, compared bit for bit with the GPU's
    logits."""
    from oracle import oracle

    x, codes, scales = wl["qat"]
    V, D = wl["scratch"].shape[1], x.shape[1]
    bm = codes[0].cpu().numpy().view(np.uint32).reshape(D // 64, V, 4)
    row_major = np.ascontiguousarray(bm.transpose(1, 0, 2)).reshape(-1)
    t0 = time.time()
    want = oracle.qat_linear_int2(x.cpu().numpy()[0], row_major, scales.cpu().numpy(), D, V, 0.0, 0.125)
    sec = time.time() - t0
    s = wl["sampler"]
    got = s.qat_lmhead(x, codes[0], scales, layout=gs_layout_block_major(), output_scale=0.125).cpu().numpy()[0]
    return {"value": round(1.0 / sec, 3), "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"1 row: cpuQatLinear restated in C (oracle/qat_ref.c), {sec:.2f} s",
            "bit_exact_with_gpu": bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))}


# ---------------------------------------------------------------------- main


def copy_probe(torch, device, stream, steps):
    """A plain 256 MiB device-to-device copy (reads and writes each byte once):
    the achievable HBM bandwidth in the same run."""
    src = torch.ones(64 << 20, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    with torch.cuda.stream(stream):
        for _ in range(3):
            dst.copy_(src)
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        for _ in range(steps):
            dst.copy_(src)
        c1.record(stream)
    torch.cuda.synchronize()
    copy_ms = c0.elapsed_time(c1) / steps
    nbytes = src.numel() * src.element_size()
    del dst, src
    return {"bytes_read": nbytes, "bytes_written": nbytes, "avg_us": round(copy_ms * 1000, 2),
            "gbps_read_plus_write": round(2 * nbytes / (copy_ms * 1e6), 1)}


def measure(wl, gs, torch, stream, steps, warmup):
    """Warmup, K timed steps (step rate), K more steps with per-kernel events.
    Returns (ms_per_step, stages, tokens, probs, flags) of the workload."""
    s = wl["sampler"]
    sp = stream.cuda_stream
    n_rot = len(wl["batches"])
    for i in range(warmup):
        launch_step(wl, i, sp)
    torch.cuda.synchronize()
    log(f"{wl['name']}: warmup {warmup} steps done")

    # the step rate: K steps bracketed by two events on the launch stream,
    # step i reading logits copy i mod n
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        launch_step(wl, i, sp)
    end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / steps
    log(f"{wl['name']}: timed {steps} steps: {ms_per_step * 1000:.1f} us/step")

    # kernel durations: K more steps, every kernel launched with start/stop
    # HIP events on the stream it runs on (the events slow a step down, so
    # the step rate above is timed without them)
    s.timing_begin(steps)
    for i in range(steps):
        launch_step(wl, i, sp)
    torch.cuda.synchronize()
    stages = s.timing_end()
    log(f"{wl['name']}: stage timing over {steps} more steps: {stages}")

    # results of the last step (each loop above counts its steps from 0, so
    # the last launch used buffer (steps - 1) mod n_rot)
    last = (steps - 1) % n_rot
    res = wl["batches"][last][1][-1] if wl["name"] not in ("lmhead", "lmhead_fused") else wl["batches"][0][1][-4]
    if wl["name"] == "qat":
        res = wl["batches"][0][1][-1]
    raw = res.cpu().numpy().view(np.uint8).reshape(-1)[: wl["rows"] * 16]
    rr = raw.view(gs.runtime.RESULT_DTYPE)
    return ms_per_step, stages, rr["token"].copy(), rr["probability"].copy(), rr["flags"].copy()


def roofline_of(wl, stages):
    """The dominant kernel's roofline object from the per-kernel timings."""
    rows = wl["rows"]
    dom = wl["dominant"]
    dom_ms, dom_calls = stages[dom]
    dom_avg_ms = dom_ms / max(1, dom_calls)
    if dom == "lmhead":
        algo = wl["lm_bytes"]
        mfma_tflops = wl["lm_flops"] / (dom_avg_ms * 1e9)
    else:
        algo = rows * wl["scan_bytes_per_row"]
        mfma_tflops = None
    achieved = algo / (dom_avg_ms * 1e6)
    kname = wl.get("kernel") or {"scan": "scan_kernel", "lmhead": "lmhead_resident_kernel"}[dom]
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(wl["name"], kname),
                "kernel": kname, "algorithmic_bytes_per_launch": int(algo),
                "kernel_avg_us": round(dom_avg_ms * 1000, 2),
                "stage_avg_us": {k: round(v[0] / v[1] * 1000, 2) for k, v in stages.items() if v[1]},
                "rotated_logits_buffers": len(wl["batches"])}
    if wl["name"] == "qat":
        # binary64 fused multiply-adds on the vector units, not MFMA
        roofline["f64_tflops"] = round(mfma_tflops, 2)
        roofline["f64_frac_vector_peak"] = round(mfma_tflops / F64_VECTOR_PEAK_TFLOPS, 4)
        roofline["logits_write_bytes"] = wl["lm_logits_bytes"]
        mfma_tflops = None
    if mfma_tflops is not None:
        roofline["mfma_tflops"] = round(mfma_tflops, 1)
        roofline["mfma_frac_bf16_dense"] = round(mfma_tflops / BF16_PEAK_TFLOPS, 4)
        # the unfused logits write, reported beside the weight-streaming figure
        roofline["logits_write_bytes"] = wl["lm_logits_bytes"]
        roofline["achieved_with_logits_write"] = round((algo + wl["lm_logits_bytes"]) / (dom_avg_ms * 1e6), 1)
    return roofline


def step_figures(wl, ms_per_step, flags, tokens):
    return {"value": round(wl["rows"] / (ms_per_step / 1000.0), 1), "ms_per_step": round(ms_per_step, 5),
            "step_hbm_gbps": round(wl["step_bytes"] / (ms_per_step * 1e6), 1),
            "step_hbm_frac": round(wl["step_bytes"] / (ms_per_step * 1e6) / HBM_PEAK_GBPS, 4),
            "rows_failed": int(np.sum(tokens < 0)),
            "rows_exact_path": int(np.sum((flags & 2) != 0)),
            "rows_topp_tie": int(np.sum((flags & 1) != 0))}


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the sampling stage shards by rows (C1-C4) or "
                                   "by vocab (lm_head) across GPUs, which is not built; run with --gpus 1"}))
        sys.exit(2)
    import torch

    import gsample as gs

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    device = torch.device("cuda", 0)
    # a dedicated stream at the default priority: torch's default stream has a
    # null handle, which the library would read as "use the context's stream"
    stream = torch.cuda.Stream(device)
    log(f"building workload {args.workload}")
    t0 = time.time()
    wl = build_workload(args.workload, gs, torch, device)
    torch.cuda.synchronize()
    log(f"workload ready in {time.time() - t0:.1f} s ({len(wl['batches'])} rotated logits buffers)")
    ms_per_step, stages, tokens, probs, flags = measure(wl, gs, torch, stream, args.steps, args.warmup)
    roofline = roofline_of(wl, stages)
    fig = step_figures(wl, ms_per_step, flags, tokens)
    config = {"workload": wl["desc"], "rows": wl["rows"], "vocab": V, "logits_dtype": wl["dtype_in"]}

    if args.copy_probe:
        cp = copy_probe(torch, device, stream, args.steps)
        # the dominant kernel against the copy's read + write rate (its own
        # traffic is almost all reads)
        cp["dominant_frac_of_copy"] = round(roofline["achieved"] / cp["gbps_read_plus_write"], 4)
        cp["step_frac_of_copy"] = round(fig["step_hbm_gbps"] / cp["gbps_read_plus_write"], 4)
        roofline["copy_probe"] = cp

    base, parity = (None, None)
    if not args.no_cpu:
        base, parity = cpu_baseline(wl, tokens, probs, args.cpu_rows, args.cpu_threads)
    qat_cpu = qat_cpu_leg(wl) if wl["name"] == "qat" and not args.no_cpu else None
    s = wl["sampler"]
    s.synchronize()
    s.close()
    del wl
    torch.cuda.empty_cache()

    also = {}
    for name in [n for n in args.also.split(",") if n and n != args.workload]:
        log(f"building workload {name}")
        w2 = build_workload(name, gs, torch, device)
        torch.cuda.synchronize()
        m2, st2, tok2, pr2, fl2 = measure(w2, gs, torch, stream, args.steps, args.warmup)
        entry = {"config": {"workload": w2["desc"], "rows": w2["rows"], "vocab": V, "logits_dtype": w2["dtype_in"]}}
        entry.update(step_figures(w2, m2, fl2, tok2))
        entry["roofline"] = roofline_of(w2, st2)
        if not args.no_cpu:
            b2, p2 = cpu_baseline(w2, tok2, pr2, max(8, args.cpu_rows // 4), args.cpu_threads)
            entry["cpu_baseline"] = b2
            if p2 is not None:
                entry["parity_sample"] = p2
        also[name] = entry
        w2["sampler"].close()
        del w2
        torch.cuda.empty_cache()

    line = {
        "metric": METRIC, "value": fig["value"], "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": fig["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32/f64",
        "precision": ("logits f32 (bf16 widened exactly); normaliser terms binary32 hardware exp2 summed in "
                      "binary64; every ranking, cut and draw decided in binary64 as the reference does"),
        "data": "synthetic",
        "config": config,
        "step_hbm_gbps": fig["step_hbm_gbps"], "step_hbm_frac": fig["step_hbm_frac"],
        "roofline": roofline, "cpu_baseline": base,
        "rows_failed": fig["rows_failed"], "rows_exact_path": fig["rows_exact_path"],
        "rows_topp_tie": fig["rows_topp_tie"],
    }
    if parity is not None:
        line["parity_sample"] = parity
    if qat_cpu is not None:
        line["qat_cpu"] = qat_cpu
    if also:
        line["also"] = also
    print(json.dumps(line), flush=True)
    bad = (parity is not None and parity["token_mismatches"]) or any(
        e.get("parity_sample", {}).get("token_mismatches") for e in also.values())
    if bad:
        sys.exit(1)


if __name__ == "__main__":
    main()
