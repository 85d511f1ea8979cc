#!/usr/bin/env python3
"""Throughput of the batched sampling stage on one MI355X.

A step is one gs_sample call (chunk scan -> row finish -> exact replay) over a
batch of synthetic logits already resident in HBM; `value` is sampled rows per
second over the timed steps. The default workload is the batched penalties +
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
  cpu_baseline  the JavaScript restatement of the reference sampler run by
                Node on one host core over a bounded sample of the same rows
                (falls back to the C restatement when node is absent), and a
                bit-exact comparison of those rows' token ids.

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
                    choices=["penalties", "single_row", "heavy_tail", "constrained", "lmhead"])
    ap.add_argument("--cpu-rows", type=int, default=128, help="rows of the CPU baseline sample (about 14 s on one core)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time a plain device copy of the logits' byte count (achievable HBM bandwidth; "
                         "the reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


# ----------------------------------------------------------------- workloads


def build_workload(name, gs, torch, device):
    """Device-resident inputs + the gs_batch for one workload.

    Returns dict(rows, batch, keep, sampler, desc, scan_bytes_per_row, step_bytes, rows_cpu, ...)."""
    W = gs.workloads
    rt = gs.runtime
    out = {"name": name}
    if name in ("penalties", "single_row"):
        w = W.penalties() if name == "penalties" else W.single_row()
        window = w.configs[0].repetitionWindow
        conf = np.stack([rt.row_config(c, seed=s) for c, s in zip(w.configs, w.seeds)])
        s = gs.Sampler(vocab_size=V, max_rows=w.rows)
        logits = torch.from_numpy(w.logits).to(device)
        batch, keep = s.prepare(logits, conf, histories=w.histories)
        per_row = 4 * V + 4 * window  # logits + window ids, read once by the scan
        out.update(rows=w.rows, sampler=s, batch=batch, keep=keep, workload=w, dtype_in="f32",
                   scan_bytes_per_row=per_row, step_bytes=w.rows * (per_row + 8),
                   dominant="scan",
                   desc=(f"{name}: {w.rows} x {V} f32 logits ~ N(0, 3^2); "
                         + ("512-id Zipf(1.1) histories, repetition 1.1, presence 0.5, frequency 0.3, window 512; "
                            "T 0.7, topK 50, topP 0.9; row r seeds SeededRandom(r)"
                            if name == "penalties" else "T 0.8, topK 40, topP 0.95, seed 42")))
        return out
    if name == "heavy_tail":
        w = W.heavy_tail()
        conf = np.stack([rt.row_config(c, seed=s) for c, s in zip(w.configs, w.seeds)])
        s = gs.Sampler(vocab_size=V, max_rows=w.rows)
        logits = torch.from_numpy(w.logits.view(np.int16)).to(device).view(torch.bfloat16)
        batch, keep = s.prepare(logits, conf)
        per_row = 2 * V
        out.update(rows=w.rows, sampler=s, batch=batch, keep=keep, workload=w, dtype_in="bf16",
                   scan_bytes_per_row=per_row, step_bytes=w.rows * (per_row + 8), dominant="scan",
                   desc=f"heavy_tail: {w.rows} x {V} bf16 logits 8 ln(rank^-1.1) + N(0, 0.5^2), permuted per row; "
                        "topP 0.9, T 1, seed = row")
        return out
    if name == "constrained":
        w = W.constrained()
        s = gs.Sampler(vocab_size=V, max_rows=w.rows)
        offsets, data = W.synthetic_vocab()
        nxt, finals = W.synthetic_dfa()
        s.set_vocab(offsets, data)
        s.set_dfa(nxt, finals)
        table = s.build_masks(list(range(64)))
        conf = np.stack([rt.row_config(c, seed=sd, mask_slot=int(st))
                         for c, sd, st in zip(w.configs, w.seeds, w.states)])
        logits = torch.from_numpy(w.logits).to(device)
        batch, keep = s.prepare(logits, conf, mask_table=table)
        per_row = 4 * V + (V // 8)  # logits + the row's legal-token bitmask
        out.update(rows=w.rows, sampler=s, batch=batch, keep=keep, workload=w, dtype_in="f32",
                   scan_bytes_per_row=per_row, step_bytes=w.rows * (per_row + 8), dominant="scan",
                   masks=table, vocab_tables=(offsets, data, nxt, finals),
                   desc=f"constrained: {w.rows} x {V} f32 logits ~ N(0, 3^2); synthetic 1-12-byte vocab, 64-state "
                        "byte DFA (~3% legal), per-row start state; topP 0.95, T 1 (masks built once per state)")
        return out
    if name == "lmhead":
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
        keep += [hidden, weight, scratch]
        out.update(rows=M, sampler=s, batch=batch, keep=keep, dtype_in="bf16", hidden=hidden, weight=weight,
                   scratch=scratch, histories=hist, states=states, masks=table,
                   lm_bytes=2 * V * D + 2 * M * D + 4 * M * V, lm_flops=2 * M * D * V,
                   step_bytes=2 * V * D + 2 * M * D + 4 * 256 * M + 8 * M, dominant="lmhead",
                   desc=f"lmhead: H {M} x {D} bf16 ~ N(0,1), W {V} x {D} bf16 ~ N(0, 0.02^2), softcap 30, "
                        "256-id histories (window 256), DFA masks, topK 64, topP 0.95, T 1, seed = row")
        return out
    raise SystemExit(f"unknown workload {name}")


def launch_step(wl, stream):
    s = wl["sampler"]
    if wl["name"] == "lmhead":
        s.lmhead_sample_launch(wl["hidden"], wl["weight"], 30.0, wl["scratch"], wl["batch"], stream)
    else:
        s.launch(wl["batch"], stream)


# -------------------------------------------------------------- CPU baseline


def cpu_baseline(wl, gs, tokens, probs, n_rows):
    """Times the reference sampler's restatement on a bounded row sample and
    compares its ids with the GPU's on those rows."""
    if wl["name"] not in ("penalties", "single_row", "heavy_tail"):
        return None, None
    w = wl["workload"]
    step = max(1, w.rows // n_rows)
    pick = list(range(0, w.rows, step))[:n_rows]
    node = shutil.which("node")
    if node:
        tmp = tempfile.mkdtemp(prefix="gs_cpu_")
        try:
            sub = np.ascontiguousarray(w.logits[pick])
            sub.tofile(os.path.join(tmp, "logits.bin"))
            spec = {"logits": os.path.join(tmp, "logits.bin"), "dtype": wl["dtype_in"], "rows": len(pick),
                    "vocab": V, "pick": list(range(len(pick))), "seeds": [w.seeds[r] for r in pick],
                    "warmup": 1, "out": os.path.join(tmp, "out.json"),
                    "configs": [{k: getattr(w.configs[r], k) for k in (
                        "temperature", "topK", "topP", "minP", "typicalP", "repetitionPenalty", "repetitionWindow",
                        "frequencyPenalty", "presencePenalty")} for r in pick]}
            if w.histories is not None:
                hist = [np.asarray(w.histories[r], np.int32) for r in pick]
                off = np.zeros(len(pick) + 1, np.float64)
                off[1:] = np.cumsum([h.size for h in hist])
                off.tofile(os.path.join(tmp, "hoff.bin"))
                np.concatenate(hist).astype(np.int32).tofile(os.path.join(tmp, "hids.bin"))
                spec["history_offsets"] = os.path.join(tmp, "hoff.bin")
                spec["history_ids"] = os.path.join(tmp, "hids.bin")
            with open(os.path.join(tmp, "spec.json"), "w") as f:
                json.dump(spec, f)
            runner = os.path.join(ROOT, "oracle", "node_runner.js")
            log(f"cpu baseline: node on {len(pick)} rows")
            subprocess.run([node, runner, os.path.join(tmp, "spec.json")], check=True, timeout=600)
            with open(os.path.join(tmp, "out.json")) as f:
                res = json.load(f)
        finally:
            shutil.rmtree(tmp, ignore_errors=True)
        seconds = res["seconds"]
        ref_tokens, ref_probs = res["tokens"], res["probabilities"]
        kind_note = f"JavaScript restatement on Node {res['node']}, 1 thread, {res['cpu_model']} ({res['host_cpus']} host cpus)"
    else:
        from oracle import oracle as orc  # the checker's C restatement

        log(f"cpu baseline: C restatement on {len(pick)} rows")
        ref_tokens, ref_probs = [], []
        seconds = 0.0
        for r in pick:
            c = w.configs[r]
            x = w.logits[r] if wl["dtype_in"] == "f32" else gs.workloads.bf16_bits_to_f32(w.logits[r])
            cfg = orc.Decoding(temperature=c.temperature, topK=c.topK, topP=c.topP, minP=c.minP, typicalP=c.typicalP,
                               repetitionPenalty=c.repetitionPenalty, repetitionWindow=c.repetitionWindow,
                               frequencyPenalty=c.frequencyPenalty, presencePenalty=c.presencePenalty)
            hist = w.histories[r] if w.histories is not None else []
            t0 = time.perf_counter()
            t, tr = orc.sample_token(x, hist, cfg, orc.draw(w.seeds[r], 0))
            seconds += time.perf_counter() - t0
            ref_tokens.append(t)
            ref_probs.append(tr.probability)
        kind_note = "C restatement (oracle/sampler_ref.c), 1 thread"
    mism = [r for k, r in enumerate(pick) if int(tokens[r]) != int(ref_tokens[k])]
    rel = max((abs(probs[r] - ref_probs[k]) / abs(ref_probs[k]) if ref_probs[k] else 0.0)
              for k, r in enumerate(pick))
    base = {"value": len(pick) / seconds, "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{len(pick)} of the {w.rows} rows (one row in {step}), {seconds:.2f} s; {kind_note}"}
    parity = {"rows_checked": len(pick), "token_mismatches": len(mism), "max_prob_rel_diff": rel}
    return base, parity


# ---------------------------------------------------------------------- main


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
    log(f"building workload {args.workload}")
    t0 = time.time()
    wl = build_workload(args.workload, gs, torch, device)
    torch.cuda.synchronize()
    log(f"workload ready in {time.time() - t0:.1f} s")
    s = wl["sampler"]
    # a dedicated stream at the default priority: torch's default stream has a
    # null handle, which the library would read as "use the context's stream"
    stream = torch.cuda.Stream(device)
    sp = stream.cuda_stream
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        launch_step(wl, sp)
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} steps done")

    # the step rate: K steps bracketed by two events on the launch stream
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        launch_step(wl, sp)
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    log(f"timed {args.steps} steps: {ms_per_step * 1000:.1f} us/step")

    # kernel durations: K more steps, every kernel launched with start/stop
    # HIP events on the stream it runs on (the events slow a step down, so
    # the step rate above is timed without them)
    s.timing_begin(args.steps)
    for _ in range(args.steps):
        launch_step(wl, sp)
    torch.cuda.synchronize()
    stages = s.timing_end()
    log(f"stage timing over {args.steps} more steps: {stages}")

    # results of the last step
    res = wl["keep"][-1] if wl["name"] != "lmhead" else wl["keep"][-4]
    raw = res.cpu().numpy().view(np.uint8).reshape(-1)[: wl["rows"] * 16]
    rr = raw.view(gs.runtime.RESULT_DTYPE)
    tokens, probs, flags = rr["token"], rr["probability"], rr["flags"]
    bad = int(np.sum(tokens < 0))
    exact_rows = int(np.sum((flags & gs.GS_FLAG_EXACT_PATH) != 0))
    tie_rows = int(np.sum((flags & gs.GS_FLAG_TOPP_TIE) != 0))

    rows = wl["rows"]
    value = rows / (ms_per_step / 1000.0)
    dom = wl["dominant"]
    dom_ms, dom_calls = stages[dom]
    dom_avg_ms = dom_ms / max(1, dom_calls)
    if dom == "lmhead":
        achieved = wl["lm_bytes"] / (dom_avg_ms * 1e6)
        mfma_tflops = wl["lm_flops"] / (dom_avg_ms * 1e9)
    else:
        achieved = rows * wl["scan_bytes_per_row"] / (dom_avg_ms * 1e6)
        mfma_tflops = None
    kname = {"scan": "scan_kernel", "lmhead": "lmhead_kernel"}[dom]
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(wl["name"], kname),
                "kernel": kname, "algorithmic_bytes_per_launch": int(
                    wl["lm_bytes"] if dom == "lmhead" else rows * wl["scan_bytes_per_row"]),
                "kernel_avg_us": round(dom_avg_ms * 1000, 2),
                "stage_avg_us": {k: round(v[0] / v[1] * 1000, 2) for k, v in stages.items() if v[1]}}
    if mfma_tflops is not None:
        roofline["mfma_tflops"] = round(mfma_tflops, 1)
        roofline["mfma_frac_bf16_dense"] = round(mfma_tflops / BF16_PEAK_TFLOPS, 4)

    if args.copy_probe:
        # a plain 256 MiB device-to-device copy: reads and writes each byte once
        src = torch.ones(64 << 20, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        with torch.cuda.stream(stream):
            for _ in range(3):
                dst.copy_(src)
            c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            c0.record(stream)
            for _ in range(args.steps):
                dst.copy_(src)
            c1.record(stream)
        torch.cuda.synchronize()
        copy_ms = c0.elapsed_time(c1) / args.steps
        nbytes = src.numel() * src.element_size()
        roofline["copy_probe"] = {"bytes_read": nbytes, "bytes_written": nbytes, "avg_us": round(copy_ms * 1000, 2),
                                  "gbps_read_plus_write": round(2 * nbytes / (copy_ms * 1e6), 1)}
        del dst, src

    base, parity = (None, None)
    if not args.no_cpu:
        base, parity = cpu_baseline(wl, gs, tokens, probs, args.cpu_rows)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": wl["desc"], "rows": rows, "vocab": V, "logits_dtype": wl["dtype_in"]},
        "step_hbm_gbps": round(wl["step_bytes"] / (ms_per_step * 1e6), 1),
        "step_hbm_frac": round(wl["step_bytes"] / (ms_per_step * 1e6) / HBM_PEAK_GBPS, 4),
        "roofline": roofline, "cpu_baseline": base,
        "rows_failed": bad, "rows_exact_path": exact_rows, "rows_topp_tie": tie_rows,
    }
    if parity is not None:
        line["parity_sample"] = parity
    s.synchronize()
    print(json.dumps(line), flush=True)
    s.close()
    if parity is not None and parity["token_mismatches"]:
        sys.exit(1)


if __name__ == "__main__":
    main()
