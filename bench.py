"""Benchmark of the paged GQA decode operator on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload llama3_8b]
                    [--num-splits 0] [--no-cpu-baseline] [--all]

One step = one decode-attention call over the whole batch of the workload (default: the
Llama-3-8B decode shape the metric is quoted on, B=64 Hq=32 Hkv=8 D=128 P=16 L=4096), inputs
resident in HBM.  The timed region is K back-to-back steps on one stream, bracketed by
torch.cuda.synchronize(); inside it HIP events bracket the main kernel of every step (the
balanced single launch, or the split-KV kernel of the split grid, whose combine kernel runs
after the second event).  Prints ONE JSON line:
  value      effective KV GB/s of whole steps = algorithmic K+V bytes / (ms_per_step)
  roofline   achieved GB/s of the main kernel alone (events around it) against 8 TB/s
  cpu_baseline  the fp32 oracle (oracle/paged_attention.py) timed on this host on a bounded
             sample of the same workload.
``--all`` prints one extra JSON line per north-star configuration (no CPU baseline).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import statistics
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

import mx_flash_attn_kernel_opt__amd as pkg  # noqa: E402
from mx_flash_attn_kernel_opt__amd import _lib  # noqa: E402
from mx_flash_attn_kernel_opt__amd import workloads as W  # noqa: E402

METRIC = "decode attn µs/call + effective KV HBM GB/s (% of MI355X peak), 1 GPU"
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 * 1024 * 1024
PROFILE_DIR = os.path.join(REPO, "profiles")


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _traffic_from_profile(kernel: str, workload: str):
    """HBM bytes per launch of the main kernel, from the committed rocprofv3 --pmc summary
    (profiles/<kernel>_<workload>_traffic.md, line 'traffic_bytes_per_launch: N'), or None."""
    path = os.path.join(PROFILE_DIR, f"{kernel}_{workload}_traffic.md")
    try:
        with open(path) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


def time_workload(inp: W.DecodeInputs, steps: int, warmup: int, num_splits: int = 0) -> dict:
    """Time `steps` calls after `warmup`; events bracket the split-KV kernel of each step."""
    spec = inp.spec
    stream = torch.cuda.current_stream()
    nbytes = inp.kv_bytes()
    # Rotate distinct copies of the KV pool when one would fit in the 256 MB MALL.
    copies = 1 if nbytes >= 3 * MALL_BYTES else min(8, max(2, math.ceil(3 * MALL_BYTES / nbytes)))
    pools = [(inp.k_cache, inp.v_cache)] + [(inp.k_cache.clone(), inp.v_cache.clone())
                                            for _ in range(copies - 1)]
    plan = pkg.plan(spec.batch, spec.num_heads, spec.num_kv_heads, spec.head_dim,
                    spec.page_size, spec.max_pages, 0, num_splits, seqlen_q=spec.seqlen_q)
    ws = pkg.make_workspace(plan["workspace_bytes"], inp.device)
    out = torch.empty_like(inp.q)
    calls = [pkg.BoundDecode(inp.q, k, v, inp.block_table, inp.seq_lens, inp.scale, out=out,
                             causal=spec.causal, num_splits=num_splits, workspace=ws,
                             stream=stream)
             for k, v in pools]
    split = plan["splits"] > 1
    main_phase = _lib.MX_PHASE_MAIN_ONLY if split else _lib.MX_PHASE_ALL

    def step(i, e0=None, e1=None):
        call = calls[i % len(calls)]
        if e0 is not None:
            e0.record(stream)
        call(main_phase)
        if e1 is not None:
            e1.record(stream)
        if split:
            call(_lib.MX_PHASE_COMBINE_ONLY)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        step(i, *ev[i])
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    total_ms = start.elapsed_time(end)
    kern_us = [a.elapsed_time(b) * 1e3 for a, b in ev]
    ms_per_step = total_ms / steps
    flags = pkg.read_device_status(ws)
    if flags:
        raise RuntimeError(f"device status flags {flags} raised during the benchmark")
    kern_mean = statistics.fmean(kern_us)
    return {
        "nbytes": nbytes,
        "plan": plan,
        "ms_per_step": ms_per_step,
        "wall_ms_per_step": wall_ms / steps,
        "kernel_us_mean": kern_mean,
        "kernel_us_median": statistics.median(kern_us),
        "kernel_us_min": min(kern_us),
        "pools": copies,
        "value_gbps": nbytes / (ms_per_step * 1e-3) / 1e9,
        "kernel_gbps": nbytes / (kern_mean * 1e-6) / 1e9,
    }


def time_append(spec: W.DecodeSpec, steps: int, warmup: int, seed: int = 0) -> dict:
    """Time the paged K/V append of one new token per sequence of `spec` (the step before the
    decode): bytes are the new rows read plus the page slots written."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    B, Hkv, D = spec.batch, spec.num_kv_heads, spec.head_dim
    inp = W.make_inputs(spec, seed=seed, device="cuda")
    lens = (inp.seq_lens - 1).clamp(min=0)   # append the last token of each sequence
    kn = torch.randn(B, Hkv, D, generator=g, device="cuda").to(torch.bfloat16)
    vn = torch.randn(B, Hkv, D, generator=g, device="cuda").to(torch.bfloat16)
    ws = pkg.make_workspace(256, "cuda")
    stream = torch.cuda.current_stream()
    # validated once through the tensor API, then called with pre-built C arguments so the
    # host-side Python wrapper does not pace the GPU
    pkg.paged_kv_append(kn, vn, inp.k_cache, inp.v_cache, inp.block_table, lens, workspace=ws,
                        stream=stream)
    fn = _lib.load().mx_paged_kv_append
    cargs = [ctypes.c_void_p(t.data_ptr()) for t in (kn, vn, inp.k_cache, inp.v_cache, lens,
                                                     inp.block_table)]
    cargs += [B, 1, Hkv, D, spec.page_size, inp.k_cache.shape[0], inp.block_table.shape[1],
              ctypes.c_void_p(ws.data_ptr()), ctypes.c_void_p(stream.cuda_stream)]

    def call():
        st = fn(*cargs)
        if st != _lib.MX_STATUS_OK:
            _lib.check(st)

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        call()
    end.record(stream)
    torch.cuda.synchronize()
    if pkg.read_device_status(ws):
        raise RuntimeError("device status flags raised during the append benchmark")
    us = start.elapsed_time(end) * 1e3 / steps
    nbytes = 2 * 2 * B * Hkv * D * 2   # K and V rows, read once and written once
    del inp
    torch.cuda.empty_cache()
    return {"metric": "paged_kv_append_us_per_call", "value": round(us, 2), "unit": "us",
            "higher_is_better": False, "steps": steps, "dtype": "bf16",
            "config": {"workload": f"append_{spec.name}", "batch": B, "seqlen_new": 1,
                       "num_kv_heads": Hkv, "head_dim": D, "page_size": spec.page_size},
            "bytes_per_call": nbytes, "GBps": round(nbytes / us / 1e3, 2),
            "note": "launch-bound: one token per sequence moves bytes_per_call"}


# The reference's contest score model (archive/round_deepnight/agentC_policy_NOTES.md:17-27):
# score_c = round(100 * R_c / (R_c + t_c)) with a fixed per-case R_c in us (fitted there to the
# contest's results), total = mean over the 14 cases.  R_c was calibrated on the MetaX C500, so
# on MI355X the score says what the same model gives these times, not a contest result.
C500_SCORE_R_US = {1: 35.5, 2: 35.5, 3: 42.5, 4: 58.5, 5: 44.5, 6: 48.0, 7: 274.0, 8: 107.0,
                   9: 308.0, 10: 62.5, 11: 244.5, 12: 560.0, 13: 236.0, 14: 166.5}
# The reference's final C500 kernel time per case in us (SOTA:submission_clean_cu_67.36.txt:3-6).
C500_CLEAN_US = {1: 7, 2: 7, 3: 9, 4: 19, 5: 15, 6: 24, 7: 204, 8: 71, 9: 207, 10: 37, 11: 182,
                 12: 352, 13: 169, 14: 115}


def c500_suite(mult: int = 10, seed: int = 42) -> list[dict]:
    """The reference's 14-case contest table through the drop-in ``run_kernel`` symbol, timed
    as its harness times it (bench_all.py:38-70: events around `iters` back-to-back calls after
    5 warm-up calls, arange block table), scored with the contest model above."""
    lib = _lib.load()
    rows = []
    for case in sorted(W.C500_CASES):
        B, cap, kv = W.C500_CASES[case]
        spec = W.c500_spec(case, table="arange")
        inp = W.make_inputs(spec, seed=seed, device="cuda")
        out = torch.zeros_like(inp.q)
        nb = B * spec.max_pages
        args = [ctypes.c_void_p(t.data_ptr()) for t in (inp.q, inp.k_cache, inp.v_cache, out,
                                                        inp.seq_lens, inp.block_table)]
        args += [B, cap, 1, 32, kv, 128, 16, nb, 0]
        iters = max(W.C500_ITERS[case] * mult, 10)
        for _ in range(5):
            lib.run_kernel(*args)
        torch.cuda.synchronize()
        _lib.check(lib.mx_last_status())
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            lib.run_kernel(*args)
        end.record()
        torch.cuda.synchronize()
        t_us = start.elapsed_time(end) * 1e3 / iters
        R = C500_SCORE_R_US[case]
        rows.append({"case": case, "batch": B, "seqlen_k": cap, "num_heads_k": kv,
                     "kv_bytes": inp.kv_bytes(), "iters": iters, "us_per_call": round(t_us, 2),
                     "score": round(100 * R / (R + t_us)),
                     "c500_clean_us": C500_CLEAN_US[case],
                     "c500_clean_score": round(100 * R / (R + C500_CLEAN_US[case])),
                     "GBps": round(inp.kv_bytes() / t_us / 1e3, 1)})
        del inp, out
        torch.cuda.empty_cache()
    return rows


def cpu_baseline(inp: W.DecodeInputs, budget_s: float) -> dict:
    """fp32 oracle (the reference CPU path restated) on a bounded sample of sequences."""
    from oracle import paged_decode_reference

    threads = torch.get_num_threads()
    B = inp.spec.batch
    order = torch.randperm(B, generator=torch.Generator().manual_seed(0)).tolist()
    warm = inp.subset([order[0]])
    paged_decode_reference(warm.q, warm.k_cache, warm.v_cache, warm.block_table,
                           warm.seq_lens, warm.scale)
    spent, nbytes, done = 0.0, 0, 0
    for b in order:
        sub = inp.subset([b])
        t0 = time.perf_counter()
        paged_decode_reference(sub.q, sub.k_cache, sub.v_cache, sub.block_table,
                               sub.seq_lens, sub.scale)
        spent += time.perf_counter() - t0
        nbytes += sub.kv_bytes()
        done += 1
        if spent >= budget_s:
            break
    gbps = nbytes / spent / 1e9
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{done} of {B} sequences of {inp.spec.name}, fp32 torch oracle "
                   f"(oracle/paged_attention.py), one sequence at a time, {spent:.1f} s; "
                   f"host {_cpu_model()}, os.cpu_count()={os.cpu_count()}, "
                   f"torch threads={threads}"),
        "us_per_call_est": round(spent / done * B * 1e6, 1),
    }


def result_line(args, spec, r, cpu=None) -> dict:
    frac = r["kernel_gbps"] / HBM_PEAK_GBPS
    line = {
        "metric": METRIC,
        "value": round(r["value_gbps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "us_per_call": round(r["ms_per_step"] * 1e3, 2),
        "hbm_frac": round(r["value_gbps"] / HBM_PEAK_GBPS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/K/V, shuffled block table)",
        "config": {
            "workload": spec.name,
            "batch": spec.batch, "num_heads": spec.num_heads,
            "num_kv_heads": spec.num_kv_heads, "head_dim": spec.head_dim,
            "page_size": spec.page_size, "max_pages": spec.max_pages,
            "seq_lens": spec.seq_lens, "seq_args": list(spec.seq_args),
            "kv_bytes": r["nbytes"], "schedule": r["plan"]["schedule"],
            "workgroups": r["plan"]["workgroups"], "splits": r["plan"]["splits"],
            "tokens_per_split": r["plan"]["tokens_per_split"], "kv_pools": r["pools"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": ("mx_paged_decode_balanced" if r["plan"]["schedule"] == "balanced"
                       else "mx_paged_decode_splitkv"),
            "achieved": round(r["kernel_gbps"], 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(frac, 4),
            "traffic": _traffic_from_profile(
                "balanced" if r["plan"]["schedule"] == "balanced" else "splitkv", spec.name),
            "kernel_us_mean": round(r["kernel_us_mean"], 2),
            "kernel_us_median": round(r["kernel_us_median"], 2),
        },
        "wall_ms_per_step": round(r["wall_ms_per_step"], 5),
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    return line


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=W.BENCH_DEFAULT)
    ap.add_argument("--num-splits", type=int, default=0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU-baseline work (bounded sample)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--all", action="store_true",
                    help="also print one line per north-star configuration")
    ap.add_argument("--suite", choices=["c500"], default=None,
                    help="run the reference's 14-case contest suite through run_kernel "
                         "instead of the main workload and print its per-case lines and score")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after timing, run 5 plain 1 GiB device copies (torch copy_) so a "
                         "rocprofv3 --pmc pass can scale FETCH_SIZE/WRITE_SIZE by a kernel of "
                         "known traffic")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this operator is benchmarked on one GPU only; multi-GPU runs "
              "(--gpus > 1) are not part of this build (sharding is described in DESIGN.md).",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no GPU available", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)

    if args.suite == "c500":
        rows = c500_suite()
        for row in rows:
            print(json.dumps({"metric": "c500_case_us_per_call", **row}), flush=True)
        score = sum(r["score"] for r in rows) / len(rows)
        ref = sum(r["c500_clean_score"] for r in rows) / len(rows)
        print(json.dumps({
            "metric": "c500_suite_score", "value": round(score, 2), "unit": "points",
            "higher_is_better": True, "n_gpus": 1, "dtype": "bf16",
            "data": "synthetic (the reference's case table and length recipe, arange table)",
            "config": {"workload": "c500_suite", "cases": len(rows)},
            "reference_c500_score": round(ref, 2),
            "sum_us": round(sum(r["us_per_call"] for r in rows), 1),
            "reference_c500_sum_us": sum(C500_CLEAN_US.values()),
            "note": "score_c = round(100 R_c / (R_c + t_c)) with the reference's C500-fitted R_c"}),
            flush=True)
        return 0

    spec = W.get_spec(args.workload)
    inp = W.make_inputs(spec, seed=args.seed, device="cuda")
    r = time_workload(inp, args.steps, args.warmup, args.num_splits)
    cpu = None if args.no_cpu_baseline else cpu_baseline(inp, args.cpu_budget)
    line = result_line(args, spec, r, cpu)
    del inp
    torch.cuda.empty_cache()
    if args.calibrate_copy:
        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    if args.all:
        for name in list(W.NORTH_STAR) + list(W.EXTRA):
            if name == spec.name:
                continue
            extra = W.make_inputs(name, seed=args.seed, device="cuda")
            steps = max(10, min(args.steps, int(2e11 // max(extra.kv_bytes(), 1))))
            rr = time_workload(extra, steps, min(args.warmup, steps), 0)
            a2 = argparse.Namespace(**{**vars(args), "steps": steps,
                                       "warmup": min(args.warmup, steps)})
            print(json.dumps(result_line(a2, extra.spec, rr)), flush=True)
            del extra
            torch.cuda.empty_cache()
        print(json.dumps(time_append(W.get_spec(W.BENCH_DEFAULT), 200, 20, args.seed)),
              flush=True)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
