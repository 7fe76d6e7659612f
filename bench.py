"""Benchmark: fused decode-time token selection on one MI355X.

Workload (the headline configuration): B=64 rows, V=151,936 bf16 logits
~N(0, 3^2), 2,048 Zipf(1.1) history ids per row, presence 0.5 + frequency
0.3 over the whole history, T 1.0, top-p 0.9, min-p 0.05, mlx_lm filter
order (top-k -> top-p -> min-p), one uniform per row.  A step is one
wh_sample call on one batch; 16 distinct input sets (>256 MB) rotate so the
logits come from HBM rather than the 256 MB Infinity Cache.

Prints one JSON line: rows/s (whole job, inputs resident in HBM), the
dominant kernel's roofline (algorithmic bytes / average kernel time measured
with HIP events on the launch stream), and the CPU baseline (the oracle's
float32 replay of the reference op order, timed on this host's cores).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload 2]
    python bench.py --workload 3         # the fused speculative verifier
    python bench.py --copy-calibration   # plain 256 MiB copies, for PMC scaling
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
METRIC = "sampled rows/sec + % of HBM peak, top-k/top-p sampling at B=64, V=151,936"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--sets", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--engine", choices=["auto", "exact"], default="auto",
                    help="sample workloads: 'exact' times the one-workgroup-per-row exact engine (no workspace)")
    ap.add_argument("--lmhead", metavar="M,K,V", default=None,
                    help="time the LM head (wh_lmhead_logits and wh_lmhead_greedy) at this shape instead")
    ap.add_argument("--summarize-profile", metavar="OUT", default=None,
                    help="write profiles/ summaries from a profiling folder (see summarize_profile)")
    return ap.parse_args()


def copy_calibration(steps: int):
    import torch

    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    for _ in range(steps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n, "launches": steps}))


def make_sets(w, nsets, dev):
    """Input set 0 is the seeded workload itself; sets 1.. are fresh draws of
    the same distributions generated on the device."""
    import torch

    from whallm_amd import synth

    sets = []
    for s in range(nsets):
        if s == 0:
            if w.dtype == "bf16":
                x = torch.from_numpy(w.logits_bits.view(np.int16)).to(dev).view(torch.bfloat16)
            else:
                x = torch.from_numpy(w.logits_f32).to(dev)
            h = None if w.history is None else torch.from_numpy(w.history).to(dev)
        else:
            g = torch.Generator(device=dev)
            g.manual_seed(1000 + s)
            base = torch.randn(w.B, w.V, device=dev, generator=g)
            if w.name.startswith("mtp"):
                x = (torch.round(base * 2.0 / 0.125) * 0.125)
            elif w.name.startswith("top-k"):
                x = torch.distributions.StudentT(3.0).sample((w.B, w.V)).to(dev) * 3.0
            else:
                x = base * float(np.std(w.logits_f32[0]))
            x = x.to(torch.bfloat16 if w.dtype == "bf16" else torch.float32).contiguous()
            h = None
            if w.history is not None:
                rng = np.random.default_rng(5000 + s)
                hh = synth.zipf_ids(rng, 1.1, w.history.shape, w.V, rng.permutation(w.V))
                h = torch.from_numpy(hh).to(dev)
        sets.append((x, h))
    return sets


def make_verify_sets(w, nsets, dev):
    """Verify input sets: set 0 is the seeded workload; sets 1.. are fresh
    draws on the device (target ~N(0, 2.5^2), draft = target + N(0, 0.5^2)
    tempered and softmaxed, draft ids drawn from the draft)."""
    import torch

    sets = []
    for s in range(nsets):
        if s == 0:
            tgt = torch.from_numpy(w.target_logits).to(dev)
            q = torch.from_numpy(w.draft_q).to(dev)
            toks = torch.from_numpy(w.draft_tokens).to(dev)
        else:
            g = torch.Generator(device=dev)
            g.manual_seed(2000 + s)
            tgt = torch.randn(w.B, w.n + 1, w.V, device=dev, generator=g) * 2.5
            dl = tgt[:, :w.n] + torch.randn(w.B, w.n, w.V, device=dev, generator=g) * 0.5
            q = torch.softmax(dl / w.temperature, dim=-1)
            toks = torch.multinomial(q.reshape(-1, w.V), 1, generator=g).reshape(w.B, w.n).to(torch.int32)
        sets.append((tgt.contiguous(), q.contiguous(), toks.contiguous()))
    return sets


def bench_verify(args):
    """Workload 3: the fused speculative verifier (wh_verify_fused)."""
    import torch

    from oracle import oracle as o
    from whallm_amd import sampling, synth

    dev = torch.device("cuda:0")
    w = synth.workload3()
    sets = make_verify_sets(w, args.sets, dev)
    u = torch.from_numpy(w.uniforms).to(dev)
    want_a, want_t = o.verify_fused(w.target_logits, w.draft_q, w.draft_tokens, w.uniforms, w.temperature)
    calls = [sampling.VerifyCall(t, q, k, w.temperature, u) for t, q, k in sets]
    a0, t0 = calls[0]()
    parity = {"rows": int(w.B), "contract_bit_exact": bool(np.array_equal(a0.cpu().numpy(), want_a)
                                                          and np.array_equal(t0.cpu().numpy(), want_t)),
              "accepted_mean": float(np.mean(want_a))}
    for i in range(args.warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0w = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        calls[i % len(calls)]()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0w
    avg_s = e0.elapsed_time(e1) / 1e3 / args.steps
    a1, t1 = calls[0]()
    parity["timed_set0_bit_exact"] = bool(np.array_equal(a1.cpu().numpy(), want_a) and np.array_equal(t1.cpu().numpy(), want_t))
    nbytes = w.bytes_per_call()
    achieved = nbytes / avg_s / 1e9
    must = w.must_read_bytes(want_a)
    traffic, traffic_src = measured_traffic(3, w.name)
    res = {
        "metric": "verified rows/sec + % of HBM peak, speculative verify at B=16, n=8, V=129,280",
        "value": w.B * args.steps / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": w.name, "B": w.B, "n": w.n, "V": w.V, "input_sets": len(sets),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "kernel": "wh_verify_fused", "kernel_avg_us": avg_s * 1e6, "algorithmic_bytes": nbytes,
                     "must_read_bytes": must, "achieved_must_read": must / avg_s / 1e9,
                     "traffic_source": traffic_src},
        "parity": parity,
    }
    if not args.no_cpu_baseline:
        try:
            cores = len(os.sched_getaffinity(0))
        except AttributeError:
            cores = os.cpu_count() or 1
        threads = max(1, min(cores, 16))
        rows = 0
        t0c = time.perf_counter()
        while True:
            o.verify_fused(w.target_logits, w.draft_q, w.draft_tokens, w.uniforms, w.temperature, threads=threads)
            rows += w.B
            el = time.perf_counter() - t0c
            if el >= args.cpu_seconds:
                break
        res["cpu_baseline"] = {"value": rows / el, "unit": "rows/s", "cores": threads, "kind": "port",
                               "sample": f"{rows} rows ({rows // w.B} passes over the seeded batch), the oracle's "
                                         f"verify contract, OpenMP over rows, {el:.1f} s; host reports {cores} usable cores"}
    print(json.dumps(res))


PROFILE_NAMES = {
    1: "wh_sample_workload1_b1_v129280_f32",
    2: "wh_sample_workload2_b64_v151936_bf16",
    3: "wh_verify_fused_workload3_b16_n8_v129280_f32",
    4: "wh_sample_workload4_b256_v129280_f32_topk",
    5: "wh_sample_workload5_b128_v151936_bf16_mtp",
}


def traffic_path(workload: int) -> str:
    return os.path.join(ROOT, "profiles", PROFILE_NAMES[workload] + ".traffic.json")


def bench_lmhead(args):
    """The LM head x [M, K] @ W[V, K]^T (bf16, float32 accumulation), alone
    and fused with greedy selection.  A step is one call; 4 weight copies
    rotate (beyond the 256 MB Infinity Cache at these shapes).  Roofline:
    W + x read once and the logits written once, over the HIP-event time per
    call; the fused form's bytes omit the logits.  Checks the fused tokens
    against the argmax of the unfused logits first."""
    import torch

    from whallm_amd import lmhead

    M, K, V = (int(v) for v in args.lmhead.split(","))
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    x = (torch.randn(M, K, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    ws = [(torch.randn(V, K, device=dev, generator=g) * 0.05).to(torch.bfloat16) for _ in range(4)]
    out = torch.empty(M, V, device=dev)
    lg = lmhead.lm_head(x, ws[0], out).clone()
    tok = lmhead.lm_head_greedy(x, ws[0])
    parity = {"greedy_equals_argmax_of_logits": bool(torch.equal(tok.long(), torch.argmax(lg, dim=1)))}
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for i in range(args.warmup):
            fn(ws[i % 4])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(args.steps):
            fn(ws[i % 4])
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / args.steps, time.perf_counter() - t0

    t_log, wall = timed(lambda w: lmhead.lm_head(x, w, out))
    t_gr, _ = timed(lambda w: lmhead.lm_head_greedy(x, w))
    # sampled rows at the reference's defaults (T 0.2, top-p 0.98): the fused
    # call against the product, then the sampler
    from whallm_amd import sampling

    u = torch.rand(M, device=dev, generator=g)
    dflt = dict(temperature=0.2, top_p=0.98)
    t_sf, _ = timed(lambda w: lmhead.lm_head_sample(x, w, uniforms=u, **dflt))
    t_su, _ = timed(lambda w: sampling.sample(lmhead.lm_head(x, w, out), uniforms=u, **dflt))
    ft = lmhead.lm_head_sample(x, ws[0], uniforms=u, **dflt)
    parity["sampled_fused_equals_unfused"] = bool(torch.equal(ft, sampling.sample(lmhead.lm_head(x, ws[0], out),
                                                                                  uniforms=u, **dflt)))
    wbytes, xbytes, obytes = V * K * 2, M * K * 2, M * V * 4
    achieved = (wbytes + xbytes + obytes) / t_log / 1e9
    res = {
        "metric": "LM head rows/sec + % of HBM peak", "value": M * args.steps / wall, "unit": "rows/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16 (fp32 accumulate)",
        "data": "synthetic", "config": {"workload": f"lm_head M={M} K={K} V={V}", "M": M, "K": K, "V": V,
                                         "weight_copies": 4, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": None, "kernel": "lmhead_logits_kernel",
                     "kernel_avg_us": t_log * 1e6, "algorithmic_bytes": wbytes + xbytes + obytes},
        "fused_greedy": {"kernel_avg_us": t_gr * 1e6, "algorithmic_bytes": wbytes + xbytes + M * 4,
                         "achieved": (wbytes + xbytes + M * 4) / t_gr / 1e9},
        "sampled_T0.2_p0.98": {"fused_us": t_sf * 1e6, "lm_head_then_sample_us": t_su * 1e6},
        "parity": parity,
    }
    print(json.dumps(res))


def measured_traffic(workload: int, name: str):
    """HBM bytes per call from the committed rocprofv3 --pmc summary of this
    workload (FETCH_SIZE and WRITE_SIZE runs, each scaled by what the counter
    reads for a 256 MiB copy).  None when there is none, when it is for
    another workload, or when it was measured on other library sources (its
    recorded source digest differs from this tree's)."""
    from whallm_amd.build import source_digest

    path = traffic_path(workload)
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    if t.get("workload") != name:
        return None, None
    if t.get("library_digest") != source_digest():
        return None, f"stale: {os.path.relpath(path, ROOT)} was measured on other library sources"
    return int(t["traffic_bytes_per_call"]), t.get("source")


def summarize_profile(workload: int, out: str, lmhead: str | None = None):
    """Write profiles/<name>.md and the traffic record bench.py reads from one
    profiling folder `out`, holding (each from the command listed in the
    summary): trace/ (--kernel-trace --stats), fetch/ and write/ (--pmc
    FETCH_SIZE / WRITE_SIZE), copy_fetch/ and copy_write/ (the 256 MiB copy
    calibration), bench.json (this bench without a profiler) and trace.json
    (its line under the kernel trace)."""
    import collections
    import csv
    import glob

    from whallm_amd.build import source_digest

    def pmc(d):
        f = glob.glob(os.path.join(out, d, "**", "*counter_collection.csv"), recursive=True)[0]
        agg = collections.defaultdict(list)
        for r in csv.DictReader(open(f)):
            agg[r["Kernel_Name"]].append(float(r["Counter_Value"]))
        return agg

    def last_json(fn):
        return json.loads(open(os.path.join(out, fn)).read().strip().splitlines()[-1])

    cf, cw, bf, bw = pmc("copy_fetch"), pmc("copy_write"), pmc("fetch"), pmc("write")
    copy = [k for k in cf if "copyBuffer" in k][0]
    copy_kib = 256 * 1024
    fscale = copy_kib / (sum(cf[copy]) / len(cf[copy]))
    wscale = copy_kib / (sum(cw[copy]) / len(cw[copy]))
    rows, tot = [], 0.0
    for k in sorted(k for k in bf if "wh::" in k and "greedy" not in k):
        f = sum(bf[k]) / len(bf[k])
        w = sum(bw[k]) / len(bw[k])
        b = (f * fscale + w * wscale) * 1024
        # the LM head's figure is its logits kernel alone: the bench also runs
        # the greedy and sampled entry points, whose kernels read the weights too
        if not lmhead or "lmhead_logits_kernel" in k:
            tot += b
        rows.append((k.split("(")[0].replace("void ", ""), len(bf[k]), f, w, f * fscale * 1024, w * wscale * 1024))
    stats = list(csv.DictReader(open(glob.glob(os.path.join(out, "trace", "**", "*kernel_stats.csv"), recursive=True)[0])))
    bench, tr = last_json("bench.json"), last_json("trace.json")
    alg = bench["roofline"]["algorithmic_bytes"]
    if lmhead:
        M, K, V = lmhead.split(",")
        name = f"wh_lmhead_m{M}_k{K}_v{V}"
        run = f"--lmhead {lmhead}"
        steps, psteps = "--steps 20 --warmup 5", "--steps 4 --warmup 1"
    else:
        name = PROFILE_NAMES[workload]
        run = f"--workload {workload}"
        steps, psteps = "--steps 200 --warmup 20 --no-cpu-baseline", "--steps 32 --warmup 4 --no-cpu-baseline"
    md = [f"# {bench['roofline']['kernel']}, {bench['config']['workload']}\n",
          "Commands (one MI355X, repository root; `cd /tmp && export TMPDIR=/tmp` first for rocprofv3; "
          "OUT is any folder):\n", "```",
          f"rocprofv3 --kernel-trace --stats --output-format csv -d OUT/trace -o t -- python3 bench.py {run} "
          f"{steps} > OUT/trace.json",
          f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o b -- python3 bench.py {run} {psteps}",
          f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o b -- python3 bench.py {run} {psteps}",
          "rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/copy_fetch -o c -- python3 bench.py --copy-calibration --steps 3",
          "rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/copy_write -o c -- python3 bench.py --copy-calibration --steps 3",
          f"python3 bench.py {run}{' ' + steps if lmhead else ''} > OUT/bench.json",
          f"python3 bench.py --summarize-profile OUT {run}", "```\n",
          f"Library source digest: `{source_digest()}`\n",
          "## Kernel trace (--kernel-trace --stats)\n", "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    ksum = 0.0
    for r in stats:
        if "wh::" not in r["Name"]:
            continue
        ksum += float(r["AverageNs"]) / 1000
        md.append(f"| {r['Name'].split('(')[0].replace('void ', '')} | {r['Calls']} | {float(r['AverageNs']) / 1000:.2f} "
                  f"| {float(r['MinNs']) / 1000:.2f} | {float(r['MaxNs']) / 1000:.2f} |")
    if lmhead:
        md.append("\nThe bench calls each entry point in turn (the logits kernel; the greedy kernel and its "
                  "per-row reduction; the sampled entry point: the product with slice maxima, then the wide "
                  "engine's wx_* kernels).")
    md.append(f"\nSum of the kernels' averages: {ksum:.2f} us{' (both entry points)' if lmhead else ' per call'}.  "
              f"The bench without the profiler measured "
              f"{bench['roofline']['kernel_avg_us']:.2f} us per call with HIP events on the launch stream (every kernel "
              f"of the call and the gaps between them); under the kernel trace it measured "
              f"{tr['roofline']['kernel_avg_us']:.2f} us.\n")
    md += ["## HBM traffic (--pmc, one counter per run)\n",
           f"Calibration: a 256 MiB device copy (`__amd_rocclr_copyBuffer`) reads FETCH_SIZE "
           f"{sum(cf[copy]) / len(cf[copy]):.1f} KiB and WRITE_SIZE {sum(cw[copy]) / len(cw[copy]):.1f} KiB per dispatch: "
           f"scale factors {fscale:.4f} (FETCH_SIZE) and {wscale:.4f} (WRITE_SIZE).\n",
           "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | read bytes (scaled) | written bytes (scaled) |",
           "|---|---|---|---|---|---|"]
    for n, c, f, w, fb, wb in rows:
        md.append(f"| {n} | {c} | {f:.1f} | {w:.1f} | {fb:,.0f} | {wb:,.0f} |")
    md.append(f"\nTraffic per call ({'the logits kernel' if lmhead else 'all kernels'}): {tot:,.0f} bytes; "
              f"algorithmic bytes per call {alg:,} (ratio {tot / alg:.3f}).")
    if "must_read_bytes" in bench["roofline"]:
        mr = bench["roofline"]["must_read_bytes"]
        md.append(f"Bytes the call must read (early exit at the first rejection, set 0): {mr:,} (traffic ratio "
                  f"{tot / mr:.3f}).")
    md += ["\n## Bench line (no profiler)\n", "```", json.dumps(bench), "```"]
    with open(os.path.join(ROOT, "profiles", name + ".md"), "w") as f:
        f.write("\n".join(md) + "\n")
    if lmhead:
        print("\n".join(md))
        return
    with open(traffic_path(workload), "w") as f:
        json.dump({"workload": bench["config"]["workload"], "traffic_bytes_per_call": round(tot),
                   "fetch_scale": fscale, "write_scale": wscale, "library_digest": source_digest(),
                   "kernels": {n: {"fetch_kib": f, "write_kib": w} for n, c, f, w, fb, wb in rows},
                   "source": f"profiles/{name}.md"}, f, indent=1)
    print("\n".join(md))


def cpu_baseline(w, seconds: float):
    from oracle import oracle as o
    from whallm_amd import synth

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, 16))
    p = synth.oracle_params(w, o.make_params)
    o.sample_faithful(w.logits_f32[:1], p[:1], w.uniforms[:1], None if w.history is None else w.history[:1],
                      None if w.history_len is None else w.history_len[:1], threads=1)
    rows = 0
    t0 = time.perf_counter()
    while True:
        o.sample_faithful(w.logits_f32, p, w.uniforms, w.history, w.history_len, threads=threads)
        rows += w.B
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": rows / el, "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{rows} rows ({rows // w.B} passes over the {w.B}-row seeded batch) of the same workload, "
                      f"float32 replay of the reference op order (sort-based top-p/min-p, sequential cumsum), "
                      f"OpenMP over rows, {el:.1f} s; host reports {cores} usable cores"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.steps)
        return
    if args.summarize_profile:
        summarize_profile(args.workload, args.summarize_profile, args.lmhead)
        return
    if args.lmhead:
        bench_lmhead(args)
        return
    if args.workload == 3:
        bench_verify(args)
        return
    import torch

    from oracle import oracle as o
    from whallm_amd import _lib, sampling, synth

    dev = torch.device("cuda:0")
    w = synth.SAMPLE_WORKLOADS[args.workload]()
    prm = dict(w.params)
    sets = make_sets(w, args.sets, dev)
    hl = None if w.history_len is None else torch.from_numpy(w.history_len).to(dev)
    kr = None if w.top_k_rows is None else torch.from_numpy(w.top_k_rows).to(dev)
    u = torch.from_numpy(w.uniforms).to(dev)

    # Parity on set 0 before timing.
    tok0 = sampling.sample(sets[0][0], history=sets[0][1], history_len=hl, uniforms=u, top_k_rows=kr,
                           engine=args.engine, **prm)
    p = synth.oracle_params(w, o.make_params)
    want, _ = o.sample(w.logits_f32, p, w.uniforms, w.history, w.history_len)
    faithful, _ = o.sample_faithful(w.logits_f32, p, w.uniforms, w.history, w.history_len)
    got = tok0.cpu().numpy()
    parity = {"rows": int(w.B), "contract_bit_exact": bool(np.array_equal(got, want)),
              "faithful_float32_agreement": float(np.mean(got == faithful))}
    if args.engine == "auto":
        paths = sampling.last_paths(dev, w.B).cpu().numpy()
        parity["rows_exact_fallback"] = int(np.sum((paths == 1) | (paths == 3)))

    # The timed loop calls the C ABI through pre-bound argument structs (one
    # per input set), as a decode loop that refills its buffers would.
    calls = [sampling.SampleCall(x, history=h, history_len=hl, uniforms=u, top_k_rows=kr, engine=args.engine, **prm)
             for x, h in sets]
    for i in range(args.warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        calls[i % len(calls)]()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_s = e0.elapsed_time(e1) / 1e3 / args.steps
    # every call's tokens must match the parity-checked reference of its set
    tok_set0 = calls[0].tokens.cpu().numpy()
    parity["timed_set0_tokens_bit_exact"] = bool(np.array_equal(tok_set0, want))
    nbytes = w.bytes_per_call()
    achieved = nbytes / avg_s / 1e9
    # the committed traffic records are the default (fast / wide) engine's
    traffic, traffic_src = measured_traffic(args.workload, w.name) if args.engine == "auto" else (None, None)
    res = {
        "metric": METRIC,
        "value": w.B * args.steps / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": w.name, "B": w.B, "V": w.V, "logits_dtype": w.dtype,
                   "history": None if w.history is None else int(w.history.shape[1]),
                   "input_sets": len(sets), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "kernel": ("wh_sample (slice_kernel + merge_kernel)" if args.engine == "auto"
                                else "wh_sample exact engine (sample_exact_kernel)"),
                     "kernel_avg_us": avg_s * 1e6, "algorithmic_bytes": nbytes,
                     "traffic_source": traffic_src},
        "parity": parity,
    }
    if args.engine != "auto":
        res["config"]["engine"] = args.engine
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
