"""rocprofv3-driven profiling of a case or of any command (MI355X).

The reference's skill/scripts/profile_case.py:27-83 runs a case's candidate
under torch.profiler and prints the per-kernel time table.  This tool keeps
that use (``run-case`` executes the same forward / forward+backward steps)
and takes the numbers from rocprofv3 instead, as text summaries fit to
commit next to the code:

  stats    rocprofv3 --kernel-trace --stats over a command; writes
           <out>/<name>.md with the command line and the per-kernel table
           (calls, average / min / max duration, share of GPU time).
  traffic  two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE) over a
           command and the same two over a plain device copy of known size
           (``bench.py --copy-calibration``); the copy's counter readings
           give bytes-per-count factors, which turn the selected kernels'
           per-dispatch readings into HBM bytes per launch.  Writes
           <out>/<name>_traffic.json and .md.
  counters one rocprofv3 --pmc pass per --pmc group of any counters; the
           median per dispatch of each, per selected kernel.  Writes
           <out>/<name>_counters.json and .md.
  mfma     one rocprofv3 --pmc pass of the derived counters MfmaUtil (the
           MFMA pipes' busy cycles over all SIMDs and the GPU-active
           cycles) and MfmaFlopsF32 (fp32 MFMA flops) for the selected
           kernels, per dispatch.  Writes <out>/<name>_mfma.json and .md.
  gaps     rocprofv3 --kernel-trace over a command; for a repeated sequence
           of dispatches (kernel-name substrings, --sequence "a;b;c") the
           median duration of each and the gap between consecutive ones
           (start minus the previous end).  Writes <out>/<name>.md.
  run-case the profiled program for a case: warmup, then --iters steps of
           the case's candidate (forward only or forward+backward).

Usage (from the repository root; rocprofv3 must be on PATH):
  python nl2cuda-kernel-agent_amd/framework/profile.py stats --name rbf_4096 \\
      -- python3 bench.py --steps 20 --warmup 5 --cpu-budget 0
  python nl2cuda-kernel-agent_amd/framework/profile.py traffic --name rbf_bwd_4096 \\
      --kernels rbf_bwd_d64_kernel,rbf_bwd_reduce_kernel -- python3 bench.py ...
  python nl2cuda-kernel-agent_amd/framework/profile.py stats --name rbf_case \\
      --case rbf

rocprofv3 is always started as a child process of this (GPU-free) process,
with the profiled program directly after ``--``; each pass has its own time
limit.  PMC passes carry no trace domains.
"""

import argparse
import csv
import glob
import json
import os
import shlex
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO = os.path.dirname(PKG)
COPY_BYTES = 256 << 20  # bench.py --copy-calibration copies this many bytes per launch
_INVOCATION = []  # this tool's own command line, recorded in the summaries


def _rocprof(args, outdir, tag, cmd, limit):
    """Runs one rocprofv3 pass; returns the output directory."""
    d = os.path.join(outdir, tag)
    os.makedirs(d, exist_ok=True)
    full = (["timeout", "-s", "KILL", str(limit), "rocprofv3"] + args +
            ["--output-format", "csv", "-d", d, "-o", "run", "--"] + cmd)
    print(f"[profile] {tag}: {' '.join(shlex.quote(c) for c in full)}", flush=True)
    t0 = time.time()
    with open(os.path.join(d, "rocprof.log"), "w") as log:
        rc = subprocess.call(full, stdout=log, stderr=subprocess.STDOUT, env=dict(os.environ))
    print(f"[profile] {tag}: rc={rc} in {time.time() - t0:.1f}s", flush=True)
    if rc not in (0,) and not glob.glob(os.path.join(d, "**", "*.csv"), recursive=True):
        raise RuntimeError(f"rocprofv3 pass {tag} failed with rc={rc}; see {d}/rocprof.log")
    return d


def _find(d, suffix):
    hits = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return hits[0]


def _short(name, width=90):
    s = name
    for cut in ("(float const", "(float*", "(int const", "(long const", "(unsigned"):
        k = s.find(cut)
        if k > 0:
            s = s[:k]
    s = s.replace("(anonymous namespace)::", "")
    return s if len(s) <= width else s[:width - 3] + "..."


def stats_table(d):
    with open(_find(d, "kernel_stats.csv")) as f:
        rows = list(csv.DictReader(f))
    out = []
    for r in rows:
        out.append({
            "kernel": _short(r["Name"]),
            "calls": int(r["Calls"]),
            "avg_us": float(r["AverageNs"]) / 1e3,
            "min_us": float(r["MinNs"]) / 1e3,
            "max_us": float(r["MaxNs"]) / 1e3,
            "pct": float(r.get("Percentage", "nan")),
        })
    return out


def cmd_stats(ns, cmd):
    d = _rocprof(["--kernel-trace", "--stats"], ns.raw, f"{ns.name}_stats", cmd, ns.limit)
    table = stats_table(d)
    lines = [f"# rocprofv3 kernel statistics: {ns.name}", "",
             "Command (repository root, `cd` into it first; TMPDIR=/tmp):", "",
             "```", " ".join(shlex.quote(c) for c in _INVOCATION), "```", "",
             "which ran:", "", "```",
             "rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- " +
             " ".join(shlex.quote(c) for c in cmd), "```", "",
             "| kernel | calls | avg µs | min µs | max µs | % GPU time |",
             "|---|---:|---:|---:|---:|---:|"]
    for r in table:
        lines.append(f"| `{r['kernel']}` | {r['calls']} | {r['avg_us']:.2f} | {r['min_us']:.2f} | "
                     f"{r['max_us']:.2f} | {r['pct']:.1f} |")
    os.makedirs(ns.out, exist_ok=True)
    path = os.path.join(ns.out, f"{ns.name}.md")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines[-len(table) - 2:]))
    print(f"[profile] wrote {path}")
    return 0


def trace_rows(d):
    """(start ns, end ns, kernel name) of every dispatch, in start order."""
    with open(_find(d, "kernel_trace.csv")) as f:
        rows = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                for r in csv.DictReader(f)]
    return sorted(rows)


def sequence_gaps(rows, pattern):
    """Every run of consecutive dispatches whose names contain pattern[0],
    pattern[1], ... in order.  Returns {"dur <k>": [us], "gap <k-1> -> <k>":
    [us]} over the runs: each element's duration and the idle time between
    the end of one element and the start of the next (negative when the next
    dispatch's start was stamped before the previous one ended)."""
    out = {}
    for i in range(len(rows) - len(pattern) + 1):
        run = rows[i:i + len(pattern)]
        if not all(p in r[2] for p, r in zip(pattern, run)):
            continue
        for k, (p, r) in enumerate(zip(pattern, run)):
            out.setdefault(f"dur {p}", []).append((r[1] - r[0]) / 1e3)
            if k:
                out.setdefault(f"gap {pattern[k - 1]} -> {p}", []).append(
                    (r[0] - run[k - 1][1]) / 1e3)
    return out


def cmd_gaps(ns, cmd):
    """Kernel durations and the gaps between them for a repeated sequence of
    dispatches (one rocprofv3 --kernel-trace pass)."""
    d = _rocprof(["--kernel-trace", "--stats"], ns.raw, f"{ns.name}_trace", cmd, ns.limit)
    rows = trace_rows(d)
    lines = [f"# rocprofv3 kernel trace, durations and gaps: {ns.name}", "",
             "Command (repository root, `cd` into it first; TMPDIR=/tmp):", "",
             "```", " ".join(shlex.quote(c) for c in _INVOCATION), "```", "",
             "which ran:", "", "```",
             "rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- " +
             " ".join(shlex.quote(c) for c in cmd), "```", "",
             "A gap is the start of a dispatch minus the end of the one before it, from the "
             "trace's own timestamps."]
    for seq in ns.sequence.split("|"):
        pattern = [p for p in seq.split(";") if p]
        res = sequence_gaps(rows, pattern)
        if not res:
            raise RuntimeError(f"no run of {pattern} in the trace")
        n = len(next(iter(res.values())))
        lines += ["", f"Sequence (kernel-name substrings, in dispatch order): "
                      f"`{' ; '.join(pattern)}`, {n} occurrences.", "",
                  "| interval | median µs | min µs | max µs |", "|---|---:|---:|---:|"]
        for k, v in res.items():
            v = sorted(v)
            lines.append(f"| {k} | {v[len(v) // 2]:.2f} | {v[0]:.2f} | {v[-1]:.2f} |")
    os.makedirs(ns.out, exist_ok=True)
    path = os.path.join(ns.out, f"{ns.name}.md")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines[14:]))
    print(f"[profile] wrote {path}")
    return 0


def counter_rows(d):
    """Per-dispatch counter readings: list of (dispatch, kernel, counter, value)."""
    path = _find(d, "counter_collection.csv")
    with open(path) as f:
        rows = list(csv.DictReader(f))
    out = []
    for r in rows:
        name = r.get("Kernel_Name") or r.get("Kernel-Name") or ""
        disp = r.get("Dispatch_Id") or r.get("Dispatch-Id") or r.get("Correlation_Id")
        cname = r.get("Counter_Name") or r.get("Counter-Name")
        val = r.get("Counter_Value") or r.get("Counter-Value")
        out.append((int(disp), name, cname, float(val)))
    return out


def per_dispatch(rows, counter, match):
    """Sum of `counter` per dispatch whose kernel name contains any of `match`."""
    acc = {}
    names = {}
    for disp, name, cname, val in rows:
        if cname != counter or not any(m in name for m in match):
            continue
        acc[disp] = acc.get(disp, 0.0) + val
        names[disp] = name
    return acc, names


def _median(values):
    v = sorted(values)
    return v[len(v) // 2]


def calibrated_counter(krows, crows, counter, kernels, copy_bytes=COPY_BYTES):
    """One PMC counter turned into bytes per launch.

    `crows` are the readings of a plain device copy that moves `copy_bytes`
    per launch (reads for FETCH_SIZE, writes for WRITE_SIZE): its median
    reading per dispatch gives the bytes one counter unit stands for, and
    each kernel's median per-dispatch reading in `krows` times that factor is
    its bytes per launch.  Readings of one dispatch (one row per shader
    engine / XCD instance) are summed first."""
    copy_vals, _ = per_dispatch(crows, counter, ["copy"])
    if not copy_vals:
        raise RuntimeError(f"no copy-kernel dispatch with {counter} readings")
    copy_med = _median(copy_vals.values())
    factor = copy_bytes / copy_med  # bytes per counter unit
    per_kernel = {}
    for k in kernels:
        vals, _ = per_dispatch(krows, counter, [k])
        if not vals:
            raise RuntimeError(f"kernel {k} has no {counter} readings")
        med = _median(vals.values())
        per_kernel[k] = {"dispatches": len(vals), "median_counter": med,
                         "bytes_per_launch": med * factor}
    return {"copy_counter_median": copy_med, "copy_dispatches": len(copy_vals),
            "bytes_per_unit": factor, "kernels": per_kernel}


def kernel_list(spec):
    """Kernel-name substrings: ';'-separated when the spec has a ';' (template
    names carry commas), else ','-separated."""
    return [k for k in spec.split(";" if ";" in spec else ",") if k]


def cmd_traffic(ns, cmd):
    kernels = kernel_list(ns.kernels)
    copy_cmd = [sys.executable, os.path.join(REPO, "bench.py"), "--copy-calibration"]
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        dk = _rocprof(["--pmc", counter], ns.raw, f"{ns.name}_{counter}", cmd, ns.limit)
        dc = _rocprof(["--pmc", counter], ns.raw, f"copy_{counter}", copy_cmd, ns.limit)
        res[counter] = calibrated_counter(counter_rows(dk), counter_rows(dc), counter, kernels)
    fetch = sum(x["bytes_per_launch"] for x in res["FETCH_SIZE"]["kernels"].values())
    write = sum(x["bytes_per_launch"] for x in res["WRITE_SIZE"]["kernels"].values())
    doc = {
        "name": ns.name,
        "kernels": kernels,
        "command": " ".join(shlex.quote(c) for c in _INVOCATION),
        "profiled": " ".join(shlex.quote(c) for c in cmd),
        "calibration": f"bench.py --copy-calibration: device copy of {COPY_BYTES} bytes "
                       f"(reads {COPY_BYTES} B, writes {COPY_BYTES} B per launch)",
        "counters": res,
        "hbm_fetch_bytes_per_launch": round(fetch),
        "hbm_write_bytes_per_launch": round(write),
        "hbm_bytes_per_launch": round(fetch + write),
    }
    if ns.algorithmic_bytes:
        doc["algorithmic_bytes_per_launch"] = ns.algorithmic_bytes
        doc["traffic_over_algorithmic"] = round((fetch + write) / ns.algorithmic_bytes, 3)
    os.makedirs(ns.out, exist_ok=True)
    jpath = os.path.join(ns.out, f"{ns.name}_traffic.json")
    with open(jpath, "w") as f:
        json.dump(doc, f, indent=1)
    lines = [f"# HBM traffic per launch: {ns.name}", "", "Command:", "", "```", doc["command"], "```",
             "", f"Calibration: {doc['calibration']}.", "",
             "| counter | copy reading (median) | bytes per unit | kernel | reading (median) | bytes per launch |",
             "|---|---:|---:|---|---:|---:|"]
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        r = res[counter]
        for k, x in r["kernels"].items():
            lines.append(f"| {counter} | {r['copy_counter_median']:.0f} | {r['bytes_per_unit']:.2f} | "
                         f"`{k}` | {x['median_counter']:.0f} | {x['bytes_per_launch']:.0f} |")
    lines += ["", f"Total HBM bytes per launch (all listed kernels): fetch "
              f"{doc['hbm_fetch_bytes_per_launch']:,} + write {doc['hbm_write_bytes_per_launch']:,} = "
              f"{doc['hbm_bytes_per_launch']:,}"]
    if ns.algorithmic_bytes:
        lines += ["", f"Algorithmic bytes per launch: {ns.algorithmic_bytes:,}; measured / "
                  f"algorithmic = {doc['traffic_over_algorithmic']:.3f}"]
    with open(os.path.join(ns.out, f"{ns.name}_traffic.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


MFMA_COUNTERS = ("MfmaUtil", "MfmaFlopsF32")


def mfma_summary(rows, kernels):
    """Median, min and max per dispatch of each MFMA counter, per kernel."""
    per_kernel = {}
    for k in kernels:
        entry = {}
        for counter in MFMA_COUNTERS:
            vals, _ = per_dispatch(rows, counter, [k])
            if not vals:
                raise RuntimeError(f"kernel {k} has no {counter} readings")
            v = sorted(vals.values())
            entry[counter] = {"dispatches": len(v), "median": v[len(v) // 2],
                              "min": v[0], "max": v[-1]}
        per_kernel[k] = entry
    return per_kernel


def cmd_mfma(ns, cmd):
    kernels = kernel_list(ns.kernels)
    d = _rocprof(["--pmc"] + list(MFMA_COUNTERS), ns.raw, f"{ns.name}_mfma", cmd, ns.limit)
    per_kernel = mfma_summary(counter_rows(d), kernels)
    doc = {"name": ns.name, "kernels": kernels,
           "command": " ".join(shlex.quote(c) for c in _INVOCATION),
           "profiled": " ".join(shlex.quote(c) for c in cmd),
           "counters": {"MfmaUtil": "percent: sum of SQ_VALU_MFMA_BUSY_CYCLES over SIMDs / "
                                    "(GRBM_GUI_ACTIVE x SIMD count) x 100",
                        "MfmaFlopsF32": "SQ_INSTS_VALU_MFMA_MOPS_F32 x 512 (fp32 MFMA flops)"},
           "per_kernel": per_kernel}
    os.makedirs(ns.out, exist_ok=True)
    with open(os.path.join(ns.out, f"{ns.name}_mfma.json"), "w") as f:
        json.dump(doc, f, indent=1)
    lines = [f"# MFMA utilisation per dispatch: {ns.name}", "", "Command:", "", "```", doc["command"],
             "```", "", "which ran one pass of:", "", "```",
             f"rocprofv3 --pmc {' '.join(MFMA_COUNTERS)} --output-format csv -d <dir> -o run -- "
             + doc["profiled"], "```", "",
             "MfmaUtil = " + doc["counters"]["MfmaUtil"] + ".  MfmaFlopsF32 = " +
             doc["counters"]["MfmaFlopsF32"] + ".", "",
             "| kernel | dispatches | MfmaUtil % (median, min-max) | MfmaFlopsF32 per dispatch (median) |",
             "|---|---:|---:|---:|"]
    for k, e in per_kernel.items():
        u, fl = e["MfmaUtil"], e["MfmaFlopsF32"]
        lines.append(f"| `{k}` | {u['dispatches']} | {u['median']:.1f} ({u['min']:.1f}-{u['max']:.1f}) | "
                     f"{fl['median']:,.0f} |")
    with open(os.path.join(ns.out, f"{ns.name}_mfma.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def counter_summary(rows, kernels, counters):
    """Median per dispatch of each counter, per kernel: {kernel: {counter:
    {"dispatches", "median"}}} (counters with no reading are left out)."""
    out = {}
    for k in kernels:
        entry = {}
        for counter in counters:
            vals, _ = per_dispatch(rows, counter, [k])
            if vals:
                entry[counter] = {"dispatches": len(vals), "median": _median(vals.values())}
        out[k] = entry
    return out


def cmd_counters(ns, cmd):
    """One rocprofv3 --pmc pass per --pmc group (each within the per-block
    limits of one pass), then the per-kernel medians per dispatch."""
    kernels = kernel_list(ns.kernels)
    table = {k: {} for k in kernels}
    passes = []
    for i, group in enumerate(ns.pmc):
        counters = group.split()
        d = _rocprof(["--pmc"] + counters, ns.raw, f"{ns.name}_pmc{i}", cmd, ns.limit)
        summ = counter_summary(counter_rows(d), kernels, counters)
        for k in kernels:
            table[k].update(summ[k])
        passes.append(" ".join(counters))
    doc = {"name": ns.name, "kernels": kernels,
           "command": " ".join(shlex.quote(c) for c in _INVOCATION),
           "profiled": " ".join(shlex.quote(c) for c in cmd), "passes": passes,
           "per_kernel": table}
    os.makedirs(ns.out, exist_ok=True)
    with open(os.path.join(ns.out, f"{ns.name}_counters.json"), "w") as f:
        json.dump(doc, f, indent=1)
    lines = [f"# PMC counters per dispatch (median): {ns.name}", "", "Command:", "", "```",
             doc["command"], "```", "", "One rocprofv3 pass per group:", ""]
    lines += [f"* `rocprofv3 --pmc {p} -- {doc['profiled']}`" for p in passes]
    for k in kernels:
        lines += ["", f"## `{k}`", "", "| counter | dispatches | median per dispatch |",
                  "|---|---:|---:|"]
        for c, v in table[k].items():
            lines.append(f"| {c} | {v['dispatches']} | {v['median']:,.1f} |")
    with open(os.path.join(ns.out, f"{ns.name}_counters.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def cmd_run_case(ns):
    """The profiled program: the case's candidate, like profile_case.py:48-78."""
    sys.path.insert(0, PKG)
    import importlib
    import torch
    from framework.protocol import dtype_of
    case = importlib.import_module(f"cases.{ns.case}").CASE
    mod, fn = (ns.impl or f"cases.{ns.case}.op:candidate").split(":")
    impl = getattr(importlib.import_module(mod), fn)
    dtype = dtype_of(case.dtype)
    inputs = {k: v.to("cuda") for k, v in
              case.make_inputs(0, dtype, "cpu", requires_grad=False).items()}
    with torch.no_grad():
        out = impl(inputs, case.params)
    G = torch.randn(out.shape, generator=torch.Generator().manual_seed(777)).to(out.dtype).cuda()

    def fwd_step():
        with torch.no_grad():
            impl(inputs, case.params)

    def full_step():
        loc = {k: (v.detach().clone().requires_grad_(True) if k in case.grad_inputs else v)
               for k, v in inputs.items()}
        impl(loc, case.params).backward(G)

    step = fwd_step if ns.mode == "forward" or not case.grad_inputs else full_step
    for _ in range(10):
        step()
    torch.cuda.synchronize()
    for _ in range(ns.iters):
        step()
    torch.cuda.synchronize()
    print(f"[run-case] case={ns.case} mode={ns.mode} iters={ns.iters} done", flush=True)
    return 0


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    _INVOCATION[:] = ["python", os.path.relpath(os.path.abspath(__file__), os.getcwd())] + argv
    cmd = []
    if "--" in argv:
        k = argv.index("--")
        argv, cmd = argv[:k], argv[k + 1:]
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="what", required=True)
    for name in ("stats", "traffic", "mfma", "counters", "gaps"):
        p = sub.add_parser(name)
        p.add_argument("--name", required=True)
        p.add_argument("--out", default=os.path.join(REPO, "profiles"))
        p.add_argument("--raw", default=os.path.join(REPO, "gpurun_out", "profile_raw"))
        p.add_argument("--limit", type=int, default=240, help="seconds per rocprofv3 pass")
        p.add_argument("--case", default=None, help="profile run-case for this case instead of a command")
        p.add_argument("--mode", choices=["forward", "both"], default="both")
        p.add_argument("--iters", type=int, default=50)
        if name == "counters":
            p.add_argument("--pmc", action="append", required=True,
                           help="space-separated counters of one pass (repeat for more passes)")
        if name in ("traffic", "mfma", "counters"):
            p.add_argument("--kernels", required=True,
                           help="kernel-name substrings, ','-separated (';' when names hold commas)")
        if name == "gaps":
            p.add_argument("--sequence", required=True,
                           help="kernel-name substrings of a repeated sequence, ';'-separated; "
                                "several sequences '|'-separated")
        if name == "traffic":
            p.add_argument("--algorithmic-bytes", type=int, default=0,
                           help="algorithmic bytes per launch of the listed kernels (for the ratio)")
    p = sub.add_parser("run-case")
    p.add_argument("--case", required=True)
    p.add_argument("--impl", default=None)
    p.add_argument("--mode", choices=["forward", "both"], default="both")
    p.add_argument("--iters", type=int, default=50)
    ns = ap.parse_args(argv)
    if ns.what == "run-case":
        return cmd_run_case(ns)
    if ns.case:
        cmd = [sys.executable, os.path.abspath(__file__), "run-case", "--case", ns.case,
               "--mode", ns.mode, "--iters", str(ns.iters)]
    if not cmd:
        ap.error("give a command after -- or --case")
    return {"stats": cmd_stats, "traffic": cmd_traffic, "mfma": cmd_mfma,
            "counters": cmd_counters, "gaps": cmd_gaps}[ns.what](ns, cmd)


if __name__ == "__main__":
    sys.exit(main())
