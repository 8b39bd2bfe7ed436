"""CPU baselines of the follow-on cases, beside the HIP candidates.

For every follow-on case at its measurement shape (the shapes
framework/roofline.py times), this times the case's reference torch path on
the host CPU, which is the reference's reference.py expression restated in
cases/<case>/reference.py:

  * the forward under no_grad;
  * the backward as out.backward(G), with the graph built outside the timed
    region;
  * 1 warmup, then 3 timed repetitions (median, time.perf_counter) at torch's
    thread count (the box's CPU share; os.cpu_count() is reported beside it).

The GPU side is the case's candidate, the HIP library through autograd, on
the same inputs: the forward, then forward + backward.  Each gets a 512 MiB
read flush before it and is timed with HIP events (median of --iters).
The RBF path's baseline is bench.py's cpu_baseline.

Usage:  python nl2cuda-kernel-agent_amd/framework/cpu_baseline.py
            [--case all|layernorm|l2norm_scale|scan|spmv|cosine_sim|softmax_ce]
Prints one JSON line per case and a closing table.
"""

import argparse
import json
import os
import statistics
import sys
import time

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if PKG not in sys.path:
    sys.path.insert(0, PKG)


def _cases():
    import cases.cosine_sim as cs
    import cases.l2norm_scale as l2
    import cases.layernorm as ln
    import cases.scan as sc
    import cases.softmax_ce as sce
    import cases.spmv as sp
    return {
        "layernorm": ("[8192, 4096]", lambda: ln.make_case(b=ln.config.BASELINE_B,
                                                           d=ln.config.BASELINE_D)),
        "l2norm_scale": ("[16384, 1024]", lambda: l2.make_case(n=16384, d=1024)),
        "scan": ("[64, 65536]", lambda: sc.make_case(b=sc.config.BASELINE_B,
                                                     d=sc.config.BASELINE_D)),
        "spmv": ("Zipf 2^20 x 2^20, nnz 16 M, D = 1", lambda: sp.baseline_case(d=1)),
        "cosine_sim": ("4096 x 4096, D = 64", lambda: cs.make_case(n=4096, m=4096, d=64)),
        "softmax_ce": ("[8192, 1024]", lambda: sce.make_case(b=8192, c=1024)),
    }


def _grad_out(out):
    import torch
    g = torch.Generator().manual_seed(777)
    return torch.randn(out.shape, generator=g, dtype=torch.float32).to(out.dtype)


def cpu_times(case, reps=3):
    """(forward s, backward s) medians of the torch CPU reference path."""
    import torch
    inputs = case.make_inputs(0, torch.float32, "cpu")
    with torch.no_grad():
        out = case.reference_forward(inputs, case.params)
    G = _grad_out(out)

    def fwd():
        with torch.no_grad():
            t0 = time.perf_counter()
            case.reference_forward(inputs, case.params)
            return time.perf_counter() - t0

    def bwd():
        loc = {k: (v.detach().clone().requires_grad_(True) if k in case.grad_inputs else v)
               for k, v in inputs.items()}
        o = case.reference_forward(loc, case.params)
        t0 = time.perf_counter()
        o.backward(G)
        return time.perf_counter() - t0

    fwd()
    bwd()
    return (statistics.median(fwd() for _ in range(reps)),
            statistics.median(bwd() for _ in range(reps)))


def gpu_times(case, candidate, dev, iters):
    """(forward ms, forward + backward ms) medians of the HIP candidate."""
    import torch
    from framework.bench import flush_caches
    inputs = {k: v.to(dev) for k, v in case.make_inputs(0, torch.float32, "cpu").items()}
    with torch.no_grad():
        out = candidate(inputs, case.params)
    G = _grad_out(out.cpu()).to(dev)
    stream = torch.cuda.current_stream(dev)

    def timed(step):
        ts = []
        for i in range(iters + 2):
            flush_caches(dev)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            step()
            b.record(stream)
            torch.cuda.synchronize()
            if i >= 2:
                ts.append(a.elapsed_time(b))
        return statistics.median(ts)

    def fwd():
        with torch.no_grad():
            candidate(inputs, case.params)

    def both():
        loc = {k: (v.detach().clone().requires_grad_(True) if k in case.grad_inputs else v)
               for k, v in inputs.items()}
        candidate(loc, case.params).backward(G)

    return timed(fwd), timed(both)


def main(argv=None):
    import importlib
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--case", default="all")
    ap.add_argument("--iters", type=int, default=10)
    ns = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        print("cpu_baseline: needs the GPU for the candidate side", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    table = _cases()
    names = list(table) if ns.case == "all" else [ns.case]
    rows = []
    for name in names:
        shape, make = table[name]
        case = make()
        candidate = importlib.import_module(f"cases.{name}.op").candidate
        print(f"[cpu_baseline] {name} {shape}", flush=True)
        cf, cb = cpu_times(case)
        gf, gfb = gpu_times(case, candidate, dev, ns.iters)
        rec = {"case": name, "shape": shape, "cpu_fwd_ms": round(cf * 1e3, 3),
               "cpu_bwd_ms": round(cb * 1e3, 3), "cpu_threads": torch.get_num_threads(),
               "os_cpu_count": os.cpu_count(), "kind": "port",
               "cpu_path": f"cases/{name}/reference.py reference_forward (+ autograd backward)",
               "gpu_fwd_ms": round(gf, 4), "gpu_fwd_bwd_ms": round(gfb, 4),
               "speedup_fwd": round(cf * 1e3 / gf, 1),
               "speedup_fwd_bwd": round((cf + cb) * 1e3 / gfb, 1)}
        print(json.dumps(rec), flush=True)
        rows.append(rec)
    print("\n| case | shape | CPU fwd ms | CPU bwd ms | threads | GPU fwd ms | GPU fwd+bwd ms | "
          "speedup fwd | speedup fwd+bwd |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        print(f"| {r['case']} | {r['shape']} | {r['cpu_fwd_ms']:.2f} | {r['cpu_bwd_ms']:.2f} | "
              f"{r['cpu_threads']} | {r['gpu_fwd_ms']:.4f} | {r['gpu_fwd_bwd_ms']:.4f} | "
              f"{r['speedup_fwd']:.0f}x | {r['speedup_fwd_bwd']:.0f}x |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
