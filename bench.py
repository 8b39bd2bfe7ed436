"""RBF forward+backward benchmark on one MI355X (prints one JSON line).

Workload: N = M = 4096, D = 64, fp32, gamma = 0.5,
X, Y ~ N(0,1)/8, upstream dK ~ N(0,1), synthetic data drawn on the host from
seed 0 and copied to HBM before timing.  One step = one forward
(rbf_forward_f32) plus one backward (rbf_backward_f32) through the C-ABI of
librbf_hip.so, on preallocated device buffers.

Timing: W untimed warmup steps, then exactly K steps between two device
synchronisations.  Before every step a 512 MiB buffer is read so the
step reads its operands from HBM, not from L2 or the 256 MiB MALL; HIP events
on the launch stream bracket the forward and the backward calls of each step
(the flush is outside them).  ``ms_per_step`` is the mean of the bracketed
step times; ``value`` is the algorithmic bytes of a step divided by it.

Algorithmic bytes (each input read once, each output written once):
  forward  4*N*M + 4*D*(N+M)          (K written; X, Y read)
  backward 8*N*M + 8*D*(N+M)          (dK, K read; X, Y read; dX, dY written)
Algorithmic flops: forward 2*N*M*D, backward 4*N*M*D (the contractions).

cpu_baseline: the reference's PyTorch CPU path (cases/rbf/reference.py:14-20
forward, autograd backward), restated op for op in oracle/rbf.py, timed on
this host's cores on a bounded row-block sample X[:S] x Y (same distributions).
"""

import argparse
import ctypes
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "nl2cuda-kernel-agent_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "RBF fwd+bwd µs, GB/s and % HBM roofline @N=M=4096,D=64 fp32 vs CPU ref"


def algorithmic(n, m, d):
    fwd_bytes = 4 * n * m + 4 * d * (n + m)
    bwd_bytes = 8 * n * m + 8 * d * (n + m)
    return fwd_bytes, bwd_bytes, 2.0 * n * m * d, 4.0 * n * m * d


def cpu_baseline(size, d, gamma, budget_s):
    """Times the torch CPU reference path on rows X[:S] against all of Y."""
    import torch
    from oracle import rbf as orbf
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    X = torch.randn(size, d, generator=g) / 8
    Y = torch.randn(size, d, generator=g) / 8

    def run(rows):
        Xs = X[:rows].clone()
        G = torch.randn(rows, size, generator=torch.Generator().manual_seed(1))
        t0 = time.perf_counter()
        with torch.no_grad():
            orbf.torch_cpu_forward(Xs, Y, gamma)
        t1 = time.perf_counter()
        Xr = Xs.clone().requires_grad_(True)
        Yr = Y.clone().requires_grad_(True)
        out = orbf.torch_cpu_forward(Xr, Yr, gamma)
        t2 = time.perf_counter()
        out.backward(G)
        t3 = time.perf_counter()
        return (t1 - t0) + (t3 - t2)

    rows = 64
    t = run(rows)  # warmup / calibration
    # choose a sample whose 3 timed repetitions take about budget_s in total
    rows = int(min(size, max(64, rows * (budget_s / 3.0) / max(t, 1e-3))))
    rows = max(64, (rows // 64) * 64)
    times = sorted(run(rows) for _ in range(3))
    med = times[1]
    fb, bb, _, _ = algorithmic(rows, size, d)
    return {
        "value": round((fb + bb) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"torch CPU broadcast reference (oracle/rbf.py torch_cpu_forward + autograd "
                   f"backward) on X[:{rows}] x Y[{size}], D={d}, median of 3 after 1 warmup; "
                   f"{med*1e3:.1f} ms per fwd+bwd; os.cpu_count()={os.cpu_count()}"),
    }


def copy_calibration():
    """A plain copy kernel of known size: reads and writes 256 MiB per launch."""
    import torch
    n = (256 << 20) // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copy calibration: 10 x {n * 4} bytes", flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU work for the cpu_baseline sample (0 = skip)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device-to-device copy 10 times (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()

    if args.copy_calibration:
        return copy_calibration()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the RBF path is single-GPU; sharded, each GPU would take a block of X rows against "
              "all of Y and one all-reduce would sum dY)", file=sys.stderr)
        return 2

    import torch
    from framework import capi
    from framework.bench import flush_caches
    from cases.rbf import op

    n = m = args.size
    d, gamma = 64, 0.5
    lib = op._lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    g = torch.Generator().manual_seed(0)
    X = (torch.randn(n, d, generator=g) / 8).to(dev)
    Y = (torch.randn(m, d, generator=g) / 8).to(dev)
    dK = torch.randn(n, m, generator=torch.Generator().manual_seed(10_000)).to(dev)
    K = torch.empty(n, m, device=dev)
    dX = torch.empty(n, d, device=dev)
    dY = torch.empty(m, d, device=dev)
    ws_bytes = lib.rbf_backward_workspace_bytes(n, m, d)
    ws = torch.empty(max(ws_bytes // 4, 1), device=dev)
    stream = torch.cuda.current_stream(dev)
    s = ctypes.c_void_p(stream.cuda_stream)
    pX, pY, pdK, pK, pdX, pdY, pws = map(capi.ptr, (X, Y, dK, K, dX, dY, ws))

    def fwd():
        st = lib.rbf_forward_f32(pX, pY, pK, n, m, d, gamma, s)
        if st:
            raise RuntimeError(lib.rbf_last_error().decode())

    def bwd():
        st = lib.rbf_backward_f32(pX, pY, pdK, pK, pdX, pdY, n, m, d, gamma, pws, ws_bytes, s)
        if st:
            raise RuntimeError(lib.rbf_last_error().decode())

    for _ in range(args.warmup):
        flush_caches(dev)
        fwd()
        bwd()
    torch.cuda.synchronize()

    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
               torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for e0, e1, e2 in events:
        flush_caches(dev)
        e0.record(stream)
        fwd()
        e1.record(stream)
        bwd()
        e2.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0

    # End-to-end RBFFunction forward + backward through autograd (the case's
    # candidate), after and outside the timed region: the C-ABI calls above
    # plus torch's output allocations and the autograd engine.
    e2e_ms = []
    Xa = X.detach().clone().requires_grad_(True)
    Ya = Y.detach().clone().requires_grad_(True)
    for i in range(min(args.steps, 10) + 2):
        flush_caches(dev)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        op.candidate({"X": Xa, "Y": Ya}, {"gamma": gamma}).backward(dK)
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 2:
            e2e_ms.append(a.elapsed_time(b))
        Xa.grad = Ya.grad = None
    e2e_ms.sort()

    fwd_ms = [a.elapsed_time(b) for a, b, _ in events]
    bwd_ms = [b.elapsed_time(c) for _, b, c in events]
    fwd_avg = sum(fwd_ms) / len(fwd_ms)
    bwd_avg = sum(bwd_ms) / len(bwd_ms)
    step_ms = fwd_avg + bwd_avg
    fb, bb, ff, bf = algorithmic(n, m, d)
    gbs = (fb + bb) / (step_ms * 1e-3) / 1e9

    fwd_tf = ff / (fwd_avg * 1e-3) / 1e12
    bwd_tf = bf / (bwd_avg * 1e-3) / 1e12
    traffic = None  # measured for the 4096 workload only
    tpath = os.path.join(REPO, "profiles", "rbf_bwd_4096_traffic.json")
    if n == 4096 and m == 4096 and d == 64 and os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None
    if args.cpu_budget > 0:
        try:
            cpu = cpu_baseline(n, d, gamma, args.cpu_budget)
        except (MemoryError, RuntimeError) as exc:  # report instead of dying
            cpu = {"value": None, "unit": "GB/s", "cores": None, "kind": "port",
                   "sample": f"skipped: {exc}"}

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (host-seeded N(0,1)/8 inputs, N(0,1) dK; copied to HBM before timing)",
        "config": {"workload": f"rbf fwd+bwd N=M={n} D={d} gamma={gamma}", "N": n, "M": m, "D": d,
                   "gamma": gamma, "flush_between_steps": "512 MiB read (evicts L2 + MALL without dirty lines)"},
        "fwd_us": round(fwd_avg * 1e3, 2),
        "bwd_us": round(bwd_avg * 1e3, 2),
        "fwd_gbs": round(fb / (fwd_avg * 1e-3) / 1e9, 1),
        "bwd_gbs": round(bb / (bwd_avg * 1e-3) / 1e9, 1),
        "pct_hbm_roofline": round(100 * gbs / HBM_PEAK_GBS, 2),
        "e2e_autograd_us": round(e2e_ms[len(e2e_ms) // 2] * 1e3, 2),
        "fwd_tflops": round(fwd_tf, 2),
        "bwd_tflops": round(bwd_tf, 2),
        "pct_fp32_roofline": round(100 * (ff + bf) / (step_ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 2),
        "roofline": {
            "kernel": "rbf_backward_f32 (pair_bwd_d64_3r_kernel<RbfBwdOp> + rbf_bwd_reduce_kernel)",
            "bound": "mfma",
            "achieved": round(bwd_tf, 3),
            "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / FP32_PEAK_TFLOPS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
