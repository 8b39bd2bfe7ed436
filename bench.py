"""RBF forward+backward benchmark on one MI355X, with every BASELINE config
beside it (prints one JSON line).

Headline workload: N = M = 4096, D = 64, fp32,
gamma = 0.5, X, Y ~ N(0,1)/8, upstream dK ~ N(0,1), synthetic data drawn on
the host from seed 0 and copied to HBM before timing.  One step = one
forward (rbf_forward_f32) plus one backward (rbf_backward_f32) through the
C-ABI of librbf_hip.so, on preallocated device buffers.

Timing: W untimed warmup steps, then exactly K steps between two device
synchronisations.  Before every step a 512 MiB buffer is read so the step
reads its operands from HBM, not from L2 or the 256 MiB MALL; HIP events on
the launch stream bracket the forward and the backward call of each step
(the flush is outside them).  ``ms_per_step`` is the geometric mean of the
bracketed step times (the reference protocol's mean, framework/bench.py);
the K steps are split into three repeats whose geometric means give ``cv``.
``value`` is the algorithmic bytes of a step divided by ``ms_per_step``.

Algorithmic work (each input read once, each output written once):
  forward  4*N*M + 4*D*(N+M) bytes, 2*N*M*D flops (K written; X, Y read)
  backward 8*N*M + 8*D*(N+M) bytes, 4*N*M*D flops (dK, K, X, Y read; dX, dY
           written)

``configs`` carries one entry per call of every BASELINE config, each
timed the same way (flush, HIP events, geometric mean of three repeats):
RBF at 2048, 4096 and 8192 (fwd, bwd; five seeds each, outputs of every
seed checked), LayerNorm [8192, 4096] (fwd, bwd), scan [64, 65536] (fp32
fwd, bwd; int32 -> int64 fwd, bit-exact), CSR SpMV on the Zipf 2^20 matrix
(fwd; bwd dX; bwd dvals + dX; and the autograd pair when vals needs a
gradient: fwd keeping X[col], bwd dvals + dX from it), and the reference's
default SpMM (M = K = 4096, D = 64; fwd; bwd dvals + dX).  Each entry gives
event us, GB/s, the fraction of its binding roof (fp32 MFMA for RBF, HBM
otherwise), and max_abs / max_rel per output against the float64 oracle,
plus the time of the reference's PyTorch CPU path for that call on this
host.  Entries with a committed rocprofv3 traffic summary (profiles/
*_traffic.json: FETCH_SIZE and WRITE_SIZE scaled by a plain copy's
readings) also carry ``traffic``: measured HBM bytes per launch, their
ratio to the algorithmic bytes, and the source file.

CPU leg (the only code here that imports oracle/): ``cpu_baseline`` times the
reference's PyTorch CPU path (cases/rbf/reference.py:14-20 forward, autograd
backward, restated op for op in oracle/rbf.py) on this host's cores on a
bounded row-block sample X[:S] x Y; the ``cpu_*`` functions compute the
float64 reference outputs the GPU outputs are compared with (``parity`` for
the headline, ``outputs`` inside each config entry) and time the CPU
reference path per config.
"""

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "nl2cuda-kernel-agent_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
MEASURED_FP32_MFMA_TFLOPS = 137.0
ATOL = RTOL = 1e-3
METRIC = "RBF fwd+bwd µs, GB/s and % HBM roofline @N=M=4096,D=64 fp32 vs CPU ref"
SEEDS = (0, 1, 2, 3, 4)
TRAFFIC_SOURCE = os.path.join("profiles", "rbf_bwd_4096_traffic.json")


def rbf_work(n, m, d):
    """(fwd bytes, bwd bytes, fwd flops, bwd flops) of one call each."""
    return (4 * n * m + 4 * d * (n + m), 8 * n * m + 8 * d * (n + m),
            2.0 * n * m * d, 4.0 * n * m * d)


def geomean(xs):
    return math.exp(sum(math.log(max(x, 1e-12)) for x in xs) / len(xs))


def repeat_stats(samples, repeats=3):
    """(geometric mean, CV of the geometric means of `repeats` equal chunks)."""
    k = max(1, len(samples) // repeats)
    chunks = [samples[i * k:(i + 1) * k] for i in range(repeats) if samples[i * k:(i + 1) * k]]
    gms = [geomean(c) for c in chunks]
    cv = statistics.pstdev(gms) / statistics.mean(gms) if len(gms) > 1 else 0.0
    return geomean(samples), cv


def cpu_info():
    """(CPU description, CPUs this process may run on).  The description is
    /proc/cpuinfo's model name with its family / model / stepping numbers
    (a virtualised host may report only "AMD EPYC" as the name) and the
    machine's logical CPU count."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                k, _, v = line.partition(":")
                fields.setdefault(k.strip(), v.strip())
    except OSError:
        pass
    model = fields.get("model name", "unknown")
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    if ids:
        model += " (" + ", ".join(ids) + ")"
    model += f", {os.cpu_count()} logical CPUs"
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count()
    return model, share


# --------------------------------------------------------------- GPU side
class Timer:
    """HIP events on the launch stream around each call, a 512 MiB read flush
    before each call (outside the events)."""

    def __init__(self, dev):
        import torch
        from framework.bench import flush_caches
        self.torch, self.dev, self.flush = torch, dev, flush_caches
        self.stream = torch.cuda.current_stream(dev)

    def us(self, fn, iters, warmup):
        torch = self.torch
        for _ in range(warmup):
            self.flush(self.dev)
            fn()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        for a, b in ev:
            self.flush(self.dev)
            a.record(self.stream)
            fn()
            b.record(self.stream)
        torch.cuda.synchronize()
        return [a.elapsed_time(b) * 1e3 for a, b in ev]


def _ok(lib, err):
    def check(st):
        if st:
            raise RuntimeError(getattr(lib, err)().decode())
    return check


class RbfGpu:
    """Device buffers and C-ABI calls of one RBF shape."""

    def __init__(self, n, d=64, gamma=0.5):
        import torch
        from framework import capi
        from cases.rbf import op
        self.torch, self.capi = torch, capi
        self.lib = op._lib()
        self.n = self.m = n
        self.d, self.gamma = d, gamma
        dev = torch.device("cuda:0")
        self.X = torch.empty(n, d, device=dev)
        self.Y = torch.empty(n, d, device=dev)
        self.dK = torch.empty(n, n, device=dev)
        self.K = torch.empty(n, n, device=dev)
        self.dX = torch.empty(n, d, device=dev)
        self.dY = torch.empty(n, d, device=dev)
        self.ws_bytes = self.lib.rbf_backward_workspace_bytes(n, n, d)
        self.ws = torch.empty(max(self.ws_bytes // 4, 1), device=dev)
        self.s = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        self.p = {k: capi.ptr(getattr(self, k)) for k in ("X", "Y", "dK", "K", "dX", "dY", "ws")}
        self.check = _ok(self.lib, "rbf_last_error")

    def load(self, seed):
        """Host-seeded inputs: X then Y ~ N(0,1)/8 from seed, dK ~ N(0,1) from seed + 10000."""
        torch = self.torch
        g = torch.Generator().manual_seed(seed)
        X = torch.randn(self.n, self.d, generator=g) / 8
        Y = torch.randn(self.m, self.d, generator=g) / 8
        dK = torch.randn(self.n, self.m, generator=torch.Generator().manual_seed(seed + 10_000))
        self.X.copy_(X)
        self.Y.copy_(Y)
        self.dK.copy_(dK)
        return X, Y, dK

    def fwd(self):
        p = self.p
        self.check(self.lib.rbf_forward_f32(p["X"], p["Y"], p["K"], self.n, self.m, self.d,
                                            self.gamma, self.s))

    def bwd(self):
        p = self.p
        self.check(self.lib.rbf_backward_f32(p["X"], p["Y"], p["dK"], p["K"], p["dX"], p["dY"],
                                             self.n, self.m, self.d, self.gamma, p["ws"],
                                             self.ws_bytes, self.s))

    def outputs(self):
        self.torch.cuda.synchronize()
        return {"K": self.K.cpu().numpy(), "dX": self.dX.cpu().numpy(),
                "dY": self.dY.cpu().numpy()}


# Per-config HBM traffic from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
# summaries (profile.py traffic, scaled by a plain copy's readings), keyed by
# (config label prefix, call).
TRAFFIC_PROFILES = {
    ("rbf N=M=4096", "forward"): "rbf_fwd_4096",
    ("rbf N=M=4096", "backward"): "rbf_bwd_4096",
    ("layernorm", "forward"): "layernorm_fwd_8192x4096",
    ("layernorm", "backward"): "layernorm_bwd_8192x4096",
    ("scan", "forward_f32"): "scan_fwd_f32_64x65536",
    ("scan", "backward_f32"): "scan_bwd_f32_64x65536",
    ("scan", "forward_i32_i64"): "scan_fwd_i32_i64_64x65536",
    ("spmv zipf", "forward"): "spmv_fwd_zipf_2p20",
    ("spmv zipf", "backward dX"): "spmv_bwd_dx_zipf_2p20",
}


def profiled_traffic(config, call, nbytes):
    """{hbm_bytes, over_algorithmic, source} for a config entry that has a
    committed traffic profile, else None."""
    for (prefix, c), name in TRAFFIC_PROFILES.items():
        if config.startswith(prefix) and call == c:
            path = os.path.join("profiles", f"{name}_traffic.json")
            try:
                with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), path)) as f:
                    hbm = json.load(f).get("hbm_bytes_per_launch")
            except (OSError, ValueError):
                return None
            if not hbm:
                return None
            return {"hbm_bytes": int(hbm), "over_algorithmic": round(hbm / nbytes, 3),
                    "source": path}
    return None


def _entry(config, call, us_samples, nbytes, flops=None, bound="hbm", extra=None):
    us, cv = repeat_stats(us_samples)
    gbs = nbytes / (us * 1e-6) / 1e9
    e = {"config": config, "call": call, "us": round(us, 2), "cv": round(cv, 4),
         "iters": len(us_samples), "bytes": nbytes, "gbs": round(gbs, 1),
         "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 2)}
    if flops:
        tf = flops / (us * 1e-6) / 1e12
        e.update(flops=int(flops), tflops=round(tf, 2),
                 pct_fp32=round(100 * tf / FP32_PEAK_TFLOPS, 2))
    frac = (e["tflops"] / FP32_PEAK_TFLOPS) if bound == "mfma" else gbs / HBM_PEAK_GBS
    e["roofline"] = {"bound": bound, "frac": round(frac, 4)}
    traffic = profiled_traffic(config, call, nbytes)
    if traffic:
        e["traffic"] = traffic
    if extra:
        e.update(extra)
    return e


def run_rbf_config(n, iters, warmup, seeds, cpu):
    """RBF fwd and bwd at N = M = n: timed on seed 0, outputs of every seed
    compared with the float64 oracle (and, at 2048, with the reference's
    torch CPU path)."""
    g = RbfGpu(n)
    fb, bb, ff, bf = rbf_work(n, n, g.d)
    errs = {}
    cpu_ref = None
    timer = Timer(g.torch.device("cuda:0"))
    t_fwd = t_bwd = None
    for seed in seeds:
        X, Y, dK = g.load(seed)
        g.fwd()
        g.bwd()
        out = g.outputs()
        if seed == seeds[0]:
            t_fwd = timer.us(g.fwd, iters, warmup)
            t_bwd = timer.us(g.bwd, iters, warmup)
        if cpu:
            merge_errors(errs, cpu_rbf_errors(X, Y, dK, out, g.gamma))
            # The reference's CPU path at full size: every seed at 2048, the
            # first seed above it (seconds per call), unless the host cannot
            # hold its [N, M, D] intermediates.
            if n <= 2048 or seed == seeds[0]:
                need = rbf_cpu_reference_bytes(n, n, g.d)
                avail = host_mem_available()
                if avail is not None and need > 0.8 * avail:
                    cpu_ref = {"skipped": (f"OOM: the torch CPU reference needs about "
                                           f"{need / 2**30:.0f} GiB of host memory at N=M={n}, "
                                           f"D={g.d}; MemAvailable is {avail / 2**30:.0f} GiB")}
                else:
                    cpu_ref = cpu_rbf_reference(X, Y, dK, out, g.gamma, cpu_ref)
    name = f"rbf N=M={n} D=64"
    common = {"seeds": list(seeds)}
    fe = _entry(name, "forward", t_fwd, fb, ff, "mfma", dict(common))
    be = _entry(name, "backward", t_bwd, bb, bf, "mfma", dict(common))
    if errs:
        fe["outputs"] = {"K": errs["K"]}
        be["outputs"] = {"dX": errs["dX"], "dY": errs["dY"]}
    if cpu_ref and "skipped" in cpu_ref:
        fe["cpu_reference"] = be["cpu_reference"] = dict(cpu_ref)
    elif cpu_ref:
        fe["cpu_reference"] = cpu_ref["fwd"]
        be["cpu_reference"] = cpu_ref["bwd"]
        for e in (fe["cpu_reference"], be["cpu_reference"]):
            e["seeds"] = list(seeds) if n <= 2048 else [seeds[0]]
    return [fe, be], errs


def rbf_cpu_reference_bytes(n, m, d):
    """Peak host memory of the reference's CPU broadcast path with autograd:
    the [n, m, d] difference, its square and their gradients (four fp32
    [n, m, d] arrays at once)."""
    return 4 * 4 * n * m * d


def host_mem_available():
    """MemAvailable of /proc/meminfo in bytes (None where it cannot be read)."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except (OSError, ValueError, IndexError):
        pass
    return None


def run_layernorm_config(iters, warmup, cpu):
    import torch
    from framework import capi
    from cases.layernorm import op
    lib = op._lib()
    B, D, eps = 8192, 4096, 1e-5
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, D, generator=g)
    w = 1 + 0.1 * torch.randn(D, generator=g)
    b = 0.1 * torch.randn(D, generator=g)
    dy = torch.randn(B, D, generator=g)
    xd, wd, bd, dyd = (t.to(dev) for t in (x, w, b, dy))
    y, dx = torch.empty_like(xd), torch.empty_like(xd)
    mean, rstd = torch.empty(B, device=dev), torch.empty(B, device=dev)
    dw, db = torch.empty(D, device=dev), torch.empty(D, device=dev)
    wsb = lib.layernorm_backward_workspace_bytes(B, D)
    ws = torch.empty(max(wsb // 4, 1), device=dev)
    s, P, chk = capi.stream_of(xd), capi.ptr, _ok(lib, "layernorm_last_error")

    def fwd():
        chk(lib.layernorm_forward_f32(P(xd), P(wd), P(bd), P(y), P(mean), P(rstd), B, D, eps, s))

    def bwd():
        chk(lib.layernorm_backward_f32(P(dyd), P(xd), P(wd), P(mean), P(rstd), P(dx), P(dw), P(db),
                                       B, D, P(ws), wsb, s))

    fwd()
    bwd()
    torch.cuda.synchronize()
    out = {k: v.cpu().numpy() for k, v in (("y", y), ("dx", dx), ("dw", dw), ("db", db))}
    timer = Timer(dev)
    name = f"layernorm [{B},{D}]"
    fe = _entry(name, "forward", timer.us(fwd, iters, warmup), 8 * B * D + 8 * D + 8 * B)
    be = _entry(name, "backward", timer.us(bwd, iters, warmup), 12 * B * D + 12 * D + 8 * B)
    if cpu:
        errs, ref_ms = cpu_layernorm(x, w, b, dy, eps, out)
        fe["outputs"] = {"y": errs["y"]}
        be["outputs"] = {k: errs[k] for k in ("dx", "dw", "db")}
        fe["cpu_reference"], be["cpu_reference"] = ref_ms
    return [fe, be]


def run_scan_config(iters, warmup, cpu):
    import torch
    from framework import capi
    from cases.scan import op
    lib = op._lib()
    R, D = 64, 65536
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    x = (torch.rand(R, D, generator=g, dtype=torch.float64) * 2 - 1).float()
    dy = torch.randn(R, D, generator=torch.Generator().manual_seed(10_000))
    xi = torch.randint(-1000, 1001, (R, D), generator=g, dtype=torch.int32)
    xd, dyd, xid = x.to(dev), dy.to(dev), xi.to(dev)
    y, dx = torch.empty_like(xd), torch.empty_like(xd)
    y64 = torch.empty(R, D, dtype=torch.int64, device=dev)
    wsb = lib.scan_workspace_bytes(R, D)
    ws = torch.empty(max(wsb // 8, 1), dtype=torch.int64, device=dev)
    s, P, chk = capi.stream_of(xd), capi.ptr, _ok(lib, "scan_last_error")
    calls = {
        "forward_f32": lambda: chk(lib.scan_forward_f32(P(xd), P(y), R, D, P(ws), wsb, s)),
        "backward_f32": lambda: chk(lib.scan_backward_f32(P(dyd), P(dx), R, D, P(ws), wsb, s)),
        "forward_i32_i64": lambda: chk(lib.scan_forward_i32_i64(P(xid), P(y64), R, D, P(ws), wsb,
                                                                s)),
    }
    off = lib.scan_status_offset(R, D) // 8
    ws[off].zero_()
    for fn in calls.values():
        fn()
    torch.cuda.synchronize()
    out = {"y": y.cpu().numpy(), "dx": dx.cpu().numpy(), "y64": y64.cpu().numpy()}
    timer = Timer(dev)
    name = f"scan [{R},{D}]"
    ents = [_entry(name, "forward_f32", timer.us(calls["forward_f32"], iters, warmup), 8 * R * D),
            _entry(name, "backward_f32", timer.us(calls["backward_f32"], iters, warmup), 8 * R * D),
            _entry(name, "forward_i32_i64", timer.us(calls["forward_i32_i64"], iters, warmup),
                   12 * R * D)]
    torch.cuda.synchronize()
    trips = int(ws[off].item()) & 0xFFFFFFFF
    for e in ents:
        e["spin_cap_trips"] = trips
    if cpu:
        errs, ref_ms = cpu_scan(x, dy, xi, out)
        ents[0]["outputs"] = {"y": errs["y"]}
        ents[1]["outputs"] = {"dx": errs["dx"]}
        ents[2]["outputs"] = {"y": errs["y64"]}
        ents[2]["bit_exact"] = errs["y64"]["bit_exact"]
        for e, k in zip(ents, ("fwd", "bwd", "int")):
            e["cpu_reference"] = ref_ms[k]
    return ents


def run_spmv_config(iters, warmup, cpu):
    import torch
    from framework import capi
    from cases.spmv import op, reference as ref
    lib = op._lib()
    M = K = 1 << 20
    dev = torch.device("cuda:0")
    t = ref.make_zipf_inputs(M, K, 1, 0, torch.int32)
    dY = torch.randn(M, 1, generator=torch.Generator().manual_seed(10_000))
    ptr, col, vals, X = (t[k].to(dev) for k in ("row_ptr", "col_idx", "vals", "X"))
    dYd = dY.to(dev)
    nnz = vals.numel()
    Y = torch.empty(M, 1, device=dev)
    dv, dX = torch.empty_like(vals), torch.empty_like(X)
    wsb = lib.spmv_backward_workspace_bytes(M, K, 1, nnz)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    s, P, chk = capi.stream_of(X), capi.ptr, _ok(lib, "spmv_last_error")

    def fwd():
        chk(lib.spmv_forward_f32_i32(P(ptr), P(col), P(vals), P(X), P(Y), M, K, 1, nnz, s))

    def bwd_dx():
        chk(lib.spmv_backward_f32_i32(P(ptr), P(col), P(vals), P(X), P(dYd), None, P(dX), M, K, 1,
                                      nnz, P(ws), wsb, s))

    def bwd_both():
        chk(lib.spmv_backward_f32_i32(P(ptr), P(col), P(vals), P(X), P(dYd), P(dv), P(dX), M, K, 1,
                                      nnz, P(ws), wsb, s))

    # The autograd pair when vals needs a gradient: the forward also keeps
    # X[col] (nnz floats) and the backward's dvals streams it.
    Xg = torch.empty_like(vals)
    dv_g, dX_g = torch.empty_like(vals), torch.empty_like(X)

    def fwd_keep():
        chk(lib.spmv_forward_gather_f32_i32(P(ptr), P(col), P(vals), P(X), P(Y), P(Xg), M, K, 1,
                                            nnz, s))

    def bwd_gathered():
        chk(lib.spmv_backward_gathered_f32_i32(P(ptr), P(col), P(vals), P(X), P(Xg), P(dYd),
                                               P(dv_g), P(dX_g), M, K, 1, nnz, P(ws), wsb, s))

    fwd()
    bwd_both()
    torch.cuda.synchronize()
    out = {"y": Y.cpu().numpy(), "dX": dX.cpu().numpy(), "dvals": dv.cpu().numpy()}
    bwd_dx()
    fwd_keep()
    bwd_gathered()
    torch.cuda.synchronize()
    out["dX_only"] = dX.cpu().numpy()
    out["y_keep"] = Y.cpu().numpy()
    out["dX_g"], out["dvals_g"] = dX_g.cpu().numpy(), dv_g.cpu().numpy()
    timer = Timer(dev)
    name = f"spmv zipf 2^20 x 2^20 nnz={nnz} D=1 int32"
    base = 4 * (M + 1) + 8 * nnz
    ents = [_entry(name, "forward", timer.us(fwd, iters, warmup), base + 4 * K + 4 * M),
            _entry(name, "backward dX", timer.us(bwd_dx, iters, warmup), base + 4 * M + 4 * K),
            _entry(name, "backward dvals + dX", timer.us(bwd_both, iters, warmup),
                   base + 4 * M + 8 * K + 4 * nnz),
            _entry(name, "forward keeping X[col]", timer.us(fwd_keep, iters, warmup),
                   base + 4 * K + 4 * M + 4 * nnz),
            _entry(name, "backward dvals + dX from the kept X[col]",
                   timer.us(bwd_gathered, iters, warmup), base + 4 * M + 4 * K + 8 * nnz)]
    ents[3]["note"] = "autograd forward when vals requires grad"
    ents[4]["note"] = "autograd backward after ents[3]; same dvals bits as the gathering backward"
    ents[4]["dvals_bitwise_equal"] = bool((dv_g == dv).all().item())
    if cpu:
        host = {k: t[k] for k in ("row_ptr", "col_idx", "vals", "X")}
        errs, ref_ms = cpu_spmv(host, dY, out)
        ents[0]["outputs"] = {"y": errs["y"]}
        ents[1]["outputs"] = {"dX": errs["dX_only"]}
        ents[2]["outputs"] = {"dX": errs["dX"], "dvals": errs["dvals"]}
        ents[3]["outputs"] = {"y": errs["y_keep"]}
        ents[4]["outputs"] = {"dX": errs["dX_g"], "dvals": errs["dvals_g"]}
        ents[0]["cpu_reference"] = ref_ms["fwd"]
        ents[2]["cpu_reference"] = ref_ms["bwd"]
    return ents


def run_spmm_config(iters, warmup, cpu):
    """The reference's default SpMM (cases/spmv/config.py: M = K = 4096,
    D = 64, 64 nonzeros per row, int64 indices as the reference requires):
    forward, and the backward with dvals and dX (the autograd call)."""
    import torch
    from framework import capi
    from cases.spmv import op, reference as ref
    lib = op._lib()
    dev = torch.device("cuda:0")
    t = ref.make_inputs(0, torch.float32, "cpu")
    M = t["row_ptr"].numel() - 1
    K, D = t["X"].shape
    dY = torch.randn(M, D, generator=torch.Generator().manual_seed(10_000))
    ptr, col, vals, X = (t[k].to(dev) for k in ("row_ptr", "col_idx", "vals", "X"))
    dYd = dY.to(dev)
    nnz = vals.numel()
    Y = torch.empty(M, D, device=dev)
    dv, dX = torch.empty_like(vals), torch.empty_like(X)
    wsb = lib.spmv_backward_workspace_bytes(M, K, D, nnz)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    s, P, chk = capi.stream_of(X), capi.ptr, _ok(lib, "spmv_last_error")

    def fwd():
        chk(lib.spmv_forward_f32_i64(P(ptr), P(col), P(vals), P(X), P(Y), M, K, D, nnz, s))

    def bwd():
        chk(lib.spmv_backward_f32_i64(P(ptr), P(col), P(vals), P(X), P(dYd), P(dv), P(dX), M, K,
                                      D, nnz, P(ws), wsb, s))

    def bwd_dx():
        chk(lib.spmv_backward_f32_i64(P(ptr), P(col), P(vals), P(X), P(dYd), None, P(dX), M, K,
                                      D, nnz, P(ws), wsb, s))

    fwd()
    bwd()
    torch.cuda.synchronize()
    out = {"y": Y.cpu().numpy(), "dX": dX.cpu().numpy(), "dvals": dv.cpu().numpy()}
    bwd()
    torch.cuda.synchronize()
    repeat = bool(torch.equal(dX.cpu(), torch.from_numpy(out["dX"])))
    timer = Timer(dev)
    name = f"spmm reference default M=K={M} D={D} nnz={nnz} int64"
    base = 8 * (M + 1) + 12 * nnz
    ents = [_entry(name, "forward", timer.us(fwd, iters, warmup), base + 4 * K * D + 4 * M * D),
            _entry(name, "backward dvals + dX", timer.us(bwd, iters, warmup),
                   base + 4 * M * D + 8 * K * D + 4 * nnz,
                   extra={"dX_bitwise_repeatable": repeat}),
            _entry(name, "backward dX", timer.us(bwd_dx, iters, warmup),
                   base + 4 * M * D + 4 * K * D)]
    if cpu:
        host = {k: t[k] for k in ("row_ptr", "col_idx", "vals", "X")}
        out["dX_only"] = out["dX"]
        errs, ref_ms = cpu_spmv(host, dY, out)
        ents[0]["outputs"] = {"y": errs["y"]}
        ents[1]["outputs"] = {"dX": errs["dX"], "dvals": errs["dvals"]}
        ents[0]["cpu_reference"] = ref_ms["fwd"]
        ents[1]["cpu_reference"] = ref_ms["bwd"]
    return ents


# ------------------------------------------------------------------ CPU leg
def errors(got, ref, atol=ATOL, rtol=RTOL):
    """max_abs, max_rel (over entries with |ref| > atol; smaller ones are
    governed by the absolute bound) and the allclose verdict."""
    import numpy as np
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = np.abs(got - ref)
    aref = np.abs(ref)
    big = aref > atol
    return {"max_abs": float(diff.max()) if diff.size else 0.0,
            "max_rel": float((diff[big] / aref[big]).max()) if big.any() else 0.0,
            "allclose": bool(np.all(diff <= atol + rtol * aref))}


def merge_errors(acc, new):
    for k, e in new.items():
        if k not in acc:
            acc[k] = dict(e)
        else:
            acc[k]["max_abs"] = max(acc[k]["max_abs"], e["max_abs"])
            acc[k]["max_rel"] = max(acc[k]["max_rel"], e["max_rel"])
            acc[k]["allclose"] = acc[k]["allclose"] and e["allclose"]


def cpu_rbf_errors(X, Y, dK, out, gamma):
    """GPU outputs against the float64 oracle (oracle/rbf.py)."""
    from oracle import rbf as orbf
    Xn, Yn = X.numpy(), Y.numpy()
    K = orbf.forward_f64(Xn, Yn, gamma)
    e = {"K": errors(out["K"], K)}
    dX, dY = orbf.backward_f64(Xn, Yn, dK.numpy(), K, gamma)
    e["dX"] = errors(out["dX"], dX)
    e["dY"] = errors(out["dY"], dY)
    return e


def _median_ms(fn, reps=3):
    fn()  # warmup
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(ts)


def cpu_rbf_reference(X, Y, dK, out, gamma, acc):
    """the reference's torch CPU path (oracle/rbf.py
    torch_cpu_forward, autograd backward) at full size for this seed: its
    time, and the GPU outputs against its fp32 outputs."""
    import torch
    from oracle import rbf as orbf
    acc = acc or {"fwd": {"ms": [], "threads": torch.get_num_threads()},
                  "bwd": {"ms": [], "threads": torch.get_num_threads()}, "errs": {}}
    with torch.no_grad():
        K = orbf.torch_cpu_forward(X, Y, gamma)
    acc["fwd"]["ms"].append(round(_median_ms(lambda: _no_grad(orbf.torch_cpu_forward, X, Y,
                                                                gamma)), 2))
    Xr, Yr = X.clone().requires_grad_(True), Y.clone().requires_grad_(True)

    def bwd():
        Xr.grad = Yr.grad = None
        o = orbf.torch_cpu_forward(Xr, Yr, gamma)
        t0 = time.perf_counter()
        o.backward(dK)
        return (time.perf_counter() - t0) * 1e3

    bwd()
    acc["bwd"]["ms"].append(round(statistics.median(bwd() for _ in range(3)), 2))
    errs = {"K": errors(out["K"], K.numpy()), "dX": errors(out["dX"], Xr.grad.numpy()),
            "dY": errors(out["dY"], Yr.grad.numpy())}
    merge_errors(acc["errs"], errs)
    acc["fwd"]["gpu_vs_cpu_reference"] = {"K": acc["errs"]["K"]}
    acc["bwd"]["gpu_vs_cpu_reference"] = {"dX": acc["errs"]["dX"], "dY": acc["errs"]["dY"]}
    acc["fwd"]["what"] = acc["bwd"]["what"] = (
        "torch CPU broadcast reference (reference.py:14-20) at full size, median of 3 after "
        "1 warmup per seed; backward timed without the graph build")
    return acc


def _no_grad(fn, *a):
    import torch
    with torch.no_grad():
        return fn(*a)


def cpu_layernorm(x, w, b, dy, eps, out):
    import torch
    from oracle import layernorm as oln
    xn = x.numpy()
    y, _, _ = oln.forward_f64(xn, w.numpy(), b.numpy(), eps)
    dx, dw, db = oln.backward_f64(dy.numpy(), xn, w.numpy(), eps)
    errs = {"y": errors(out["y"], y), "dx": errors(out["dx"], dx), "dw": errors(out["dw"], dw),
            "db": errors(out["db"], db)}
    fwd_ms = _median_ms(lambda: _no_grad(oln.torch_cpu_forward, x, w, b, eps))
    xr, wr, br = (t.clone().requires_grad_(True) for t in (x, w, b))

    def bwd():
        o = oln.torch_cpu_forward(xr, wr, br, eps)
        t0 = time.perf_counter()
        o.backward(dy)
        return (time.perf_counter() - t0) * 1e3

    bwd()
    bwd_ms = statistics.median(bwd() for _ in range(3))
    th = torch.get_num_threads()
    return errs, ({"ms": round(fwd_ms, 2), "threads": th},
                  {"ms": round(bwd_ms, 2), "threads": th})


def cpu_scan(x, dy, xi, out):
    import numpy as np
    import torch
    from oracle import scan as osc
    y = osc.cumsum_f32(x.numpy())
    dx = osc.reverse_cumsum_f32(dy.numpy())
    y64 = osc.cumsum_i64(xi.numpy())
    e64 = errors(out["y64"], y64)
    e64["bit_exact"] = bool(np.array_equal(out["y64"], y64))
    errs = {"y": errors(out["y"], y), "dx": errors(out["dx"], dx), "y64": e64}
    th = torch.get_num_threads()
    return errs, {"fwd": {"ms": round(_median_ms(lambda: osc.torch_cpu_forward(x)), 2),
                          "threads": th},
                  "bwd": {"ms": round(_median_ms(lambda: torch.flip(torch.cumsum(
                      torch.flip(dy, [-1]), -1), [-1])), 2), "threads": th},
                  "int": {"ms": round(_median_ms(lambda: osc.torch_cpu_forward(xi)), 2),
                          "threads": th}}


def cpu_spmv(host, dY, out):
    import torch
    from oracle import spmv as osp
    args = [host[k].numpy() for k in ("row_ptr", "col_idx", "vals", "X")]
    y = osp.forward_f64(*args)
    dvals, dX = osp.backward_f64(*args, dY.numpy())
    ref = {"y": y, "dX": dX, "dX_only": dX, "dvals": dvals, "y_keep": y, "dX_g": dX,
           "dvals_g": dvals}
    errs = {k: errors(out[k], r) for k, r in ref.items() if k in out}
    rp, ci, v, X = (host[k] for k in ("row_ptr", "col_idx", "vals", "X"))
    th = torch.get_num_threads()
    fwd_ms = _median_ms(lambda: _no_grad(osp.torch_cpu_forward, rp.long(), ci.long(), v, X))
    vr, Xr = v.clone().requires_grad_(True), X.clone().requires_grad_(True)

    def bwd():
        o = osp.torch_cpu_forward(rp.long(), ci.long(), vr, Xr)
        t0 = time.perf_counter()
        o.backward(dY)
        return (time.perf_counter() - t0) * 1e3

    bwd()
    bwd_ms = statistics.median(bwd() for _ in range(3))
    return errs, {"fwd": {"ms": round(fwd_ms, 2), "threads": th},
                  "bwd": {"ms": round(bwd_ms, 2), "threads": th,
                          "what": "autograd of the torch CPU reference: dvals and dX"}}


def cpu_baseline(size, d, gamma, budget_s, model, share):
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
    fb, bb, _, _ = rbf_work(rows, size, d)
    return {
        "value": round((fb + bb) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": model,
        "sample": (f"torch CPU broadcast reference (oracle/rbf.py torch_cpu_forward + autograd "
                   f"backward) on X[:{rows}] x Y[{size}], D={d}, median of 3 after 1 warmup; "
                   f"{med*1e3:.1f} ms per fwd+bwd; torch threads {threads}, CPU share {share}, "
                   f"os.cpu_count()={os.cpu_count()}; {model}"),
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
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU work for the cpu_baseline sample (0 = skip the whole "
                         "CPU leg: no cpu_baseline, parity or per-config errors)")
    ap.add_argument("--configs", default="all",
                    help="comma list of rbf2048,rbf4096,rbf8192,layernorm,scan,spmv,spmm, "
                         "'all' or 'none' (headline only)")
    ap.add_argument("--config-iters", type=int, default=100,
                    help="timed calls per config entry (three repeats)")
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
    model, share = cpu_info()
    torch.set_num_threads(max(1, share))
    cpu = args.cpu_budget > 0
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    n = m = args.size
    d, gamma = 64, 0.5
    g = RbfGpu(n, d, gamma)
    X, Y, dK = g.load(0)
    stream = torch.cuda.current_stream(dev)
    timer = Timer(dev)

    for _ in range(args.warmup):
        timer.flush(dev)
        g.fwd()
        g.bwd()
    torch.cuda.synchronize()

    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
               torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for e0, e1, e2 in events:
        timer.flush(dev)
        e0.record(stream)
        g.fwd()
        e1.record(stream)
        g.bwd()
        e2.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    print(f"[bench] headline rbf {n}: {args.steps} steps timed", file=sys.stderr, flush=True)
    out0 = g.outputs()  # the timed region's own outputs (seed 0), checked below

    # End-to-end RBFFunction forward + backward through autograd (the case's
    # candidate), after and outside the timed region: the C-ABI calls above
    # plus torch's output allocations and the autograd engine.
    from cases.rbf import op
    e2e_us = []
    Xa = g.X.detach().clone().requires_grad_(True)
    Ya = g.Y.detach().clone().requires_grad_(True)
    for i in range(min(args.steps, 10) + 2):
        timer.flush(dev)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        op.candidate({"X": Xa, "Y": Ya}, {"gamma": gamma}).backward(g.dK)
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 2:
            e2e_us.append(a.elapsed_time(b) * 1e3)
        Xa.grad = Ya.grad = None

    fwd_us = [a.elapsed_time(b) * 1e3 for a, b, _ in events]
    bwd_us = [b.elapsed_time(c) * 1e3 for _, b, c in events]
    step_us = [f + b for f, b in zip(fwd_us, bwd_us)]
    step_gm, step_cv = repeat_stats(step_us)
    fwd_gm, fwd_cv = repeat_stats(fwd_us)
    bwd_gm, bwd_cv = repeat_stats(bwd_us)
    fb, bb, ff, bf = rbf_work(n, m, d)
    gbs = (fb + bb) / (step_gm * 1e-6) / 1e9
    fwd_tf = ff / (fwd_gm * 1e-6) / 1e12
    bwd_tf = bf / (bwd_gm * 1e-6) / 1e12

    traffic = None  # measured for the 4096 workload only
    tpath = os.path.join(REPO, TRAFFIC_SOURCE)
    if n == 4096 and m == 4096 and d == 64 and os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    # per-config entries (GPU timings; errors and CPU reference times from the CPU leg)
    wanted = {"all": ["rbf2048", "rbf4096", "rbf8192", "layernorm", "scan", "spmv", "spmm"],
              "none": []}.get(args.configs, [c for c in args.configs.split(",") if c])
    configs = []
    it, wu = args.config_iters, 3
    headline_errs = None
    for c in wanted:
        print(f"[bench] config {c}", file=sys.stderr, flush=True)
        if c.startswith("rbf"):
            ents, errs = run_rbf_config(int(c[3:]), it, wu, SEEDS, cpu)
            configs += ents
            if int(c[3:]) == n:
                headline_errs = errs
        elif c == "layernorm":
            configs += run_layernorm_config(it, wu, cpu)
        elif c == "scan":
            configs += run_scan_config(it, wu, cpu)
        elif c == "spmv":
            configs += run_spmv_config(it, wu, cpu)
        elif c == "spmm":
            configs += run_spmm_config(it, wu, cpu)
        else:
            raise SystemExit(f"bench.py: unknown config {c!r}")

    parity = None
    if cpu:
        print("[bench] parity of the timed outputs", file=sys.stderr, flush=True)
        timed = cpu_rbf_errors(X, Y, dK, out0, gamma)
        parity = {"vs": "oracle/rbf.py float64 (forward_f64, backward_f64)",
                  "atol": ATOL, "rtol": RTOL, "timed_outputs": timed}
        if headline_errs:
            parity["seeds"] = list(SEEDS)
            parity["all_seeds"] = headline_errs
        parity["pass"] = all(e["allclose"] for e in timed.values()) and (
            not headline_errs or all(e["allclose"] for e in headline_errs.values()))

    cpu_line = None
    if cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        try:
            cpu_line = cpu_baseline(n, d, gamma, args.cpu_budget, model, share)
        except (MemoryError, RuntimeError) as exc:  # report instead of dying
            cpu_line = {"value": None, "unit": "GB/s", "cores": None, "kind": "port",
                        "sample": f"skipped: {exc}"}

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_gm * 1e-3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (host-seeded N(0,1)/8 inputs, N(0,1) dK; copied to HBM before timing)",
        "config": {"workload": f"rbf fwd+bwd N=M={n} D={d} gamma={gamma}", "N": n, "M": m, "D": d,
                   "gamma": gamma, "flush_between_steps": "512 MiB read (evicts L2 + MALL without dirty lines)",
                   "timing": "HIP events per call, geometric mean over the K steps, "
                             "CV over three repeats"},
        "cv": round(step_cv, 4),
        "fwd_us": round(fwd_gm, 2),
        "bwd_us": round(bwd_gm, 2),
        "fwd_cv": round(fwd_cv, 4),
        "bwd_cv": round(bwd_cv, 4),
        "fwd_gbs": round(fb / (fwd_gm * 1e-6) / 1e9, 1),
        "bwd_gbs": round(bb / (bwd_gm * 1e-6) / 1e9, 1),
        "pct_hbm_roofline": round(100 * gbs / HBM_PEAK_GBS, 2),
        "e2e_autograd_us": round(statistics.median(e2e_us), 2),
        "fwd_tflops": round(fwd_tf, 2),
        "bwd_tflops": round(bwd_tf, 2),
        "pct_fp32_roofline": round(100 * (ff + bf) / (step_gm * 1e-6) / 1e12 / FP32_PEAK_TFLOPS, 2),
        "roofline": {
            "kernel": "rbf_backward_f32 (pair_bwd_d64_3r_kernel<RbfBwdOp> + rbf_bwd_reduce_kernel)",
            "bound": "mfma",
            "achieved": round(bwd_tf, 3),
            "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / FP32_PEAK_TFLOPS, 4),
            # the fp32 MFMA rate a microbenchmark sustains on this part (8
            # independent chains per wave, 8 waves per SIMD)
            "measured_peak": MEASURED_FP32_MFMA_TFLOPS,
            "frac_of_measured": round(bwd_tf / MEASURED_FP32_MFMA_TFLOPS, 4),
            "measured_peak_source": "profiles/peaks_mi355x.md (framework/peaks.hip)",
            "traffic": traffic,
            "traffic_source": (f"{TRAFFIC_SOURCE}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                               "passes over bench.py, scaled by a 256 MiB copy's readings")
            if traffic else None,
        },
        "parity": parity,
        "cpu_baseline": cpu_line,
        "configs": configs,
        "wall_s_timed_region": round(wall, 4),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
