"""Measured peak rates of the MI355X this runs on, beside the published ones.

The roofline fractions of this package are priced against AMD's published
MI355X peaks: HBM3E 8.0 TB/s and dense fp32 matrix 157.3 TFLOP/s.  This
tool measures what one GPU actually sustains, with the hand-written
microbenchmarks of framework/peaks.hip:

  read   grid-stride float4 read of a 1 GiB buffer (4 or 8 loads in flight)
  write  float4 stores to a 1 GiB buffer
  copy   1 GiB to 1 GiB (bytes read + bytes written)

The stream kernels run over a sweep of launch shapes (workgroups of 256
threads, and the read's loads in flight); each rate is the best of the
sweep, and the sweep is printed too.  The buffers are 4x the 256 MB
last-level cache (MALL), so the rates are HBM rates.
  mfma   v_mfma_f32_16x16x4f32 in 8 independent chains per wave, 8 waves
         per SIMD; also the shader clock during the loop (s_memtime ticks
         against the 100 MHz s_memrealtime counter)

Each rate is the median of --iters launches timed with HIP events on the
launch stream.  Prints one JSON line per rate and a table.

--sized-copy MiB[,MiB...] instead measures the copy kernel at the sizes of
the streaming cases (for example 16 MiB in + 16 MiB out is a [64, 65536]
fp32 scan), with a 512 MiB read between launches so that neither buffer
starts in the MALL, over the same sweep of workgroup counts.  At these
sizes the launch ramp and the tail are a visible share of the time, so the
copy rate there is the practical ceiling of a kernel that reads and writes
that many bytes once.  Run it under rocprofv3 --kernel-trace --stats for the
kernel-time figures beside the event times printed here.

Usage:  python nl2cuda-kernel-agent_amd/framework/peaks.py [--iters 20]
        python nl2cuda-kernel-agent_amd/framework/peaks.py --sized-copy 16,64,128
"""

import argparse
import json
import os
import statistics
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if PKG not in sys.path:
    sys.path.insert(0, PKG)

from framework import capi  # noqa: E402
from framework.loader import load_kernel  # noqa: E402

KERNEL_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "peaks_hip"
SOURCES = ["peaks.hip"]

HBM_PEAK_GBS = 8000.0
FP32_MATRIX_PEAK_TFLOPS = 157.3
PEAK_CLOCK_GHZ = 2.4
STREAM_BYTES = 1 << 30
SWEEP_BLOCKS = (1024, 2048, 4096, 8192, 16384, 32768)


def bind_library(lib):
    V, I64, I, S = capi.c_void_p, capi.c_int64, capi.c_int, capi.c_size_t
    capi.bind(lib, "peaks_read_f32x4", [V, I64, V, I, I, V])
    capi.bind(lib, "peaks_write_f32x4", [V, I64, I, V])
    capi.bind(lib, "peaks_copy_f32x4", [V, V, I64, I, V])
    capi.bind(lib, "peaks_mfma_f32_flops", [I, I], capi.c_double)
    capi.bind(lib, "peaks_mfma_f32", [V, V, I, I, V])
    capi.bind_last_error(lib, "peaks_last_error")
    return lib


def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _median_ms(fn, iters, stream):
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return statistics.median(ts)


def _median_ms_flushed(fn, flush, iters, stream):
    """Like _median_ms, with flush() run (outside the timed region) before
    every launch."""
    import torch
    ts = []
    for i in range(iters + 3):
        flush()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            ts.append(e0.elapsed_time(e1))
    return statistics.median(ts)


def sized_copy(sizes_mib, iters, blocks=None):
    """Copy kernel at the given sizes, with a 512 MiB read flush before each
    launch; prints one JSON line per launch shape and the best per size."""
    import torch
    dev = torch.device("cuda:0")
    lib = _lib()
    stream = torch.cuda.current_stream(dev)
    s = capi.stream_of(torch.empty(1, device=dev))
    P = capi.ptr

    def ok(st):
        capi.check(st, lib.peaks_last_error, "peaks")

    fl_n4 = (512 << 20) // 16
    fl = torch.ones(fl_n4 * 4, device=dev)
    sink = torch.empty(max(SWEEP_BLOCKS), device=dev)

    def flush():
        ok(lib.peaks_read_f32x4(P(fl), fl_n4, P(sink), 8192, 8, s))

    rows = []
    for mib in sizes_mib:
        n4 = (mib << 20) // 16
        a = torch.ones(n4 * 4, device=dev)
        b = torch.empty_like(a)
        top = None
        for g in blocks or (256, 512) + SWEEP_BLOCKS:
            t = _median_ms_flushed(lambda g=g: ok(lib.peaks_copy_f32x4(P(a), P(b), n4, g, s)),
                                   flush, iters, stream)
            gbs = 2 * (mib << 20) / (t * 1e-3) / 1e9
            print(json.dumps({"rate": f"copy {mib} MiB", "launch": f"{g} x 256",
                              "gbs": round(gbs, 1), "ms": round(t, 4)}), flush=True)
            if top is None or gbs > top[0]:
                top = (gbs, t, g)
        rows.append((mib, top))
        del a, b
    print("\n| bytes in + out | best launch | event time | rate (in + out) | fraction of 8 TB/s |")
    print("|---|---|---:|---:|---:|")
    for mib, (gbs, t, g) in rows:
        print(f"| {mib} + {mib} MiB | {g} x 256 | {1000 * t:.2f} µs | {gbs:,.0f} GB/s | "
              f"{100 * gbs / HBM_PEAK_GBS:.1f} % |")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--mfma-iters", type=int, default=4000, help="even")
    ap.add_argument("--sized-copy", default=None,
                    help="comma-separated MiB: copy at these sizes (flushed) instead")
    ap.add_argument("--blocks", default=None,
                    help="comma-separated workgroup counts for --sized-copy (default: a sweep)")
    ns = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        print("peaks: needs the GPU", file=sys.stderr)
        return 2
    if ns.sized_copy:
        blocks = tuple(int(v) for v in ns.blocks.split(",")) if ns.blocks else None
        return sized_copy([int(v) for v in ns.sized_copy.split(",")], ns.iters, blocks)
    dev = torch.device("cuda:0")
    lib = _lib()
    stream = torch.cuda.current_stream(dev)
    s = capi.stream_of(torch.empty(1, device=dev))
    P = capi.ptr

    def ok(st):
        capi.check(st, lib.peaks_last_error, "peaks")

    n4 = STREAM_BYTES // 16
    a = torch.ones(n4 * 4, device=dev)
    b = torch.empty_like(a)
    sink = torch.empty(max(SWEEP_BLOCKS), device=dev)
    rows = []
    sweep = []

    def best(name, nbytes, variants):
        top = None
        for label, fn in variants:
            t = _median_ms(fn, ns.iters, stream)
            gbs = nbytes / (t * 1e-3) / 1e9
            sweep.append({"rate": name, "launch": label, "gbs": round(gbs, 1), "ms": round(t, 4)})
            print(json.dumps(sweep[-1]), flush=True)
            if top is None or gbs > top[0]:
                top = (gbs, t, label)
        rows.append((f"{name} ({top[2]})", top[0], "GB/s", HBM_PEAK_GBS, top[1]))

    best("HBM read", STREAM_BYTES,
         [(f"{g} x 256, {u} loads", lambda g=g, u=u: ok(lib.peaks_read_f32x4(P(a), n4, P(sink), g, u, s)))
          for u in (4, 8) for g in SWEEP_BLOCKS])
    best("HBM write", STREAM_BYTES,
         [(f"{g} x 256", lambda g=g: ok(lib.peaks_write_f32x4(P(b), n4, g, s))) for g in SWEEP_BLOCKS])
    best("HBM copy (read + write)", 2 * STREAM_BYTES,
         [(f"{g} x 256", lambda g=g: ok(lib.peaks_copy_f32x4(P(a), P(b), n4, g, s)))
          for g in SWEEP_BLOCKS])
    del a, b
    props = torch.cuda.get_device_properties(dev)
    cus = props.multi_processor_count
    blocks = cus * 4 * 2  # 8 waves of 64 per SIMD (4 SIMDs per CU, 4 waves per workgroup)
    out = torch.empty(blocks * 256, device=dev)
    clk = torch.zeros(2, dtype=torch.int64, device=dev)
    flops = lib.peaks_mfma_f32_flops(blocks, ns.mfma_iters)
    t = _median_ms(lambda: ok(lib.peaks_mfma_f32(P(out), P(clk), blocks, ns.mfma_iters, s)),
                   ns.iters, stream)
    ticks, real = (int(v) for v in clk.cpu())
    ghz = ticks / (real / 100e6) / 1e9 if real else float("nan")
    rows.append(("fp32 MFMA (16x16x4)", flops / (t * 1e-3) / 1e12, "TFLOP/s",
                 FP32_MATRIX_PEAK_TFLOPS, t))
    for name, val, unit, peak, ms in rows:
        print(json.dumps({"rate": name, "value": round(val, 1), "unit": unit, "published_peak": peak,
                          "frac_of_published": round(val / peak, 4), "ms": round(ms, 4)}), flush=True)
    print(json.dumps({"rate": "shader clock during the MFMA loop", "value": round(ghz, 3),
                      "unit": "GHz", "published_peak": PEAK_CLOCK_GHZ, "cus": cus,
                      "fp32_matrix_peak_at_this_clock_tflops":
                          round(FP32_MATRIX_PEAK_TFLOPS * ghz / PEAK_CLOCK_GHZ, 1)}), flush=True)
    print("\n| rate | measured | published | fraction |")
    print("|---|---:|---:|---:|")
    for name, val, unit, peak, _ in rows:
        print(f"| {name} | {val:,.0f} {unit} | {peak:,.1f} {unit} | {100 * val / peak:.1f} % |")
    print(f"| shader clock (MFMA loop) | {ghz:.2f} GHz | {PEAK_CLOCK_GHZ} GHz | "
          f"{100 * ghz / PEAK_CLOCK_GHZ:.1f} % |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
