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

--coexec instead measures memory staging beside fp32 MFMA work on every CU
(peak_coexec_kernel): four staging waves stream 64 x 64 tile pairs (the RBF
backward's pattern) while eight waves run MFMAs, which shows how much of
the memory side an MFMA-bound kernel can keep going on waves of its own.

Usage:  python nl2cuda-kernel-agent_amd/framework/peaks.py [--iters 20]
        python nl2cuda-kernel-agent_amd/framework/peaks.py --coexec
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
    capi.bind(lib, "peaks_coexec", [V, V, V, V, I, I, I, I, I, I, I, V])
    capi.bind(lib, "peaks_joint", [V, V, V, V, I, I, I, I, I, I, V])
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


def coexec(iters, tiles=64, mfma_iters=3840):
    """Staging waves beside fp32 MFMA waves on every CU (peak_coexec_kernel):
    the stagers' time per 32 KB tile pair and the MFMA waves' rate, for no
    MFMA, 16x16x4 and 32x32x2 MFMAs, staging through registers or straight
    into LDS, with one or two MFMA waves and one or two staging waves per
    SIMD.  Prints one JSON line per configuration and a table."""
    import torch
    dev = torch.device("cuda:0")
    lib = _lib()
    s = capi.stream_of(torch.empty(1, device=dev))
    P = capi.ptr
    n = 4096
    A = torch.ones(n * n, device=dev)
    B = torch.ones(n * n, device=dev)
    out = torch.zeros(2, device=dev)
    ticks = torch.zeros(4096, dtype=torch.int64, device=dev)
    blocks = min(256, torch.cuda.get_device_properties(dev).multi_processor_count)
    flops_per = {1: 2.0 * 16 * 16 * 4, 2: 2.0 * 32 * 32 * 2}
    names = {0: "none", 1: "16x16x4", 2: "32x32x2"}
    configs = [(kind, direct, 8, 4) for kind in (0, 1, 2) for direct in (0, 1)]
    configs += [(1, direct, mw, ns) for direct in (0, 1) for mw, ns in ((4, 4), (8, 8), (4, 8))]
    rows = []
    for kind, direct, mw, ns_w in configs:
        tile_ns, mfma_tf = [], []
        for _ in range(iters):
            capi.check(lib.peaks_coexec(P(A), P(B), P(out), P(ticks), blocks, tiles, kind,
                                        mfma_iters, direct, mw, ns_w, s),
                       lib.peaks_last_error, "peaks")
            torch.cuda.synchronize()
            t = ticks.cpu().numpy()
            tile_ns.append(statistics.median(t[:ns_w * blocks].tolist()) * 10.0 / tiles)
            if kind:
                mt = statistics.median([int(t[2048 + 8 * b + w]) for b in range(blocks)
                                        for w in range(mw)]) * 10.0
                mfma_tf.append(blocks * mw * mfma_iters * 8 * flops_per[kind] / (mt * 1e-9) / 1e12)
        ns = statistics.median(tile_ns)
        tf = statistics.median(mfma_tf) if mfma_tf else None
        row = {"rate": "staging beside MFMA", "mfma": names[kind],
               "mfma_waves_per_simd": mw // 4 if kind else 0, "stagers_per_simd": ns_w // 4,
               "staging": "direct to LDS" if direct else "through registers",
               "ns_per_tile": round(ns, 1), "staging_tbs": round(blocks * 32768 / ns / 1e3, 2),
               "mfma_tflops": round(tf, 1) if tf else None}
        print(json.dumps(row), flush=True)
        rows.append(row)
    print("\n| MFMA | MFMA waves / SIMD | stagers / SIMD | staging | ns per 32 KB tile pair per CU | "
          "staging TB/s (chip) | MFMA TFLOP/s |")
    print("|---|---:|---:|---|---:|---:|---:|")
    for r in rows:
        print(f"| {r['mfma']} | {r['mfma_waves_per_simd']} | {r['stagers_per_simd']} | {r['staging']} | "
              f"{r['ns_per_tile']:,.0f} | {r['staging_tbs']:.2f} | "
              f"{r['mfma_tflops'] if r['mfma_tflops'] else '-'} |")
    return 0


def joint(iters, tiles=64):
    """The same MFMA work per SIMD on one or two waves beside a pipelined
    staging wave (peak_joint_kernel): 64 tile pairs of 32 KB per CU straight
    into LDS with two or three in flight, and 0-1536 rounds of eight fp32
    16x16x4 MFMAs per SIMD (1024 rounds = 128 MFMAs per tile pair, the RBF
    backward's ratio).  Reports the workgroup span and each side's time
    (median over the CUs, median of `iters` launches)."""
    import torch
    dev = torch.device("cuda:0")
    lib = _lib()
    s = capi.stream_of(torch.empty(1, device=dev))
    P = capi.ptr
    n = 4096
    A = torch.ones(n * n, device=dev)
    B = torch.ones(n * n, device=dev)
    out = torch.zeros(2, device=dev)
    ticks = torch.zeros(1024, dtype=torch.int64, device=dev)
    blocks = min(256, torch.cuda.get_device_properties(dev).multi_processor_count)
    rows = []
    for depth in (2, 3):
        for simd_iters in (0, 512, 1024, 1536):
            for mw, inl in ((((0, 0),) if simd_iters == 0 else ((4, 0), (8, 0), (4, 1)))):
                span, stg, mf = [], [], []
                for _ in range(iters):
                    capi.check(lib.peaks_joint(P(A), P(B), P(out), P(ticks), blocks, tiles,
                                               simd_iters, mw, depth, inl, s),
                               lib.peaks_last_error, "peaks")
                    torch.cuda.synchronize()
                    t = ticks.cpu().numpy()[:4 * blocks].reshape(blocks, 4)
                    span.append(statistics.median(t[:, 0].tolist()) / 100.0)
                    stg.append(statistics.median(t[:, 1].tolist()) / 100.0)
                    mf.append(statistics.median(t[:, 2].tolist()) / 100.0)
                row = {"rate": "joint staging + MFMA", "depth": depth, "simd_mfma_rounds": simd_iters,
                       "mfma_waves_per_simd": mw // 4,
                       "staged_by": "the MFMA wave" if inl else ("a staging wave" if mw else "-"),
                       "span_us": round(statistics.median(span), 2),
                       "staging_us": round(statistics.median(stg), 2),
                       "mfma_us": round(statistics.median(mf), 2)}
                print(json.dumps(row), flush=True)
                rows.append(row)
    print("\n| tiles in flight | MFMA rounds per SIMD | MFMA waves / SIMD | tiles staged by | "
          "workgroup span µs | staging µs | MFMA µs |")
    print("|---:|---:|---:|---|---:|---:|---:|")
    for r in rows:
        print(f"| {r['depth']} | {r['simd_mfma_rounds']} | {r['mfma_waves_per_simd']} | "
              f"{r['staged_by']} | {r['span_us']:.2f} | {r['staging_us']:.2f} | {r['mfma_us']:.2f} |")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--mfma-iters", type=int, default=4000, help="even")
    ap.add_argument("--sized-copy", default=None,
                    help="comma-separated MiB: copy at these sizes (flushed) instead")
    ap.add_argument("--blocks", default=None,
                    help="comma-separated workgroup counts for --sized-copy (default: a sweep)")
    ap.add_argument("--coexec", action="store_true",
                    help="staging waves beside MFMA waves on one CU instead (peak_coexec_kernel)")
    ap.add_argument("--joint", action="store_true",
                    help="the same MFMA work on one or two waves per SIMD beside a pipelined "
                         "staging wave instead (peak_joint_kernel)")
    ns = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        print("peaks: needs the GPU", file=sys.stderr)
        return 2
    if ns.coexec:
        return coexec(min(ns.iters, 7))
    if ns.joint:
        return joint(min(ns.iters, 7))
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
