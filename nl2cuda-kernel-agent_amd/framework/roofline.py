"""Roofline report for the follow-on cases (layernorm, l2norm_scale, scan,
spmv, cosine_sim, softmax_ce) on one GPU.

For each case's acceptance workload this times every C-ABI entry point
directly on preallocated device buffers: a 512 MiB read flush before each
call (so operands come from HBM, not L2 or the MALL), HIP events on the
launch stream around the call, ``--iters`` timed calls after ``--warmup``.
Achieved GB/s = algorithmic bytes / mean time (each input read once, each
output written once; the byte counts are stated per entry), against the
MI355X HBM peak of 8 TB/s; the MFMA-bound cosine entries also give TFLOP/s
(2NMD forward, 4NMD backward) against 157.3 TF.  Event times include the
launch (a few us); rocprofv3 kernel times (framework/profile.py stats) give
the kernel-only figure.

Usage:  python nl2cuda-kernel-agent_amd/framework/roofline.py
            [--case all|layernorm|l2norm|scan|spmv|cosine|softmax_ce]
Prints one JSON line per measurement and a closing table.
"""

import argparse
import ctypes
import json
import os
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA (AMD published)


def _timer(dev, iters, warmup):
    import torch
    from framework.bench import flush_caches

    def time_us(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        stream = torch.cuda.current_stream(dev)
        for _ in range(iters):
            flush_caches(dev)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        ts.sort()
        trim = ts[len(ts) // 10: len(ts) - len(ts) // 10] or ts
        return sum(trim) / len(trim)

    return time_us


def _check(st, lib, err):
    if st != 0:
        raise RuntimeError(getattr(lib, err)().decode())


def layernorm(dev, time_us):
    import torch
    from framework import capi
    from cases.layernorm import op
    lib = op._lib()
    B, D = 8192, 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, D, generator=g).to(dev)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev)
    b = (0.1 * torch.randn(D, generator=g)).to(dev)
    dy = torch.randn(B, D, generator=g).to(dev)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    mean, rstd = torch.empty(B, device=dev), torch.empty(B, device=dev)
    dw, db = torch.empty(D, device=dev), torch.empty(D, device=dev)
    wsb = lib.layernorm_backward_workspace_bytes(B, D)
    ws = torch.empty(max(wsb // 4, 1), device=dev)
    s, P = capi.stream_of(x), capi.ptr
    out = []
    t = time_us(lambda: _check(lib.layernorm_forward_f32(P(x), P(w), P(b), P(y), P(mean), P(rstd),
                                                         B, D, 1e-5, s), lib, "layernorm_last_error"))
    out.append(("layernorm", "forward_f32 [8192,4096]", t, 8 * B * D + 8 * D + 8 * B,
                "read x, w, bias; write y, mean, rstd"))
    t = time_us(lambda: _check(lib.layernorm_backward_f32(P(dy), P(x), P(w), P(mean), P(rstd), P(dx),
                                                          P(dw), P(db), B, D, P(ws), wsb, s),
                               lib, "layernorm_last_error"))
    out.append(("layernorm", "backward_f32 [8192,4096]", t, 12 * B * D + 12 * D + 8 * B,
                "read dy, x, w, mean, rstd; write dx, dw, dbias"))
    return out


SCAN_SHAPES = ((64, 65536), (4096, 4096))


def l2norm(dev, time_us):
    """L2-norm-scale (HBM-bound): forward reads X and g, writes Y and the
    norms; backward reads dY, X, g and the norms, writes dX and dg."""
    import torch
    from framework import capi
    from cases.l2norm_scale import op, config
    lib = op._lib()
    out = []
    for N, D in config.BENCH_SHAPES:
        gen = torch.Generator().manual_seed(0)
        x = torch.randn(N, D, generator=gen).to(dev)
        g = torch.randn(D, generator=gen).to(dev)
        dy = torch.randn(N, D, generator=gen).to(dev)
        y, dx = torch.empty_like(x), torch.empty_like(x)
        norm, dg = torch.empty(N, device=dev), torch.empty(D, device=dev)
        wsb = lib.l2norm_scale_backward_workspace_bytes(N, D)
        ws = torch.empty(max(wsb // 4, 1), device=dev)
        s, P = capi.stream_of(x), capi.ptr
        t = time_us(lambda: _check(lib.l2norm_scale_forward_f32(P(x), P(g), P(y), P(norm), N, D,
                                                                1e-6, s), lib, "l2norm_scale_last_error"))
        out.append(("l2norm_scale", f"forward_f32 [{N},{D}]", t, 8 * N * D + 4 * D + 4 * N,
                    "read X, g; write Y, norm"))
        t = time_us(lambda: _check(lib.l2norm_scale_backward_f32(P(dy), P(x), P(g), P(norm), P(dx),
                                                                 P(dg), N, D, P(ws), wsb, s),
                                   lib, "l2norm_scale_last_error"))
        out.append(("l2norm_scale", f"backward_f32 [{N},{D}]", t, 12 * N * D + 8 * D + 4 * N,
                    "read dY, X, g, norm; write dX, dg"))
    return out


def softmax_ce(dev, time_us):
    """Softmax cross-entropy (HBM-bound): forward reads logits and labels,
    writes lse and the loss; backward reads logits, labels, lse and gout,
    writes dlogits.  The forward's scratch (one partial per workgroup, 4 KiB)
    is not counted."""
    import torch
    from framework import capi
    from cases.softmax_ce import op, config
    lib = op._lib()
    out = []
    for B, C in config.BENCH_SHAPES:
        gen = torch.Generator().manual_seed(0)
        x = torch.randn(B, C, generator=gen).to(dev)
        lab = torch.randint(0, C, (B,), generator=gen).to(dev)
        dx = torch.empty_like(x)
        loss, lse = torch.empty(1, device=dev), torch.empty(B, device=dev)
        gout = torch.ones(1, device=dev)
        wsb = lib.softmax_ce_forward_workspace_bytes(B, C)
        ws = torch.empty(max(wsb // 4, 1), device=dev)
        s, P = capi.stream_of(x), capi.ptr
        t = time_us(lambda: _check(lib.softmax_ce_forward_f32(P(x), P(lab), P(loss), P(lse), B, C,
                                                              P(ws), wsb, s),
                                   lib, "softmax_ce_last_error"))
        out.append(("softmax_ce", f"forward_f32 [{B},{C}]", t, 4 * B * C + 12 * B + 4,
                    "read logits, labels; write lse, loss"))
        t = time_us(lambda: _check(lib.softmax_ce_backward_f32(P(x), P(lab), P(lse), P(gout), P(dx),
                                                               B, C, s),
                                   lib, "softmax_ce_last_error"))
        out.append(("softmax_ce", f"backward_f32 [{B},{C}]", t, 8 * B * C + 12 * B + 4,
                    "read logits, labels, lse, gout; write dlogits"))
    return out


def scan(dev, time_us, shapes=SCAN_SHAPES):
    import torch
    from framework import capi
    from cases.scan import op
    lib = op._lib()
    out = []
    for R, D in shapes:
        g = torch.Generator().manual_seed(0)
        x = (torch.rand(R, D, generator=g) * 2 - 1).to(dev)
        xi = torch.randint(-1000, 1001, (R, D), generator=g, dtype=torch.int32).to(dev)
        y = torch.empty_like(x)
        y64 = torch.empty(R, D, dtype=torch.int64, device=dev)
        y32 = torch.empty_like(xi)
        wsb = lib.scan_workspace_bytes(R, D)
        ws = torch.empty(max(wsb // 4, 1), device=dev)  # zeroed once
        s, P = capi.stream_of(x), capi.ptr
        shape = f"[{R},{D}]"
        for name, fn, nbytes, what in (
                ("forward_f32", lambda: lib.scan_forward_f32(P(x), P(y), R, D, P(ws), wsb, s),
                 8 * R * D, "read x, write y (f32)"),
                ("backward_f32", lambda: lib.scan_backward_f32(P(x), P(y), R, D, P(ws), wsb, s),
                 8 * R * D, "read dy, write dx (f32)"),
                ("forward_i32_i64", lambda: lib.scan_forward_i32_i64(P(xi), P(y64), R, D, P(ws), wsb, s),
                 12 * R * D, "read int32, write int64"),
                ("forward_i32", lambda: lib.scan_forward_i32(P(xi), P(y32), R, D, P(ws), wsb, s),
                 8 * R * D, "read int32, write int32")):
            t = time_us(lambda fn=fn: _check(fn(), lib, "scan_last_error"))
            out.append(("scan", f"{name} {shape}", t, nbytes, what))
    return out


def spmv(dev, time_us):
    import torch
    from framework import capi
    from cases.spmv import op, reference as ref
    lib = op._lib()
    M = K = 1 << 20
    t = ref.make_zipf_inputs(M, K, 1, 0, torch.int32)
    ptr, col, vals, X = (t[k].to(dev) for k in ("row_ptr", "col_idx", "vals", "X"))
    nnz = vals.numel()
    Y = torch.empty(M, 1, device=dev)
    dY = torch.randn(M, 1, generator=torch.Generator().manual_seed(1)).to(dev)
    dv, dX = torch.empty_like(vals), torch.empty_like(X)
    wsb = lib.spmv_backward_workspace_bytes(M, K, 1, nnz)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    s, P = capi.stream_of(X), capi.ptr
    base = 4 * (M + 1) + 8 * nnz
    out = []
    tt = time_us(lambda: _check(lib.spmv_forward_f32_i32(P(ptr), P(col), P(vals), P(X), P(Y), M, K, 1,
                                                        nnz, s), lib, "spmv_last_error"))
    out.append(("spmv", "forward_f32_i32 zipf 2^20 D=1", tt, base + 4 * K + 4 * M,
                "read row_ptr, col_idx, vals, x; write y"))
    tt = time_us(lambda: _check(lib.spmv_backward_f32_i32(P(ptr), P(col), P(vals), P(X), P(dY), None,
                                                         P(dX), M, K, 1, nnz, P(ws), wsb, s),
                                lib, "spmv_last_error"))
    out.append(("spmv", "backward dx only, zipf 2^20", tt, base + 4 * M + 4 * K,
                "read structure, dy; write dx"))
    tt = time_us(lambda: _check(lib.spmv_backward_f32_i32(P(ptr), P(col), P(vals), P(X), P(dY), P(dv),
                                                         P(dX), M, K, 1, nnz, P(ws), wsb, s),
                                lib, "spmv_last_error"))
    out.append(("spmv", "backward dvals + dx, zipf 2^20", tt, base + 4 * M + 8 * K + 4 * nnz,
                "read structure, dy, x; write dvals, dx"))
    # the autograd pair when vals needs a gradient: the forward keeps x[col]
    # and the backward streams it
    xg = torch.empty_like(vals)
    tt = time_us(lambda: _check(lib.spmv_forward_gather_f32_i32(P(ptr), P(col), P(vals), P(X), P(Y),
                                                               P(xg), M, K, 1, nnz, s),
                                lib, "spmv_last_error"))
    out.append(("spmv", "forward keeping x[col], zipf 2^20", tt, base + 4 * K + 4 * M + 4 * nnz,
                "read row_ptr, col_idx, vals, x; write y, x[col]"))
    tt = time_us(lambda: _check(lib.spmv_backward_gathered_f32_i32(
        P(ptr), P(col), P(vals), P(X), P(xg), P(dY), P(dv), P(dX), M, K, 1, nnz, P(ws), wsb, s),
        lib, "spmv_last_error"))
    out.append(("spmv", "backward dvals + dx from kept x[col], zipf 2^20", tt,
                base + 4 * M + 4 * K + 8 * nnz, "read structure, dy, x[col]; write dvals, dx"))
    return out


COSINE_SIZES = (2048, 4096)


def cosine(dev, time_us, sizes=COSINE_SIZES):
    """Pairwise cosine similarity (fp32 MFMA-bound): flops = 2NMD forward,
    4NMD backward; bytes = each input read once, each output written once."""
    import torch
    from framework import capi
    from cases.cosine_sim import op
    lib = op._lib()
    out = []
    for n in sizes:
        D = 64
        g = torch.Generator().manual_seed(0)
        A = torch.randn(n, D, generator=g).to(dev)
        B = torch.randn(n, D, generator=g).to(dev)
        dS = torch.randn(n, n, generator=g).to(dev)
        S = torch.empty(n, n, device=dev)
        ia, ib = torch.empty(n, device=dev), torch.empty(n, device=dev)
        dA, dB = torch.empty_like(A), torch.empty_like(B)
        wsb = lib.cosine_sim_backward_workspace_bytes(n, n, D)
        ws = torch.empty(max(wsb // 4, 1), device=dev)
        s, P = capi.stream_of(A), capi.ptr
        t = time_us(lambda: _check(lib.cosine_sim_forward_f32(P(A), P(B), P(S), P(ia), P(ib), n, n,
                                                              D, 1e-8, s), lib, "cosine_sim_last_error"))
        out.append(("cosine_sim", f"forward_f32 [{n},{n}] D=64", t, 4 * n * n + 8 * n * D + 8 * n,
                    "read A, B; write S, inv_a, inv_b", 2 * n * n * D))
        t = time_us(lambda: _check(lib.cosine_sim_backward_f32(P(A), P(B), P(ia), P(ib), P(dS), P(dA),
                                                               P(dB), n, n, D, P(ws), wsb, s),
                                   lib, "cosine_sim_last_error"))
        out.append(("cosine_sim", f"backward_f32 [{n},{n}] D=64", t, 4 * n * n + 16 * n * D + 8 * n,
                    "read dS, A, B, inv_a, inv_b; write dA, dB", 4 * n * n * D))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--case", default="all",
                    choices=["all", "layernorm", "l2norm", "scan", "spmv", "cosine",
                             "softmax_ce"])
    ap.add_argument("--iters", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--scan-shape", default=None, metavar="RxD",
                    help="time only this scan shape (default: 64x65536 and 4096x4096)")
    ap.add_argument("--cosine-size", type=int, default=None, metavar="N",
                    help="time only N x N cosine similarity (default: 2048 and 4096)")
    ns = ap.parse_args(argv)
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    time_us = _timer(dev, ns.iters, ns.warmup)
    scan_shapes = SCAN_SHAPES
    if ns.scan_shape:
        r, d = (int(v) for v in ns.scan_shape.lower().split("x"))
        scan_shapes = ((r, d),)
    cos_sizes = (ns.cosine_size,) if ns.cosine_size else COSINE_SIZES
    cases = {"layernorm": layernorm, "l2norm": l2norm,
             "scan": lambda dv, t: scan(dv, t, scan_shapes), "spmv": spmv,
             "cosine": lambda dv, t: cosine(dv, t, cos_sizes), "softmax_ce": softmax_ce}
    rows = []
    for name in (cases if ns.case == "all" else [ns.case]):
        for case, what, t, nbytes, detail, *flops in cases[name](dev, time_us):
            gbs = nbytes / (t * 1e-6) / 1e9
            rec = {"case": case, "entry": what, "us": round(t, 2), "bytes": nbytes,
                   "gbs": round(gbs, 1), "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                   "bytes_are": detail}
            if flops:
                tf = flops[0] / (t * 1e-6) / 1e12
                rec.update(flops=flops[0], tflops=round(tf, 1),
                           pct_fp32=round(100 * tf / FP32_PEAK_TFLOPS, 1))
            print(json.dumps(rec), flush=True)
            rows.append(rec)
    print("\n| case | entry | event µs | algorithmic bytes | GB/s | % of 8 TB/s | TFLOP/s | % of 157.3 TF |")
    print("|---|---|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        tf = f"{r['tflops']:.1f} | {r['pct_fp32']:.1f}" if "tflops" in r else "— | —"
        print(f"| {r['case']} | {r['entry']} | {r['us']:.2f} | {r['bytes']:,} | {r['gbs']:.0f} | "
              f"{r['pct_hbm']:.1f} | {tf} |")
    return 0


if __name__ == "__main__":
    sys.exit(main())
