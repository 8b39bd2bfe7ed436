"""Timing harness: candidate vs a baseline, forward and backward.

Same protocol as the reference's framework/bench.py:27-178: warmup, then
``iters`` timed calls with device events, geometric mean, ``repeats`` rounds
to compute the coefficient of variation, up to ``max_retries`` re-measurements
while CV > 5 %, backward timed with the autograd graph rebuilt outside the
timed region.  Added for MI355X:

  * a cache flush between timed iterations: a read of PROTOCOL.flush_bytes
    (512 MiB) evicts the 4 MiB L2 of every XCD and the 256 MiB MALL, so each
    timed call reads its operands from HBM (``flush=False`` disables it).  The
    flush reads rather than writes: a 512 MiB write leaves ~256 MB of dirty
    MALL lines whose write-back then competes with the timed kernel's reads
    (measured on MI355X: a linear 256 MiB read runs at ~3.0 TB/s right after
    a write flush and at ~6.0 TB/s after a read flush);
  * ``time_ms`` is exposed for other drivers (the repository's bench.py).

The baseline defaults to ``torch.compile(case.reference_forward)`` as in the
reference; ``baseline="eager"`` times the eager reference instead.
"""

import math
import os
import sys
from dataclasses import dataclass

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import torch  # noqa: E402

from framework.protocol import PROTOCOL, dtype_of  # noqa: E402

_FLUSH = {}


def _flush_buffer(device):
    key = str(device)
    if key not in _FLUSH:
        buf = torch.zeros(PROTOCOL.flush_bytes // 4, dtype=torch.float32, device=device)
        torch.cuda.synchronize()
        _FLUSH[key] = (buf, torch.empty(1, dtype=torch.float32, device=device))
    return _FLUSH[key]


def flush_caches(device="cuda"):
    """Read a 512 MiB buffer so no operand stays in L2 or the MALL (and no
    dirty lines are left behind to be written back during the next call)."""
    buf, sink = _flush_buffer(device)
    torch.sum(buf, dim=0, out=sink[0])


def _geomean(xs):
    return math.exp(sum(math.log(max(x, 1e-12)) for x in xs) / len(xs))


def time_ms(fn, warmup=None, iters=None, flush=True, setup=None, device="cuda"):
    """Per-iteration device time (ms) of ``fn`` between two HIP events.

    ``setup`` (optional) runs before each iteration outside the timed region
    and returns the callable to time (used for backward: it rebuilds the
    graph).  Returns the list of times.
    """
    p = PROTOCOL
    warmup = p.warmup if warmup is None else warmup
    iters = p.iters if iters is None else iters
    for _ in range(warmup):
        (setup() if setup else fn)()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        call = setup() if setup else fn
        if flush:
            flush_caches(device)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        call()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
    return times


@dataclass
class Timing:
    """One stable measurement of a call: ``rounds_ms`` holds the geometric
    mean of each round of ``PROTOCOL.iters`` timed iterations; ``center_ms``
    is their geometric mean and ``cv`` their coefficient of variation.  The
    measurement is ``stable`` when cv <= PROTOCOL.cv_threshold; ``tries``
    counts the measurements taken to get there (at most max_retries + 1)."""
    label: str
    rounds_ms: list
    center_ms: float
    cv: float
    stable: bool
    tries: int = 1


def spread(values):
    """Population coefficient of variation (inf for a non-positive mean)."""
    m = sum(values) / len(values)
    if m <= 0:
        return float("inf")
    return math.sqrt(sum((v - m) ** 2 for v in values) / len(values)) / m


def until_stable(label, measure_round, rounds=None, cv_limit=None, retries=None):
    """Measure ``rounds`` rounds (``measure_round()`` returns one round's
    per-iteration times) and repeat the whole measurement while their
    geomeans spread by more than ``cv_limit``, at most ``retries`` extra
    times.  Returns the Timing with the lowest spread seen, so an unstable
    result is still the best one the retries produced."""
    p = PROTOCOL
    rounds = p.repeats if rounds is None else rounds
    cv_limit = p.cv_threshold if cv_limit is None else cv_limit
    retries = p.max_retries if retries is None else retries
    kept = None
    for n in range(1, retries + 2):
        centers = [_geomean(measure_round()) for _ in range(rounds)]
        t = Timing(label, centers, _geomean(centers), spread(centers), False, n)
        t.stable = t.cv <= cv_limit
        if kept is None or t.cv < kept.cv:
            kept = t
        if t.stable:
            break
    kept.tries = n
    return kept


def time_forward(fn, inputs, params, flush=True):
    """Forward calls under no_grad on detached inputs."""
    frozen = {k: v.detach() for k, v in inputs.items()}

    def call():
        with torch.no_grad():
            fn(frozen, params)
    return until_stable("forward", lambda: time_ms(call, flush=flush))


def time_backward(fn, inputs, params, grad_inputs, G, flush=True):
    """``out.backward(G)`` alone: each iteration first rebuilds the forward
    graph on fresh leaf copies, outside the timed region."""
    def fresh_graph():
        leaves = {k: v.detach().clone().requires_grad_(k in grad_inputs)
                  for k, v in inputs.items()}
        out = fn(leaves, params)
        return lambda: out.backward(G)
    return until_stable("backward", lambda: time_ms(None, flush=flush, setup=fresh_graph))


def compare(case, candidate, device=None, seed=0, baseline="compile", flush=True):
    """Time candidate vs baseline; returns (report_str, passed) like the reference."""
    p = PROTOCOL
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    assert str(device).startswith("cuda"), "timing needs the GPU"
    dtype = dtype_of(case.dtype)

    inputs = {k: v.to(device) for k, v in
              case.make_inputs(seed, dtype, "cpu", requires_grad=False).items()}
    with torch.no_grad():
        out = candidate(inputs, case.params)
    g = torch.Generator(device="cpu").manual_seed(777)
    G = torch.randn(out.shape, dtype=out.dtype, generator=g).to(device)

    base_fn = torch.compile(case.reference_forward) if baseline == "compile" \
        else case.reference_forward
    base_name = "baseline(torch.compile)" if baseline == "compile" else "baseline(eager)"

    lines = [f"=== timing: case={case.name} (HIP events, geomean, flush={flush}) ===",
             f"grad_inputs={case.grad_inputs} params={case.params} dtype={case.dtype}"]
    results = {}
    with_bwd = len(case.grad_inputs) > 0
    for name, fn in [(base_name, base_fn), ("candidate", candidate)]:
        fres = time_forward(fn, inputs, case.params, flush)
        bres = time_backward(fn, inputs, case.params, case.grad_inputs, G, flush) \
            if with_bwd else None
        results[name] = (fres, bres)
        lines.append(f"\n[{name}]")
        for t in (fres, bres):
            if t is not None:
                lines.append(f"  {t.label:<8}: {t.center_ms:.4f} ms  CV={t.cv * 100:.2f}%  "
                             f"x{t.tries}  {'ok' if t.stable else 'CV over threshold'}")

    bf, bb = results[base_name]
    cf, cb = results["candidate"]
    fwd_speedup = bf.center_ms / cf.center_ms
    lines.append("\n[speedup candidate vs baseline]")
    lines.append(f"  forward : {fwd_speedup:.4f}x  (target >={p.speedup_target}x) "
                 f"{'PASS' if fwd_speedup >= p.speedup_target else 'FAIL'}")
    passed = fwd_speedup >= p.speedup_target
    cvs = [bf, cf]
    if with_bwd:
        bwd_speedup = bb.center_ms / cb.center_ms
        lines.append(f"  backward: {bwd_speedup:.4f}x  (target >={p.speedup_target}x) "
                     f"{'PASS' if bwd_speedup >= p.speedup_target else 'FAIL'}")
        passed = passed and bwd_speedup >= p.speedup_target
        cvs += [bb, cb]
    cv_ok = all(r.stable for r in cvs)
    passed = passed and cv_ok
    if not cv_ok:
        lines.append("  CV > 5% present: result invalid, re-measure")
    lines.append(f"\n=== verdict: {'PASS' if passed else 'FAIL'} ===")
    return "\n".join(lines), passed


def parse_verdict(report, passed):
    """One-line machine-readable summary, same grammar as the reference's
    bench_case.py:_parse_verdict (skill/scripts/bench_case.py:33-54):
    ``VERDICT=<PASS|BENCH_FAIL|CV_INVALID> fwd=<x>x bwd=<x>x cv_ok=<0|1>``."""
    import re
    sp = dict(re.findall(r"(forward|backward)\s*:\s*([0-9.]+)x\s*\(target", report))
    cv_ok = 0 if "CV > 5% present" in report else 1
    verdict = "CV_INVALID" if cv_ok == 0 else ("PASS" if passed else "BENCH_FAIL")
    return f"VERDICT={verdict} fwd={sp.get('forward', '?')}x bwd={sp.get('backward', '?')}x cv_ok={cv_ok}"
