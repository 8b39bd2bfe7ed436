"""Parity harness: checks a candidate against the case's reference.

Same procedure as the reference's framework/verify.py:35-105:
  * forward: for every seed, allclose(candidate, reference) plus max abs error;
  * backward: same seed, upstream G = randn(out.shape) from seed + 10000,
    allclose of every grad input's gradient.

Differences, all required by this build's acceptance bar:
  * atol = rtol = 1e-3 (PROTOCOL), and the max relative error is reported
    next to the max absolute error;
  * inputs and G are drawn once on the host (CPU generator) and copied to the
    candidate's device, so the reference and the candidate see identical
    tensors; the reference runs on ``ref_device`` (default "cpu", the
    reference's PyTorch CPU path);
  * integer outputs are compared for exact equality (after casting both sides
    to int64, since torch.cumsum of int32 returns int64).
"""

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import torch  # noqa: E402

from framework.protocol import PROTOCOL, dtype_of  # noqa: E402


def _clone_requires_grad(inputs, grad_inputs, device=None):
    out = {}
    for k, v in inputs.items():
        t = v.detach().clone()
        if device is not None:
            t = t.to(device)
        if k in grad_inputs:
            t.requires_grad_(True)
        out[k] = t
    return out


def compare_tensors(got, ref, atol=None, rtol=None):
    """Returns (ok, max_abs, max_rel) of ``got`` against ``ref`` (on CPU)."""
    p = PROTOCOL
    atol = p.atol if atol is None else atol
    rtol = p.rtol if rtol is None else rtol
    got = got.detach().to("cpu")
    ref = ref.detach().to("cpu")
    if got.shape != ref.shape:
        return False, float("inf"), float("inf")
    if not ref.dtype.is_floating_point:
        g, r = got.to(torch.int64), ref.to(torch.int64)
        diff = (g - r).abs()
        m = diff.max().item() if diff.numel() else 0
        return bool(torch.equal(g, r)), float(m), float(m)
    g, r = got.to(torch.float64), ref.to(torch.float64)
    if g.numel() == 0:
        return True, 0.0, 0.0
    diff = (g - r).abs()
    # torch.allclose's rule (the reference's check): |g - r| <= atol + rtol |r|,
    # equal infinities close, NaN never close.
    ok = bool(torch.isclose(g, r, rtol=rtol, atol=atol).all().item())
    max_abs = torch.nan_to_num(diff, nan=0.0).max().item()
    rel = diff / r.abs().clamp_min(1e-30)
    max_rel = torch.nan_to_num(rel, nan=0.0, posinf=0.0).max().item()
    return ok, max_abs, max_rel


def _upstream(shape, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, dtype=dtype, generator=g)


def verify_forward(case, impl, device="cuda", ref_device="cpu"):
    """Forward parity over PROTOCOL.seeds: (ok, [(seed, ok, max_abs, max_rel)])."""
    p = PROTOCOL
    dtype = dtype_of(case.dtype)
    results = []
    for seed in p.seeds:
        base = case.make_inputs(seed, dtype, "cpu", requires_grad=False)
        ref_in = {k: v.to(ref_device) for k, v in base.items()}
        imp_in = {k: v.to(device) for k, v in base.items()}
        with torch.no_grad():
            out_ref = case.reference_forward(ref_in, case.params)
            out_imp = impl(imp_in, case.params)
        if device != "cpu" and str(device).startswith("cuda"):
            torch.cuda.synchronize()
        ok, max_abs, max_rel = compare_tensors(out_imp, out_ref)
        results.append((seed, ok, max_abs, max_rel))
    return all(r[1] for r in results), results


def verify_backward(case, impl, device="cuda", ref_device="cpu"):
    """Backward parity: (ok, [(seed, ok, {name: (max_abs, max_rel)})])."""
    p = PROTOCOL
    dtype = dtype_of(case.dtype)
    results = []
    for seed in p.seeds:
        base = case.make_inputs(seed, dtype, "cpu", requires_grad=False)

        ref_in = _clone_requires_grad(base, case.grad_inputs, ref_device)
        out_ref = case.reference_forward(ref_in, case.params)
        G = _upstream(out_ref.shape, out_ref.dtype, seed + 10_000)
        out_ref.backward(G.to(ref_device))
        ref_grads = {k: ref_in[k].grad.detach().clone() for k in case.grad_inputs}

        imp_in = _clone_requires_grad(base, case.grad_inputs, device)
        out_imp = impl(imp_in, case.params)
        out_imp.backward(G.to(device))
        if str(device).startswith("cuda"):
            torch.cuda.synchronize()

        per_ok, per_err = {}, {}
        for k in case.grad_inputs:
            ok, max_abs, max_rel = compare_tensors(imp_in[k].grad, ref_grads[k])
            per_ok[k] = ok
            per_err[k] = (max_abs, max_rel)
        results.append((seed, all(per_ok.values()), per_err))
    return all(r[1] for r in results), results


def verify_all(case, impl, device=None, ref_device="cpu", backward=None):
    """Full parity run; returns (ok, report_str) like the reference."""
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    if backward is None:
        backward = len(case.grad_inputs) > 0
    lines = [f"=== parity: case={case.name} (device={device}, reference on {ref_device}) ===",
             f"grad_inputs={case.grad_inputs} params={case.params} dtype={case.dtype} "
             f"atol={PROTOCOL.atol} rtol={PROTOCOL.rtol}"]

    fwd_ok, fwd = verify_forward(case, impl, device, ref_device)
    lines.append(f"\n[forward] {'PASS' if fwd_ok else 'FAIL'}")
    for seed, ok, a, r in fwd:
        lines.append(f"  seed={seed}: {'ok' if ok else 'X'}  max_abs_err={a:.3e}  max_rel_err={r:.3e}")

    overall = fwd_ok
    if backward:
        bwd_ok, bwd = verify_backward(case, impl, device, ref_device)
        lines.append(f"\n[backward] {'PASS' if bwd_ok else 'FAIL'}")
        for seed, ok, errs in bwd:
            errstr = " ".join(f"d{k}_abs={a:.3e} d{k}_rel={r:.3e}" for k, (a, r) in errs.items())
            lines.append(f"  seed={seed}: {'ok' if ok else 'X'}  {errstr}")
        overall = overall and bwd_ok

    lines.append(f"\n=== overall: {'PASS' if overall else 'FAIL'} ===")
    return overall, "\n".join(lines)
