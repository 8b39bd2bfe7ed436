"""Softmax cross-entropy parity on the GPU (through the HIP library) against
the float64 oracle: the reference default [8192, 1024] and a large
vocabulary [4096, 8192] (logits ~ N(0, 1), labels uniform), every
row-cached width class with full and ragged rows, the generic path (C not a
multiple of 4, misaligned logits, C > 8192), batches that leave the last
workgroup short, large-magnitude logits, an upstream gradient other than 1,
an out-of-range label (NaN, as documented), an empty batch (NaN loss), a
bitwise-repeatable loss, and the framework's verify_all at the reference
defaults.

Tolerances: loss and lse at atol = rtol = 1e-3.  dlogits is of order
1 / B, so it is compared after scaling by B / gout (that is, as
softmax - onehot) at atol = rtol = 1e-3, and unscaled with a relative bound
of 1e-4 of its largest entry."""

import math

import numpy as np
import pytest
import torch

from conftest import announce
from framework.verify import verify_all
from oracle import softmax_ce as osc

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _read_trip_counter(monkeypatch):
    """Every forward through op.py zeroes the workspace's trip counter first
    and reads it after, raising if workgroup 0's wait hit its spin cap."""
    monkeypatch.setenv("NL2K_CHECK", "1")


def _inputs(b, c, seed, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(b, c, generator=gen) * scale
    labels = torch.randint(0, c, (b,), generator=gen)
    return logits, labels


def _close(name, got, ref, atol=1e-3, rtol=1e-3):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    print(f"  {name}: max_abs={max_abs:.3e}")
    assert np.all(err <= atol + rtol * np.abs(ref)), f"{name}: max_abs {max_abs:.3e}"


def _check(logits, labels, gout=1.0, ldev=None):
    from cases.softmax_ce import op
    xd = (logits.cuda() if ldev is None else ldev).requires_grad_(True)
    loss = op.candidate({"logits": xd, "labels": labels.cuda()}, {})
    loss.backward(torch.tensor(gout, device="cuda"))
    _, lse = op.sce_forward(xd.detach(), labels.cuda())
    torch.cuda.synchronize()
    x, lab = logits.double().numpy(), labels.numpy()
    rloss, rlse = osc.forward_f64(x, lab)
    _close("loss", [loss.item()], [rloss])
    _close("lse", lse.cpu().numpy(), rlse)
    rd = osc.backward_f64(x, lab, gout)
    got = xd.grad.cpu().double().numpy()
    B = x.shape[0]
    _close("dlogits*B/gout", got * B / gout, rd * B / gout)
    if rd.size:
        # C = 1 has an all-zero gradient: the bound is then exact equality
        err, top = float(np.abs(got - rd).max()), float(np.abs(rd).max())
        print(f"  dlogits max_abs={err:.3e} (largest entry {top:.3e})")
        assert err <= 1e-4 * top
    return loss.detach()


@pytest.mark.parametrize("b,c,seed", [(8192, 1024, 0), (4096, 8192, 1)])
def test_softmax_ce_bench_shapes(b, c, seed):
    announce(f"softmax_ce [{b}, {c}] seed={seed}")
    _check(*_inputs(b, c, seed))


# width classes of the row-cached forward: C/4 <= 64, <= 256 (one wave per
# row), <= 512, <= 1024, <= 2048 (a workgroup per row), each full and ragged;
# then the one-pass workgroup-per-row kernel (C % 4 != 0, C > 8192; float4
# or scalar loads) and the lane-per-row kernel (C <= 8, 16, 32)
@pytest.mark.parametrize("b,c", [(37, 4), (100, 100), (64, 256), (70, 1000), (5, 1024),
                                 (33, 1500), (16, 2048), (9, 3000), (12, 4096), (7, 6000),
                                 (3, 8192), (1, 1), (20, 7), (6, 8196), (4, 12000),
                                 (1000, 32000), (33, 50257), (5, 128256), (4000, 10), (70, 32),
                                 (300, 17), (64, 33), (1025, 8), (2, 2), (4097, 64), (999, 128),
                                 (130, 96), (50, 12)])
def test_softmax_ce_shapes(b, c):
    announce(f"softmax_ce [{b}, {c}]")
    _check(*_inputs(b, c, b + c))


@pytest.mark.parametrize("b", [1, 1023, 1025, 5000, 20000])
def test_softmax_ce_ragged_batches(b):
    announce(f"softmax_ce [{b}, 256] (last workgroup short)")
    _check(*_inputs(b, 256, b))


def test_softmax_ce_gout_large_logits_misaligned():
    announce("softmax_ce gout = -0.37, logits * 50, misaligned logits")
    logits, labels = _inputs(300, 512, 3)
    _check(logits, labels, gout=-0.37)
    _check(logits * 50.0, labels)
    buf = torch.empty(logits.numel() + 1, device="cuda")
    buf[1:].copy_(logits.reshape(-1).cuda())
    _check(logits, labels, ldev=buf[1:].view(300, 512))


def test_softmax_ce_out_of_range_label_gives_nan():
    announce("softmax_ce label = C and label = -1 -> NaN")
    from cases.softmax_ce import op
    logits, labels = _inputs(64, 1024, 4)
    for bad in (1024, -1):
        lab = labels.clone()
        lab[10] = bad
        loss, lse = op.sce_forward(logits.cuda(), lab.cuda())
        d = op.sce_backward(logits.cuda(), lab.cuda(), lse, torch.ones(1, device="cuda"))
        torch.cuda.synchronize()
        assert math.isnan(loss.item())
        assert torch.isnan(d[10]).all() and not torch.isnan(d[11]).any()


def test_softmax_ce_empty_batch():
    announce("softmax_ce B = 0")
    from cases.softmax_ce import op
    logits, labels = _inputs(0, 64, 5)
    loss, lse = op.sce_forward(logits.cuda(), labels.cuda())
    d = op.sce_backward(logits.cuda(), labels.cuda(), lse, torch.ones(1, device="cuda"))
    torch.cuda.synchronize()
    assert math.isnan(loss.item()) and lse.shape == (0,) and d.shape == (0, 64)


def test_softmax_ce_loss_deterministic():
    announce("softmax_ce loss bitwise repeatable")
    logits, labels = _inputs(8192, 1024, 6)
    first = _check(logits, labels)
    again = _check(logits, labels)
    assert torch.equal(first, again)


def test_softmax_ce_workspace_contents_never_taken():
    """The forward's partial losses travel through nonce-tagged slots in the
    caller's workspace: a workspace full of random bits, then the same one
    reused by a second call on other logits, must give each call its own
    loss (the oracle's, and bit for bit a fresh workspace's)."""
    announce("softmax_ce forward on a random-filled, then reused, workspace")
    from framework import capi
    from cases.softmax_ce import op
    lib = op._lib()
    b, c = 8192, 1024
    need = lib.softmax_ce_forward_workspace_bytes(b, c)
    ws = torch.randint(-2**62, 2**62, (need // 8,), dtype=torch.int64,
                       generator=torch.Generator().manual_seed(3)).cuda()
    s = capi.stream_of(ws)
    for seed in (11, 12):
        logits, labels = _inputs(b, c, seed)
        x, lab = logits.cuda(), labels.cuda()
        loss = torch.empty(1, device="cuda")
        lse = torch.empty(b, device="cuda")
        st = lib.softmax_ce_forward_f32(capi.ptr(x), capi.ptr(lab), capi.ptr(loss), capi.ptr(lse),
                                        b, c, capi.ptr(ws), need, s)
        capi.check(st, lib.softmax_ce_last_error, "softmax_ce_forward")
        fresh, _ = op.sce_forward(x, lab)
        torch.cuda.synchronize()
        ref_loss, _ = osc.forward_f64(logits.numpy(), labels.numpy())
        _close("loss", loss.cpu(), np.array([ref_loss]))
        assert torch.equal(loss, fresh.reshape(1))


def test_softmax_ce_verify_all_reference_defaults():
    announce("softmax_ce verify_all (reference defaults [8192, 1024])")
    from cases.softmax_ce import CASE, op
    ok, report = verify_all(CASE, op.candidate, device="cuda")
    print(report)
    assert ok, report
