"""L2-norm-scale parity on the GPU (through the HIP library) against the
float64 oracle at atol = rtol = 1e-3: the reference default [16384, 1024]
and the LayerNorm acceptance shape [8192, 4096] (X, g, dY ~ N(0, 1)), every
row-cached width class, the generic path (odd D, misaligned X, D > 8192),
zero rows, a large eps, an empty batch, deterministic dg, and the
framework's verify_all at the reference defaults."""

import numpy as np
import pytest
import torch

from conftest import announce
from framework.verify import verify_all
from oracle import l2norm_scale as ol

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _inputs(n, d, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=gen)
    g = torch.randn(d, generator=gen)
    dy = torch.randn(n, d, generator=torch.Generator().manual_seed(seed + 10_000))
    return x, g, dy


def _close(name, got, ref, atol=1e-3, rtol=1e-3):
    got = got.detach().cpu().double().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    print(f"  {name}: max_abs={max_abs:.3e}")
    assert np.all(err <= atol + rtol * np.abs(ref)), f"{name}: max_abs {max_abs:.3e}"


def _check(x, g, dy, eps=EPS, xdev=None):
    from cases.l2norm_scale import op
    xd = (x.cuda() if xdev is None else xdev).requires_grad_(True)
    gd = g.cuda().requires_grad_(True)
    y = op.candidate({"X": xd, "g": gd}, {"eps": eps})
    y.backward(dy.cuda())
    _, norm = op.l2n_forward(xd.detach(), gd.detach(), eps)
    torch.cuda.synchronize()
    xn, gn, dyn = x.double().numpy(), g.double().numpy(), dy.double().numpy()
    ry, rn = ol.forward_f64(xn, gn, eps)
    _close("y", y, ry)
    _close("norm", norm, rn)
    rdx, rdg = ol.backward_f64(xn, gn, dyn, eps)
    _close("dX", xd.grad, rdx)
    _close("dg", gd.grad, rdg)
    return gd.grad


@pytest.mark.parametrize("n,d,seed", [(16384, 1024, 0), (8192, 4096, 1)])
def test_l2norm_bench_shapes(n, d, seed):
    announce(f"l2norm_scale [{n}, {d}] seed={seed}")
    _check(*_inputs(n, d, seed))


@pytest.mark.parametrize("n,d", [(5, 4), (33, 64), (17, 100), (300, 256), (64, 1000),
                                 (40, 1024), (9, 2048), (3, 8192), (2, 8196), (7, 12000),
                                 (1, 1), (4099, 1000), (2050, 4100), (4097, 4096),
                                 (3, 2048), (513, 1028), (4097, 8192), (1000, 6000),
                                 (4099, 512), (2050, 300),
                                 (16385, 64), (1000, 128), (4097, 96), (4099, 600),
                                 (1030, 768), (5, 16384),
                                 (33, 12288), (3, 20000)])
def test_l2norm_shapes(n, d):
    announce(f"l2norm_scale [{n}, {d}]")
    _check(*_inputs(n, d, n + d))


def test_l2norm_zero_rows_large_eps_misaligned():
    announce("l2norm_scale zero rows, eps = 0.5, misaligned X")
    x, g, dy = _inputs(200, 512, 3)
    x[5] = 0.0
    _check(x, g, dy)
    _check(x, g, dy, eps=0.5)
    buf = torch.empty(x.numel() + 1, device="cuda")
    buf[1:].copy_(x.reshape(-1).cuda())
    _check(x, g, dy, xdev=buf[1:].view(200, 512))


def test_l2norm_empty_batch():
    announce("l2norm_scale N = 0")
    from cases.l2norm_scale import op
    x, g, dy = _inputs(0, 64, 4)
    y, norm = op.l2n_forward(x.cuda(), g.cuda(), EPS)
    dx, dg = op.l2n_backward(x.cuda(), g.cuda(), dy.cuda(), norm)
    torch.cuda.synchronize()
    assert y.shape == (0, 64) and torch.all(dg == 0)


def test_l2norm_dg_deterministic():
    announce("l2norm_scale dg bitwise repeatable")
    x, g, dy = _inputs(4096, 1024, 5)
    first = _check(x, g, dy).clone()
    again = _check(x, g, dy)
    assert torch.equal(first, again)


def test_l2norm_verify_all_reference_defaults():
    announce("l2norm_scale verify_all (reference defaults [16384, 1024])")
    from cases.l2norm_scale import CASE, op
    ok, report = verify_all(CASE, op.candidate, device="cuda")
    print(report)
    assert ok, report
