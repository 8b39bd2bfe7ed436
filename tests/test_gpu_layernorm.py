"""LayerNorm parity on the GPU (through the HIP library) against the float64
oracle at atol = rtol = 1e-3: the acceptance workload x [8192, 4096]
(gamma = 1 + 0.1 N, beta = 0.1 N), every row-cached width class, the generic
path (odd D, misaligned pointers, D > 8192), empty batches, and the
framework's verify_all against the case's reference."""

import numpy as np
import pytest
import torch

from conftest import announce
from framework.verify import verify_all
from oracle import layernorm as oln

pytestmark = pytest.mark.gpu
EPS = 1e-5


def _inputs(b, d, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, d, generator=g)
    w = 1 + 0.1 * torch.randn(d, generator=g)
    bias = 0.1 * torch.randn(d, generator=g)
    dy = torch.randn(b, d, generator=torch.Generator().manual_seed(seed + 10_000))
    return x, w, bias, dy


def _close(name, got, ref, atol=1e-3, rtol=1e-3):
    got = got.detach().cpu().double().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    print(f"  {name}: max_abs={max_abs:.3e}")
    assert np.all(err <= atol + rtol * np.abs(ref)), f"{name}: max_abs {max_abs:.3e}"


def _run(x, w, bias, dy, xdev=None):
    from cases.layernorm import op
    xd = (x.cuda() if xdev is None else xdev).requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    bd = bias.cuda().requires_grad_(True)
    y = op.candidate({"X": xd, "gamma": wd, "beta": bd}, {"eps": EPS})
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    return y.detach(), xd.grad, wd.grad, bd.grad


def _check(x, w, bias, dy, xdev=None):
    y, dx, dw, db = _run(x, w, bias, dy, xdev)
    ry, _, _ = oln.forward_f64(x.numpy(), w.numpy(), bias.numpy(), EPS)
    rdx, rdw, rdb = oln.backward_f64(dy.numpy(), x.numpy(), w.numpy(), EPS)
    _close("y", y, ry)
    _close("dx", dx, rdx)
    _close("dgamma", dw, rdw)
    _close("dbeta", db, rdb)


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_layernorm_baseline_8192x4096(seed):
    announce(f"layernorm 8192x4096 seed={seed}")
    _check(*_inputs(8192, 4096, seed))


@pytest.mark.parametrize("b,d", [(5, 4), (33, 64), (17, 100), (300, 256), (64, 1000),
                                 (4096, 1024), (100, 2048), (7, 8192), (3, 8196), (9, 10000),
                                 (1, 1), (2, 3), (1025, 1537), (4099, 1000), (2050, 4100),
                                 (4097, 4096), (3, 2048), (513, 1028), (4097, 8192),
                                 (1000, 6000), (33, 4100),
                                 (4099, 512), (2050, 300), (16384, 256),
                                 (16385, 64), (1000, 128), (4097, 96), (3, 128), (70, 8),
                                 (4099, 600), (1030, 768), (257, 1020),
                                 (5, 16384), (33, 12288), (2, 16380), (700, 10000), (3, 20000)])
def test_layernorm_shapes(b, d):
    announce(f"layernorm b={b} d={d}")
    _check(*_inputs(b, d, b + d))


def test_layernorm_misaligned_input():
    announce("layernorm misaligned")
    x, w, bias, dy = _inputs(40, 256, 7)
    buf = torch.empty(40 * 256 + 1, device="cuda")
    buf[1:].copy_(x.reshape(-1).cuda())
    _check(x, w, bias, dy, xdev=buf[1:].view(40, 256))


def test_layernorm_empty_batch():
    announce("layernorm B=0")
    from cases.layernorm import op
    x = torch.zeros(0, 64, device="cuda")
    w = torch.ones(64, device="cuda")
    b = torch.zeros(64, device="cuda")
    y, mean, rstd = op.layernorm_forward(x, w, b, EPS)
    assert y.shape == (0, 64)
    dx, dw, db = op.layernorm_backward(torch.zeros(0, 64, device="cuda"), x, w, mean, rstd)
    torch.cuda.synchronize()
    assert dx.shape == (0, 64) and torch.all(dw == 0) and torch.all(db == 0)


def test_layernorm_constant_rows():
    announce("layernorm constant rows")
    x = torch.full((8, 512), 3.0)
    w = torch.ones(512)
    b = torch.linspace(-1, 1, 512)
    dy = torch.randn(8, 512, generator=torch.Generator().manual_seed(3))
    _check(x, w, b, dy)


@pytest.mark.parametrize("b,d", [(64, 4096), (96, 1024), (70, 64)])
def test_layernorm_nan_row_stays_in_its_row(b, d):
    """A NaN in one row of x makes that row of y and dx NaN (its mean and
    variance are NaN, as in torch's layer_norm) and, through the column sums,
    every element of dgamma; dbeta does not involve x and stays finite.
    The other rows match the oracle."""
    announce(f"layernorm NaN row [{b},{d}]")
    x, w, bias, dy = _inputs(b, d, 31)
    x[5, 17] = float("nan")
    y, dx, dw, db = _run(x, w, bias, dy)
    yc, dxc = y.cpu(), dx.cpu()
    assert torch.isnan(yc[5]).all() and torch.isnan(dxc[5]).all()
    assert not torch.isnan(torch.cat([yc[:5], yc[6:]])).any()
    assert not torch.isnan(torch.cat([dxc[:5], dxc[6:]])).any()
    assert torch.isnan(dw.cpu()).all() and not torch.isnan(db.cpu()).any()
    keep = [i for i in range(b) if i != 5]
    xk = x[keep]
    ry, _, _ = oln.forward_f64(xk.numpy(), w.numpy(), bias.numpy(), EPS)
    rdx, _, rdb = oln.backward_f64(dy[keep].numpy(), xk.numpy(), w.numpy(), EPS)
    _close("y (other rows)", yc[keep], ry)
    _close("dx (other rows)", dxc[keep], rdx)
    _close("dbeta", db, rdb + dy[5].double().numpy())


def test_layernorm_param_grads_deterministic():
    announce("layernorm repeatability")
    x, w, bias, dy = _inputs(2048, 4096, 11)
    a = _run(x, w, bias, dy)
    b = _run(x, w, bias, dy)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_layernorm_verify_all_reference_defaults():
    announce("layernorm verify_all (reference defaults 4096x1024)")
    from cases.layernorm import CASE, op
    ok, report = verify_all(CASE, op.candidate, device="cuda")
    print(report)
    assert ok, report
