"""Pins oracle/l2norm_scale.py (CPU only): hand values, unit length, brute
force, float64 torch autograd of the reference expression, finite
differences, the x . dx identity, and planted mistakes that must fail."""

import numpy as np
import pytest
import torch

from oracle import l2norm_scale as ol


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def _torch_ref(x, g, dy, eps):
    xt = torch.tensor(x, requires_grad=True)
    gt = torch.tensor(g, requires_grad=True)
    norm = torch.sqrt((xt * xt).sum(dim=-1, keepdim=True) + eps)
    y = (xt / norm) * gt
    y.backward(torch.tensor(dy))
    return y.detach().numpy(), xt.grad.numpy(), gt.grad.numpy()


def test_hand_values_and_unit_length():
    y, n = ol.forward_f64([[3.0, 4.0], [0.0, 2.0]], [1.0, 10.0], 0.0)
    assert np.allclose(n, [5.0, 2.0])
    assert np.allclose(y, [[0.6, 8.0], [0.0, 10.0]])
    x = _rand((9, 33), 0)
    y, _ = ol.forward_f64(x, np.ones(33), 0.0)
    assert np.allclose((y * y).sum(axis=1), 1.0)


def test_brute_force():
    x, g = _rand((4, 6), 1), _rand(6, 2)
    assert np.allclose(ol.forward_f64(x, g, 1e-6)[0], ol.forward_loops(x, g, 1e-6), atol=1e-14)


@pytest.mark.parametrize("eps", [1e-6, 0.5])
def test_matches_torch_autograd(eps):
    x, g, dy = _rand((12, 20), 3), _rand(20, 4), _rand((12, 20), 5)
    y, dx, dg = _torch_ref(x, g, dy, eps)
    assert np.allclose(ol.forward_f64(x, g, eps)[0], y, atol=1e-14)
    gx, gg = ol.backward_f64(x, g, dy, eps)
    assert np.allclose(gx, dx, atol=1e-12)
    assert np.allclose(gg, dg, atol=1e-12)


def test_finite_differences():
    x, g, dy = _rand((3, 5), 6), _rand(5, 7), _rand((3, 5), 8)
    eps, h = 1e-3, 1e-6
    gx, gg = ol.backward_f64(x, g, dy, eps)
    for arr, grad, which in ((x, gx, 0), (g, gg, 1)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            p, m = arr.copy(), arr.copy()
            p[idx] += h
            m[idx] -= h
            fp = ol.forward_f64(p, g, eps)[0] if which == 0 else ol.forward_f64(x, p, eps)[0]
            fm = ol.forward_f64(m, g, eps)[0] if which == 0 else ol.forward_f64(x, m, eps)[0]
            num[idx] = ((fp - fm) * dy).sum() / (2 * h)
        assert np.allclose(grad, num, atol=1e-7)


def test_scale_invariance_identity():
    # y is invariant to scaling a row when eps = 0, so x . dx = 0 row by row
    x, g, dy = _rand((7, 16), 9), _rand(16, 10), _rand((7, 16), 11)
    dx, _ = ol.backward_f64(x, g, dy, 0.0)
    assert np.allclose((x * dx).sum(axis=1), 0.0, atol=1e-12)


def _bad(kind, x, g, dy, eps):
    if kind == "mean_not_sum":
        norm = np.sqrt((x * x).mean(axis=1) + eps)
    elif kind == "eps_outside":
        norm = np.sqrt((x * x).sum(axis=1)) + eps
    else:
        norm = np.sqrt((x * x).sum(axis=1) + eps)
    xh = x / norm[:, None]
    gd = dy * g[None, :]
    dot = (xh * gd).sum(axis=1)
    if kind == "no_projection":
        return gd / norm[:, None], (dy * xh).sum(axis=0)
    if kind == "dg_unnormalised":
        return (gd - xh * dot[:, None]) / norm[:, None], (dy * x).sum(axis=0)
    return (gd - xh * dot[:, None]) / norm[:, None], (dy * xh).sum(axis=0)


@pytest.mark.parametrize("kind", ["mean_not_sum", "eps_outside", "no_projection", "dg_unnormalised"])
def test_planted_mistakes_are_caught(kind):
    eps = 0.5
    x, g, dy = _rand((6, 8), 12), _rand(8, 13), _rand((6, 8), 14)
    _, dx, dg = _torch_ref(x, g, dy, eps)
    bx, bg = _bad(kind, x, g, dy, eps)
    assert not (np.allclose(bx, dx, atol=1e-6) and np.allclose(bg, dg, atol=1e-6)), kind
