"""Pins the LayerNorm oracle (CPU only)."""

import math

import numpy as np
import pytest
import torch

from oracle import layernorm as oln
from oracle import native


def _inputs(b, d, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, d)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    bb = (0.1 * rng.standard_normal(d)).astype(np.float32)
    dy = rng.standard_normal((b, d)).astype(np.float32)
    return x, w, bb, dy


def test_forward_known_values():
    y, mean, rstd = oln.forward_f64([[1.0, 2.0, 3.0]], [1.0, 1.0, 1.0], [0.0, 0.0, 0.0], 0.0)
    s = math.sqrt(1.5)
    np.testing.assert_allclose(y, [[-s, 0.0, s]], rtol=1e-14)
    assert mean[0] == 2.0 and abs(rstd[0] - math.sqrt(1.5)) < 1e-14
    y2, _, _ = oln.forward_f64([[1.0, 2.0, 3.0]], [2.0, 1.0, 1.0], [1.0, 0.5, 0.0], 0.0)
    np.testing.assert_allclose(y2, [[-2 * s + 1.0, 0.5, s]], rtol=1e-14)
    # constant row: variance 0, output = bias (xhat = 0 for any eps > 0)
    y3, _, _ = oln.forward_f64([[5.0, 5.0]], [3.0, 3.0], [0.25, -1.0], 1e-5)
    np.testing.assert_allclose(y3, [[0.25, -1.0]], atol=1e-12)


def test_forward_vs_c_and_torch():
    x, w, b, _ = _inputs(37, 129)
    y, mean, rstd = oln.forward_f64(x, w, b, 1e-5)
    cy, cm, cr = native.layernorm_forward(x, w, b, 1e-5)
    np.testing.assert_allclose(y, cy, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mean, cm, rtol=1e-12, atol=1e-14)
    ty = oln.torch_cpu_forward(*(torch.tensor(a, dtype=torch.float64) for a in (x, w, b)), 1e-5)
    np.testing.assert_allclose(y, ty.numpy(), rtol=1e-12, atol=1e-12)


def test_backward_vs_finite_differences():
    x, w, b, dy = _inputs(3, 5, seed=1)
    dx, dw, db = oln.backward_f64(dy, x, w, 1e-5)
    fx, fw, fb = oln.finite_difference_grads(x, w, b, dy, 1e-5)
    np.testing.assert_allclose(dx, fx, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(dw, fw, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(db, fb, rtol=1e-5, atol=1e-7)


def test_backward_vs_torch_autograd_f64():
    x, w, b, dy = _inputs(16, 64, seed=2)
    t = [torch.tensor(a, dtype=torch.float64) for a in (x, w, b, dy)]
    tx, tw, tb = oln.torch_cpu_backward(t[0], t[1], t[2], t[3], 1e-5)
    dx, dw, db = oln.backward_f64(dy, x, w, 1e-5)
    np.testing.assert_allclose(dx, tx.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, tb.numpy(), rtol=1e-10, atol=1e-12)


def test_backward_identities():
    x, w, b, dy = _inputs(20, 96, seed=3)
    dx, dw, db = oln.backward_f64(dy, x, w, 1e-5)
    np.testing.assert_allclose(dx.sum(axis=1), 0.0, atol=1e-12)  # shift invariance of each row
    np.testing.assert_allclose(db, dy.astype(np.float64).sum(axis=0), rtol=1e-14)


def _bad_no_xhat_term(dy, x, w, eps):
    dx, dw, db = oln.backward_f64(dy, x, w, eps)
    _, mean, rstd = oln.forward_f64(x, w, np.zeros_like(w), eps)
    g = np.asarray(dy, np.float64) * w
    return rstd[:, None] * (g - g.mean(axis=-1, keepdims=True)), dw, db


def _bad_unbiased_var(dy, x, w, eps):
    x = np.asarray(x, np.float64)
    d = x.shape[1]
    return oln.backward_f64(dy, x * math.sqrt(d / (d - 1)), w, eps)


def _bad_swapped_params(dy, x, w, eps):
    dx, dw, db = oln.backward_f64(dy, x, w, eps)
    return dx, db, dw


@pytest.mark.parametrize("bad", [_bad_no_xhat_term, _bad_unbiased_var, _bad_swapped_params])
def test_planted_mistakes_are_caught(bad):
    x, w, b, dy = _inputs(3, 5, seed=4)
    fx, fw, fb = oln.finite_difference_grads(x, w, b, dy, 1e-5)
    bx, bw, bb = bad(dy, x, w, 1e-5)
    ok = (np.allclose(bx, fx, rtol=1e-5, atol=1e-7) and np.allclose(bw, fw, rtol=1e-5, atol=1e-7)
          and np.allclose(bb, fb, rtol=1e-5, atol=1e-7))
    assert not ok
