"""Pins oracle/softmax_ce.py (CPU only): closed forms, brute force, float64
torch autograd of the reference expression, finite differences, invariants,
logits near the float32 limits, and planted mistakes that must fail."""

import math

import numpy as np
import pytest
import torch

from oracle import softmax_ce as osc


def _case(b, c, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((b, c)) * scale, rng.integers(0, c, b)


def _torch_ref(x, lab, gout):
    # the reference expression (cases/softmax_ce/reference.py:18-21) in float64
    xt = torch.tensor(x, requires_grad=True)
    logp = xt - torch.logsumexp(xt, dim=-1, keepdim=True)
    loss = (-logp.gather(1, torch.tensor(lab).unsqueeze(1)).squeeze(1)).mean()
    loss.backward(torch.tensor(gout, dtype=torch.float64))
    return loss.item(), xt.grad.numpy()


def test_closed_forms():
    # equal logits: every class has probability 1/C, so the loss is log C
    for c in (1, 2, 7, 1024):
        loss, lse = osc.forward_f64(np.full((3, c), 2.5), [0, c - 1, c // 2])
        assert math.isclose(loss, math.log(c), abs_tol=1e-12)
        assert np.allclose(lse, 2.5 + math.log(c))
    # two classes: loss = softplus(other - own)
    x = np.array([[0.3, -1.2], [4.0, 1.0]])
    loss, _ = osc.forward_f64(x, [0, 1])
    want = (math.log1p(math.exp(-1.5)) + math.log1p(math.exp(3.0))) / 2
    assert math.isclose(loss, want, rel_tol=1e-14)
    # gradient of equal logits: (1/C - onehot) / B
    d = osc.backward_f64(np.zeros((2, 4)), [1, 3])
    assert np.allclose(d, [[0.125, -0.375, 0.125, 0.125], [0.125, 0.125, 0.125, -0.375]])


def test_brute_force():
    x, lab = _case(5, 9, 1, scale=3.0)
    assert math.isclose(osc.forward_f64(x, lab)[0], osc.forward_loops(x, lab), rel_tol=1e-13)


@pytest.mark.parametrize("gout", [1.0, -0.75])
def test_matches_torch_autograd(gout):
    x, lab = _case(16, 37, 2, scale=4.0)
    loss, grad = _torch_ref(x, lab, gout)
    assert math.isclose(osc.forward_f64(x, lab)[0], loss, rel_tol=1e-13)
    assert np.allclose(osc.backward_f64(x, lab, gout), grad, atol=1e-15)


def test_finite_differences():
    x, lab = _case(3, 6, 3)
    h, gout = 1e-6, 0.8
    num = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        p, m = x.copy(), x.copy()
        p[idx] += h
        m[idx] -= h
        num[idx] = gout * (osc.forward_f64(p, lab)[0] - osc.forward_f64(m, lab)[0]) / (2 * h)
    assert np.allclose(osc.backward_f64(x, lab, gout), num, atol=1e-9)


def test_invariants():
    x, lab = _case(11, 50, 4, scale=2.0)
    loss, lse = osc.forward_f64(x, lab)
    shifted = x + np.random.default_rng(5).standard_normal(11)[:, None] * 30
    assert math.isclose(osc.forward_f64(shifted, lab)[0], loss, rel_tol=1e-12)
    d = osc.backward_f64(x, lab, 1.0)
    assert np.allclose(d.sum(axis=1), 0.0, atol=1e-15)
    assert np.allclose(np.exp(x - lse[:, None]).sum(axis=1), 1.0)
    assert np.all(d[np.arange(11), lab] < 0) and np.all(np.delete(d.ravel(), lab + 50 * np.arange(11)) > 0)


def test_extreme_logits():
    # near the float32 range: the max shift keeps exp finite
    x = np.array([[3.0e38, 0.0, -3.0e38], [-1.0e30, -1.0e30 + 1.0, -1.0e30]])
    loss, lse = osc.forward_f64(x, [0, 1])
    assert np.isfinite(loss) and np.allclose(lse, [3.0e38, -1.0e30 + 1.0 + math.log(1 + 2 * math.exp(-1.0))])


def _bad(kind, x, lab, gout):
    B = x.shape[0]
    if kind == "no_max_shift":
        lse = np.log(np.exp(x).sum(axis=1))
    else:
        lse = osc.lse_f64(x)
    p = np.exp(x - lse[:, None])
    sign = 1.0 if kind == "onehot_sign" else -1.0
    p[np.arange(B), (lab + 1) % x.shape[1] if kind == "label_shift" else lab] += sign
    if kind == "no_mean":
        return p * gout
    return p * gout / B


@pytest.mark.parametrize("kind", ["no_max_shift", "onehot_sign", "label_shift", "no_mean"])
def test_planted_mistakes_fail(kind):
    x, lab = _case(6, 12, 6, scale=2.0)
    x[0, 0] = 800.0  # overflows exp without the max shift
    _, grad = _torch_ref(x, lab, 0.5)
    with np.errstate(over="ignore", invalid="ignore"):
        bad = _bad(kind, x, lab, 0.5)
    assert not np.allclose(bad, grad, atol=1e-6)
    assert np.allclose(osc.backward_f64(x, lab, 0.5), grad, atol=1e-15)
