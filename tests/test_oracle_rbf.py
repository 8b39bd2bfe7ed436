"""Pins the RBF oracle (CPU only).

Each check is chosen so that a plausible mistake in the oracle -- a dropped
row/column-sum term, a wrong sign or factor, a transposed operand -- fails at
least one of them; test_planted_mistakes_are_caught plants such mistakes in
copies of the oracle and checks that the pins reject them.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import native
from oracle import rbf as orbf

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rbf_ref_small.npz")


def _inputs(n, m, d, scale=0.125, seed=0):
    rng = np.random.default_rng(seed)
    X = (rng.standard_normal((n, d)) * scale).astype(np.float32)
    Y = (rng.standard_normal((m, d)) * scale).astype(np.float32)
    G = rng.standard_normal((n, m)).astype(np.float32)
    return X, Y, G


# ------------------------------------------------------------------ forward
def test_forward_known_values():
    X = np.array([[0.0, 0.0], [1.0, 2.0]])
    Y = np.array([[3.0, 4.0], [1.0, 2.0], [0.0, 0.0]])
    K = orbf.forward_f64(X, Y, 0.5)
    expect = np.array([[math.exp(-12.5), math.exp(-2.5), 1.0],
                       [math.exp(-4.0), 1.0, math.exp(-2.5)]])
    np.testing.assert_allclose(K, expect, rtol=1e-14, atol=0)


def test_forward_invariants():
    X, Y, _ = _inputs(31, 23, 64)
    K = orbf.forward_f64(X, Y, 0.5)
    assert np.all(K > 0) and np.all(K <= 1)
    np.testing.assert_allclose(orbf.forward_f64(Y, X, 0.5), K.T, rtol=1e-14)
    np.testing.assert_allclose(np.diag(orbf.forward_f64(X, X, 0.5)), 1.0, rtol=0, atol=1e-14)
    assert np.all(orbf.forward_f64(X, Y, 0.0) == 1.0)


def test_forward_closed_form_vs_bruteforce():
    for (n, m, d) in [(1, 1, 1), (5, 7, 3), (40, 33, 64), (17, 64, 100)]:
        X, Y, _ = _inputs(n, m, d, scale=0.3, seed=n)
        np.testing.assert_allclose(orbf.forward_f64(X, Y, 0.5),
                                   orbf.forward_bruteforce_f64(X, Y, 0.5), rtol=1e-12, atol=1e-15)


def test_forward_d1_by_hand():
    X = np.array([[0.5], [-1.0]])
    Y = np.array([[0.0], [2.0], [-1.5]])
    gamma = 0.25
    expect = [[math.exp(-gamma * (a - b) ** 2) for b in (0.0, 2.0, -1.5)] for a in (0.5, -1.0)]
    np.testing.assert_allclose(orbf.forward_f64(X, Y, gamma), expect, rtol=1e-14)


def test_c_oracle_matches_numpy_forward():
    X, Y, _ = _inputs(70, 45, 64)
    np.testing.assert_allclose(native.rbf_forward(X, Y, 0.5), orbf.forward_f64(X, Y, 0.5),
                               rtol=1e-12, atol=1e-15)


# ----------------------------------------------------------------- backward
def test_backward_vs_finite_differences():
    X, Y, G = _inputs(5, 7, 3, scale=0.5, seed=3)
    for gamma in (0.5, 1.0 / 64.0, 2.0):
        K = orbf.forward_f64(X, Y, gamma)
        dX, dY = orbf.backward_f64(X, Y, G, K, gamma)
        fX, fY = orbf.finite_difference_grads(X, Y, G, gamma)
        np.testing.assert_allclose(dX, fX, rtol=1e-6, atol=1e-8)
        np.testing.assert_allclose(dY, fY, rtol=1e-6, atol=1e-8)


def test_backward_vs_loops_and_c():
    X, Y, G = _inputs(6, 9, 4, scale=0.5, seed=4)
    K = orbf.forward_f64(X, Y, 0.5)
    dX, dY = orbf.backward_f64(X, Y, G, K, 0.5)
    lX, lY = orbf.backward_loops(X.tolist(), Y.tolist(), G.tolist(), K.tolist(), 0.5)
    np.testing.assert_allclose(dX, lX, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(dY, lY, rtol=1e-12, atol=1e-14)
    cX, cY = native.rbf_backward(X, Y, G, K, 0.5)
    np.testing.assert_allclose(dX, cX, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(dY, cY, rtol=1e-12, atol=1e-14)


def test_backward_vs_torch_autograd_f64():
    X, Y, G = _inputs(20, 13, 64, seed=5)
    Xt = torch.tensor(X, dtype=torch.float64, requires_grad=True)
    Yt = torch.tensor(Y, dtype=torch.float64, requires_grad=True)
    diff = Xt.unsqueeze(1) - Yt.unsqueeze(0)
    torch.exp(-0.5 * diff.pow(2).sum(-1)).backward(torch.tensor(G, dtype=torch.float64))
    K = orbf.forward_f64(X, Y, 0.5)
    dX, dY = orbf.backward_f64(X, Y, G, K, 0.5)
    np.testing.assert_allclose(dX, Xt.grad.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(dY, Yt.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_backward_translation_identity_and_gamma0():
    X, Y, G = _inputs(50, 40, 64, seed=6)
    K = orbf.forward_f64(X, Y, 0.5)
    dX, dY = orbf.backward_f64(X, Y, G, K, 0.5)
    # K depends on X, Y only through X_i - Y_j, so shifting both by c leaves L
    # unchanged: sum_i dX_i + sum_j dY_j = 0.
    np.testing.assert_allclose(dX.sum(0) + dY.sum(0), 0.0, atol=1e-12)
    zX, zY = orbf.backward_f64(X, Y, G, orbf.forward_f64(X, Y, 0.0), 0.0)
    assert np.all(zX == 0) and np.all(zY == 0)


# ------------------------------------------------ reference's own CPU loops
def test_oracle_vs_committed_reference_fixtures():
    z = np.load(GOLDEN)
    for name in ("tiny", "small", "ragged", "refdefault"):
        X, Y, G = z[f"{name}_X"], z[f"{name}_Y"], z[f"{name}_G"]
        gamma = float(z[f"{name}_gamma"])
        K = orbf.forward_f64(X, Y, gamma)
        np.testing.assert_allclose(K, z[f"{name}_K"], rtol=1e-5, atol=1e-6)
        dX, dY = orbf.backward_f64(X, Y, G, K, gamma)
        np.testing.assert_allclose(dX, z[f"{name}_dX"], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(dY, z[f"{name}_dY"], rtol=1e-4, atol=1e-5)


@pytest.mark.skipif(native.ref_lib() is None, reason="oracle/_ref not built (needs /root/reference)")
def test_oracle_vs_reference_loops_live():
    X, Y, G = _inputs(64, 48, 64, seed=7)
    Kref = native.ref_rbf_forward(X, Y, 0.5)
    K = orbf.forward_f64(X, Y, 0.5)
    np.testing.assert_allclose(K, Kref, rtol=1e-5, atol=1e-6)
    rX, rY = native.ref_rbf_backward(X, Y, G, Kref, 0.5)
    dX, dY = orbf.backward_f64(X, Y, G, K, 0.5)
    np.testing.assert_allclose(dX, rX, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dY, rY, rtol=1e-4, atol=1e-5)


def test_torch_cpu_path_matches_oracle():
    X, Y, G = _inputs(64, 80, 64, seed=8)
    Xt, Yt, Gt = map(torch.from_numpy, (X, Y, G))
    K = orbf.torch_cpu_forward(Xt, Yt, 0.5).numpy()
    np.testing.assert_allclose(K, orbf.forward_f64(X, Y, 0.5), rtol=1e-5, atol=1e-6)
    dX, dY = orbf.torch_cpu_backward(Xt, Yt, Gt, 0.5)
    rX, rY = orbf.backward_f64(X, Y, G, orbf.forward_f64(X, Y, 0.5), 0.5)
    np.testing.assert_allclose(dX.numpy(), rX, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dY.numpy(), rY, rtol=1e-4, atol=1e-5)


# ------------------------------------------------------ mutation of the oracle
def _bad_sign(X, Y, dK, K, g):
    dX, dY = orbf.backward_f64(X, Y, dK, K, g)
    return -dX, -dY


def _bad_no_rowsum(X, Y, dK, K, g):
    W = dK * K
    return 2 * g * (W @ Y), -2 * g * (W.sum(0)[:, None] * Y - W.T @ X)


def _bad_transposed(X, Y, dK, K, g):
    W = dK * K
    dX = -2 * g * (W.sum(1)[:, None] * X - W @ Y)
    dY = -2 * g * (W.sum(1)[:, None] * Y - (W @ X))  # row sums / W for W^T
    return dX, dY


def _bad_factor(X, Y, dK, K, g):
    dX, dY = orbf.backward_f64(X, Y, dK, K, g)
    return dX / 2, dY / 2


@pytest.mark.parametrize("bad", [_bad_sign, _bad_no_rowsum, _bad_transposed, _bad_factor])
def test_planted_mistakes_are_caught(bad):
    X, Y, G = _inputs(6, 6, 3, scale=0.5, seed=9)  # square, so a transpose mix-up runs
    K = orbf.forward_f64(X, Y, 0.5)
    fX, fY = orbf.finite_difference_grads(X, Y, G, 0.5)
    bX, bY = bad(X, Y, G, K, 0.5)
    ok = np.allclose(bX, fX, rtol=1e-6, atol=1e-8) and np.allclose(bY, fY, rtol=1e-6, atol=1e-8)
    assert not ok
