"""Pins oracle/cosine_sim.py (CPU only): hand values, scale invariance,
brute force, float64 torch autograd of the reference expression, central
finite differences, zero rows, and planted mistakes that must fail."""

import numpy as np
import pytest
import torch

from oracle import cosine_sim as oc

EPS = 1e-8


def _rand(n, d, seed):
    return np.random.default_rng(seed).standard_normal((n, d))


def _torch_ref(A, B, dS, eps):
    """The reference expression (cases/cosine_sim/reference.py:13-20) in
    float64 torch, with autograd for the backward."""
    At = torch.tensor(A, dtype=torch.float64, requires_grad=True)
    Bt = torch.tensor(B, dtype=torch.float64, requires_grad=True)
    Ah = At / (At.norm(dim=-1, keepdim=True) + eps)
    Bh = Bt / (Bt.norm(dim=-1, keepdim=True) + eps)
    S = (Ah[:, None, :] * Bh[None, :, :]).sum(dim=-1)
    S.backward(torch.tensor(dS, dtype=torch.float64))
    return S.detach().numpy(), At.grad.numpy(), Bt.grad.numpy()


def test_hand_values():
    A = np.array([[1.0, 0.0, 0.0], [0.0, 2.0, 0.0], [3.0, 4.0, 0.0]])
    B = np.array([[2.0, 0.0, 0.0], [0.0, 0.0, 5.0], [-3.0, -4.0, 0.0]])
    S = oc.forward_f64(A, B, 0.0)
    expect = np.array([[1.0, 0.0, -0.6], [0.0, 0.0, -0.8], [0.6, 0.0, -1.0]])
    assert np.allclose(S, expect, atol=1e-15)
    # eps shrinks every entry by the two norms' (n + eps) factors
    S1 = oc.forward_f64(A[:1], B[:1], 1.0)
    assert np.isclose(S1[0, 0], 2.0 / ((1.0 + 1.0) * (2.0 + 1.0)))


def test_scale_invariance_and_range():
    A, B = _rand(7, 16, 0), _rand(5, 16, 1)
    S = oc.forward_f64(A, B, 0.0)
    assert np.allclose(oc.forward_f64(3.5 * A, 0.25 * B, 0.0), S, atol=1e-14)
    assert np.all(np.abs(S) <= 1.0 + 1e-12)
    assert np.allclose(np.diag(oc.forward_f64(A, A, 0.0)), 1.0)


def test_brute_force_small():
    A, B = _rand(4, 5, 2), _rand(3, 5, 3)
    assert np.allclose(oc.forward_f64(A, B, EPS), oc.forward_loops(A, B, EPS), atol=1e-14)


@pytest.mark.parametrize("eps", [1e-8, 0.3])
def test_matches_torch_autograd(eps):
    A, B = _rand(9, 12, 4), _rand(6, 12, 5)
    dS = _rand(9, 6, 6)
    S, dA, dB = _torch_ref(A, B, dS, eps)
    assert np.allclose(oc.forward_f64(A, B, eps), S, atol=1e-14)
    gA, gB = oc.backward_f64(A, B, dS, eps)
    assert np.allclose(gA, dA, atol=1e-12)
    assert np.allclose(gB, dB, atol=1e-12)


def test_zero_rows_match_torch():
    A, B = _rand(4, 8, 7), _rand(3, 8, 8)
    A[1] = 0.0
    B[2] = 0.0
    dS = _rand(4, 3, 9)
    S, dA, dB = _torch_ref(A, B, dS, EPS)
    assert np.all(oc.forward_f64(A, B, EPS)[1] == 0.0)
    gA, gB = oc.backward_f64(A, B, dS, EPS)
    assert np.allclose(gA, dA, rtol=1e-12, atol=1e-6)  # zero row: dah / eps (~1e8)
    assert np.allclose(gB, dB, rtol=1e-12, atol=1e-6)


def test_finite_differences():
    A, B = _rand(3, 4, 10), _rand(2, 4, 11)
    dS = _rand(3, 2, 12)
    gA, gB = oc.backward_f64(A, B, dS, EPS)
    h = 1e-6
    for X, g, which in ((A, gA, 0), (B, gB, 1)):
        num = np.zeros_like(X)
        for idx in np.ndindex(X.shape):
            Xp, Xm = X.copy(), X.copy()
            Xp[idx] += h
            Xm[idx] -= h
            fp = oc.forward_f64(Xp, B, EPS) if which == 0 else oc.forward_f64(A, Xp, EPS)
            fm = oc.forward_f64(Xm, B, EPS) if which == 0 else oc.forward_f64(A, Xm, EPS)
            num[idx] = ((fp - fm) * dS).sum() / (2 * h)
        assert np.allclose(g, num, atol=1e-7)


def _bad(kind, A, B, dS, eps):
    sa, sb = oc.inv_norms(A, eps), oc.inv_norms(B, eps)
    dah = dS @ (B * sb[:, None])
    ah = A * sa[:, None]
    if kind == "kernel_formula":   # s_a in place of 1 / |A| in the projection
        return sa[:, None] * (dah - (ah * dah).sum(1)[:, None] * ah)
    if kind == "no_projection":
        return sa[:, None] * dah
    if kind == "untransposed_dS":  # dB built from dS instead of dS^T (square case)
        dbh = dS @ (A * sa[:, None])
        return oc._project(B, sb, dbh)
    if kind == "sign":
        return -oc._project(A, sa, dah)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["kernel_formula", "no_projection", "untransposed_dS", "sign"])
def test_planted_mistakes_are_caught(kind):
    eps = 0.5  # large enough that 1/|A| and 1/(|A| + eps) differ
    A, B = _rand(6, 6, 13), _rand(6, 6, 14)
    dS = _rand(6, 6, 15)
    _, dA, dB = _torch_ref(A, B, dS, eps)
    got = _bad(kind, A, B, dS, eps)
    ref = dB if kind == "untransposed_dS" else dA
    assert not np.allclose(got, ref, atol=1e-6), kind
