"""RBF oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Reference definition: cases/rbf/reference.py:14-20 (K = exp(-gamma * sum_d
(X[i,d]-Y[j,d])^2), backward by autograd); formulas of the backward:
cases/rbf/delivery/README.md:10-12 and the naive loops of
cases/rbf/delivery/rbf_test.cu:24-52 (coef = -2 gamma G K).

Pins (tests/test_oracle_rbf.py):
  * forward_f64 vs forward_bruteforce_f64 (independent broadcast form) and vs
    hand-computed values; invariants K(x,x) = 1, symmetry, gamma = 0 -> 1;
  * backward_f64 vs central finite differences of forward_f64 (float64),
    vs the loop restatement backward_loops, vs torch float64 autograd of the
    broadcast form, and the translation identity sum dX + sum dY = 0;
  * both vs the reference's own CPU loops compiled from
    cases/rbf/delivery/rbf_test.cu into oracle/_ref (when built) and vs the
    committed fixtures in tests/golden/rbf_ref_*.npz that those loops wrote.
"""

import numpy as np


def forward_f64(X, Y, gamma):
    """K in float64 via |x|^2 + |y|^2 - 2 x.y (reference.py:14-20 semantics)."""
    X = np.asarray(X, dtype=np.float64)
    Y = np.asarray(Y, dtype=np.float64)
    nx = np.einsum("ij,ij->i", X, X)
    ny = np.einsum("ij,ij->i", Y, Y)
    d = nx[:, None] + ny[None, :] - 2.0 * (X @ Y.T)
    np.maximum(d, 0.0, out=d)
    return np.exp(-gamma * d)


def forward_bruteforce_f64(X, Y, gamma):
    """K in float64 by the broadcast form diff -> square -> sum (small sizes)."""
    X = np.asarray(X, dtype=np.float64)
    Y = np.asarray(Y, dtype=np.float64)
    diff = X[:, None, :] - Y[None, :, :]
    return np.exp(-gamma * np.sum(diff * diff, axis=-1))


def backward_f64(X, Y, dK, K, gamma):
    """(dX, dY) in float64: W = dK o K, dX = -2g(rowsum(W) X - W Y),
    dY = -2g(colsum(W) Y - W^T X) (delivery/README.md:10-12)."""
    X = np.asarray(X, dtype=np.float64)
    Y = np.asarray(Y, dtype=np.float64)
    W = np.asarray(dK, dtype=np.float64) * np.asarray(K, dtype=np.float64)
    dX = -2.0 * gamma * (W.sum(axis=1)[:, None] * X - W @ Y)
    dY = -2.0 * gamma * (W.sum(axis=0)[:, None] * Y - W.T @ X)
    return dX, dY


def backward_loops(X, Y, dK, K, gamma):
    """Pure-Python restatement of delivery/rbf_test.cu:37-52 (tiny sizes)."""
    N, D = len(X), len(X[0])
    M = len(Y)
    dX = [[0.0] * D for _ in range(N)]
    dY = [[0.0] * D for _ in range(M)]
    for i in range(N):
        for j in range(M):
            coef = -2.0 * gamma * float(dK[i][j]) * float(K[i][j])
            for d in range(D):
                diff = float(X[i][d]) - float(Y[j][d])
                dX[i][d] += coef * diff
                dY[j][d] -= coef * diff
    return np.array(dX), np.array(dY)


def finite_difference_grads(X, Y, dK, gamma, h=1e-6):
    """Central differences of L = sum(dK o K(X, Y)) in float64 (tiny sizes)."""
    X = np.array(X, dtype=np.float64)
    Y = np.array(Y, dtype=np.float64)
    dK = np.asarray(dK, dtype=np.float64)

    def loss(a, b):
        return float(np.sum(dK * forward_bruteforce_f64(a, b, gamma)))

    gX = np.zeros_like(X)
    gY = np.zeros_like(Y)
    for idx in np.ndindex(*X.shape):
        p, m = X.copy(), X.copy()
        p[idx] += h
        m[idx] -= h
        gX[idx] = (loss(p, Y) - loss(m, Y)) / (2 * h)
    for idx in np.ndindex(*Y.shape):
        p, m = Y.copy(), Y.copy()
        p[idx] += h
        m[idx] -= h
        gY[idx] = (loss(X, p) - loss(X, m)) / (2 * h)
    return gX, gY


def torch_cpu_forward(X, Y, gamma):
    """Op-for-op restatement of reference.py:14-20 on CPU torch tensors."""
    diff = X.unsqueeze(1) - Y.unsqueeze(0)
    dist_sq = diff.pow(2).sum(dim=-1)
    import torch
    return torch.exp(-gamma * dist_sq)


def torch_cpu_backward(X, Y, G, gamma):
    """Autograd backward of torch_cpu_forward with upstream G
    (framework/verify.py:59-65); returns (dX, dY)."""
    Xr = X.detach().clone().requires_grad_(True)
    Yr = Y.detach().clone().requires_grad_(True)
    out = torch_cpu_forward(Xr, Yr, gamma)
    out.backward(G)
    return Xr.grad, Yr.grad
