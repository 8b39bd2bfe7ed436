"""CPU oracle of the L2-norm-scale case -- TEST INFRASTRUCTURE ONLY.

Restates cases/l2norm_scale/reference.py:12-17 in float64 with numpy:
  * ``forward_f64``: norm = sqrt(sum_j x^2 + eps) per row, y = x / norm * g;
  * ``backward_f64``: autograd of that expression for upstream dy,
        xh = x / norm,  dx = (g dy - xh (xh . (g dy))) / norm,
        dg = sum over rows of dy xh;
  * ``forward_loops``: brute force for tiny inputs.

Pinned by tests/test_oracle_l2norm.py: hand values (a 3-4-5 row), unit
length of the normalised rows, brute force, float64 torch autograd of the
reference expression, central finite differences, the invariant
x . dx = eps-weighted term (0 when eps = 0), and planted mistakes that must
fail (a LayerNorm-style mean in place of the sum, eps outside the root, a
dropped projection, dg without the normalisation).
"""

import numpy as np


def forward_f64(x, g, eps):
    """(y, norm) of reference.py:12-17 in float64."""
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    norm = np.sqrt((x * x).sum(axis=1) + eps)
    return x / norm[:, None] * g[None, :], norm


def backward_f64(x, g, dy, eps):
    """(dx, dg): autograd of forward_f64 for upstream dy."""
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    norm = np.sqrt((x * x).sum(axis=1) + eps)
    xh = x / norm[:, None]
    gd = dy * g[None, :]
    dot = (xh * gd).sum(axis=1)
    dx = (gd - xh * dot[:, None]) / norm[:, None]
    dg = (dy * xh).sum(axis=0)
    return dx, dg


def forward_loops(x, g, eps):
    """Brute force, one element at a time."""
    x = np.asarray(x, dtype=np.float64)
    y = np.zeros_like(x)
    for i in range(x.shape[0]):
        n = (sum(float(v) * float(v) for v in x[i]) + eps) ** 0.5
        for j in range(x.shape[1]):
            y[i, j] = float(x[i, j]) / n * float(g[j])
    return y
