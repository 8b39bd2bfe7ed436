"""CPU oracle of the cosine-similarity case -- TEST INFRASTRUCTURE ONLY.

Restates cases/cosine_sim/reference.py:13-20 in float64 with numpy:
  * ``forward_f64``: s = 1 / (|row| + eps) per row of A and B, then
    S = (s_a A) (s_b B)^T;
  * ``backward_f64``: autograd of that expression for upstream dS,
        dah = dS (s_b B),   dA = s_a dah - ((s_a A) . dah) / |A| (s_a A)
    per row (the second term is 0 for a zero row: torch's norm backward
    gives 0 there), and symmetrically for dB with dS^T;
  * ``forward_loops``: brute force for tiny inputs.

Pinned by tests/test_oracle_cosine.py: hand values (orthogonal, parallel,
antiparallel rows), scale invariance, brute force, float64 torch autograd of
the reference expression (forward and backward, zero rows included),
central finite differences, and planted mistakes that must fail (the
reference CUDA kernel's s_a in place of 1/|A| at a large eps, a dropped
projection term, an untransposed dS for dB, a sign flip).
"""

import numpy as np


def inv_norms(V, eps):
    V = np.asarray(V, dtype=np.float64)
    return 1.0 / (np.sqrt((V * V).sum(axis=1)) + eps)


def forward_f64(A, B, eps):
    """reference.py:13-20: S[i, j] = (A_i . B_j) s_a[i] s_b[j]."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    return (A * inv_norms(A, eps)[:, None]) @ (B * inv_norms(B, eps)[:, None]).T


def _project(V, s, dvh):
    """s dvh - ((s V) . dvh) / |V| (s V) per row; 0 for the second term when |V| = 0."""
    vh = V * s[:, None]
    nrm = np.sqrt((V * V).sum(axis=1))
    dot = (vh * dvh).sum(axis=1)
    coef = np.divide(dot, nrm, out=np.zeros_like(dot), where=nrm > 0)
    return s[:, None] * dvh - coef[:, None] * vh


def backward_f64(A, B, dS, eps):
    """(dA, dB): autograd of forward_f64 for upstream dS [N, M]."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    dS = np.asarray(dS, dtype=np.float64)
    sa, sb = inv_norms(A, eps), inv_norms(B, eps)
    dah = dS @ (B * sb[:, None])
    dbh = dS.T @ (A * sa[:, None])
    return _project(A, sa, dah), _project(B, sb, dbh)


def forward_loops(A, B, eps):
    """Brute force, one pair at a time."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    S = np.zeros((A.shape[0], B.shape[0]))
    for i in range(A.shape[0]):
        na = sum(float(v) * float(v) for v in A[i]) ** 0.5
        for j in range(B.shape[0]):
            nb = sum(float(v) * float(v) for v in B[j]) ** 0.5
            dot = sum(float(a) * float(b) for a, b in zip(A[i], B[j]))
            S[i, j] = dot / ((na + eps) * (nb + eps))
    return S
