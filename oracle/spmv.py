"""CPU oracle of the CSR SpMM / SpMV case -- TEST INFRASTRUCTURE ONLY.

Restates cases/spmv/reference.py:8-23 (Y[m] = sum over row m of vals * X[col])
and its autograd backward (dvals[p] = dY[row(p)] . X[col(p)], dX = A^T dY)
in float64 with numpy:
  * ``forward_f64``: per-nonzero contributions summed by row
    (np.add.reduceat over the non-empty rows; empty rows are 0);
  * ``backward_f64``: dvals by row-expanded dot products, dX by per-column
    np.bincount (D = 1) or per-feature bincount (D > 1);
  * ``forward_loops``: brute force for tiny inputs;
  * ``torch_cpu_forward``: the reference path itself, op for op (the CPU
    baseline).

Pinned by tests/test_oracle_spmv.py: hand-computed values, brute force, a
dense float64 matmul of the densified A, the torch CPU path, float64 torch
autograd, the C restatement (oracle/csrc/oracle.c), the adjoint identities
<A x, dy> = <x, A^T dy> = sum_p vals[p] dvals[p], and planted mistakes
(transposed product, dropped duplicate, off-by-one row) that must fail.
"""

import numpy as np


def row_ids(row_ptr):
    row_ptr = np.asarray(row_ptr, dtype=np.int64)
    return np.repeat(np.arange(row_ptr.shape[0] - 1, dtype=np.int64), np.diff(row_ptr))


def forward_f64(row_ptr, col_idx, vals, X):
    row_ptr = np.asarray(row_ptr, dtype=np.int64)
    col = np.asarray(col_idx, dtype=np.int64)
    X = np.asarray(X, dtype=np.float64)
    v = np.asarray(vals, dtype=np.float64)
    M = row_ptr.shape[0] - 1
    contrib = v[:, None] * X[col]
    Y = np.zeros((M, X.shape[1]))
    nonempty = np.diff(row_ptr) > 0
    if contrib.shape[0]:
        Y[nonempty] = np.add.reduceat(contrib, row_ptr[:-1][nonempty], axis=0)
    return Y


def backward_f64(row_ptr, col_idx, vals, X, dY):
    row_ptr = np.asarray(row_ptr, dtype=np.int64)
    col = np.asarray(col_idx, dtype=np.int64)
    X = np.asarray(X, dtype=np.float64)
    dY = np.asarray(dY, dtype=np.float64)
    v = np.asarray(vals, dtype=np.float64)
    rows = row_ids(row_ptr)
    dvals = np.einsum("pd,pd->p", dY[rows], X[col]) if col.size else np.zeros(0)
    K, D = X.shape
    dX = np.empty((K, D))
    for d in range(D):
        dX[:, d] = np.bincount(col, weights=v * dY[rows, d], minlength=K)
    return dvals, dX


def forward_loops(row_ptr, col_idx, vals, X):
    M = len(row_ptr) - 1
    Y = np.zeros((M, np.asarray(X).shape[1]))
    for m in range(M):
        for p in range(int(row_ptr[m]), int(row_ptr[m + 1])):
            Y[m] += float(vals[p]) * np.asarray(X[int(col_idx[p])], dtype=np.float64)
    return Y


def densify(row_ptr, col_idx, vals, K):
    M = len(row_ptr) - 1
    A = np.zeros((M, K))
    np.add.at(A, (row_ids(row_ptr), np.asarray(col_idx, dtype=np.int64)),
              np.asarray(vals, dtype=np.float64))
    return A


def torch_cpu_forward(row_ptr, col_idx, vals, X):
    import torch
    row_counts = row_ptr[1:] - row_ptr[:-1]
    row_idx = torch.repeat_interleave(torch.arange(row_counts.shape[0]), row_counts)
    contributions = vals.unsqueeze(1) * X.index_select(0, col_idx)
    out = torch.zeros((row_counts.shape[0], X.shape[1]), dtype=X.dtype)
    return out.index_add_(0, row_idx, contributions)
