"""Pins the SpMV oracle (CPU only) and checks the acceptance workload's
input recipe."""

import numpy as np
import pytest
import torch

from oracle import native
from oracle import spmv as osp
from cases.spmv import reference as ref


def _random_csr(m, k, lens, seed, d=1):
    rng = np.random.default_rng(seed)
    ptr = np.zeros(m + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    col = rng.integers(0, k, int(ptr[-1]))
    vals = rng.standard_normal(int(ptr[-1])).astype(np.float32)
    X = rng.standard_normal((k, d)).astype(np.float32)
    return ptr, col, vals, X


def test_known_values():
    ptr = [0, 2, 2, 3]
    col = [0, 2, 1]
    vals = np.array([1.0, 2.0, -3.0], np.float32)
    X = np.array([[1.0], [10.0], [100.0]], np.float32)
    assert np.array_equal(osp.forward_f64(ptr, col, vals, X)[:, 0], [201.0, 0.0, -30.0])
    dY = np.array([[1.0], [5.0], [2.0]])
    dvals, dX = osp.backward_f64(ptr, col, vals, X, dY)
    assert np.array_equal(dvals, [1.0, 100.0, 20.0])
    assert np.array_equal(dX[:, 0], [1.0, -6.0, 2.0])


@pytest.mark.parametrize("d", [1, 3, 64])
def test_forward_vs_loops_dense_and_torch(d):
    rng = np.random.default_rng(d)
    lens = rng.integers(0, 9, 50)
    ptr, col, vals, X = _random_csr(50, 40, lens, d, d)
    y = osp.forward_f64(ptr, col, vals, X)
    assert np.allclose(y, osp.forward_loops(ptr, col, vals, X), atol=1e-12)
    assert np.allclose(y, osp.densify(ptr, col, vals, 40) @ X.astype(np.float64), atol=1e-12)
    t = osp.torch_cpu_forward(torch.from_numpy(ptr), torch.from_numpy(col), torch.from_numpy(vals),
                              torch.from_numpy(X))
    assert np.allclose(y, t.numpy(), atol=1e-4)


@pytest.mark.parametrize("d", [1, 5])
def test_backward_vs_autograd_and_adjoint(d):
    rng = np.random.default_rng(10 + d)
    lens = rng.integers(0, 12, 70)
    ptr, col, vals, X = _random_csr(70, 33, lens, 10 + d, d)
    dY = rng.standard_normal((70, d))
    dvals, dX = osp.backward_f64(ptr, col, vals, X, dY)
    v = torch.from_numpy(vals.astype(np.float64)).requires_grad_(True)
    Xt = torch.from_numpy(X.astype(np.float64)).requires_grad_(True)
    out = ref.reference_forward({"row_ptr": torch.from_numpy(ptr), "col_idx": torch.from_numpy(col),
                                 "vals": v, "X": Xt}, {})
    out.backward(torch.from_numpy(dY))
    assert np.allclose(dvals, v.grad.numpy(), atol=1e-12)
    assert np.allclose(dX, Xt.grad.numpy(), atol=1e-12)
    y = osp.forward_f64(ptr, col, vals, X)
    assert np.isclose(np.sum(y * dY), np.sum(X.astype(np.float64) * dX))
    assert np.isclose(np.sum(y * dY), np.sum(vals.astype(np.float64) * dvals))


def test_c_restatement_agrees():
    if native.lib() is None:
        pytest.skip("oracle/lib/liboracle.so not built")
    rng = np.random.default_rng(3)
    lens = rng.integers(0, 20, 300)
    ptr, col, vals, X = _random_csr(300, 200, lens, 3, 8)
    assert np.allclose(native.spmm_csr(ptr, col, vals, X), osp.forward_f64(ptr, col, vals, X),
                       atol=1e-9)


def test_zipf_recipe():
    lens = ref.zipf_row_lengths(1 << 16, 1 << 16, 0)
    assert lens.sum() == 16 * (1 << 16) and lens.min() >= 1 and lens.max() <= 4096
    assert np.array_equal(lens, ref.zipf_row_lengths(1 << 16, 1 << 16, 0))  # deterministic
    cols = ref.sorted_unique_columns(lens, 1 << 16, 0)
    ptr = np.zeros(lens.size + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    rows = osp.row_ids(ptr)
    key = rows * (1 << 16) + cols
    assert np.all(np.diff(key) > 0)  # sorted, unique within each row
    assert cols.min() >= 0 and cols.max() < (1 << 16)


def _transposed(ptr, col, vals, X):
    return osp.densify(ptr, col, vals, X.shape[0]).T[: len(ptr) - 1, : X.shape[0]] @ X


def _drop_duplicates(ptr, col, vals, X):
    A = np.zeros((len(ptr) - 1, X.shape[0]))
    A[osp.row_ids(ptr), col] = vals  # last write wins: duplicates lost
    return A @ X


def _row_shift(ptr, col, vals, X):
    return np.roll(osp.forward_f64(ptr, col, vals, X), 1, axis=0)


@pytest.mark.parametrize("bad", [_transposed, _drop_duplicates, _row_shift])
def test_planted_mistakes_are_caught(bad):
    rng = np.random.default_rng(5)
    m = k = 40
    lens = rng.integers(1, 30, m)
    ptr, col, vals, X = _random_csr(m, k, lens, 5, 2)
    good = osp.forward_f64(ptr, col, vals, X)
    assert np.allclose(good, osp.forward_loops(ptr, col, vals, X))
    assert not np.allclose(bad(ptr, col, vals, X), good, atol=1e-3)
