"""CPU oracle of the scan case -- TEST INFRASTRUCTURE ONLY.

Restates cases/scan/reference.py:8-9 (torch.cumsum over the last dim) and
its autograd backward (description.md:6-15: dX[b, j] = sum_{i >= j} dY[b, i]).

* ``cumsum_f32``: float32 input, accumulated in float64 along the row and
  rounded once to float32 -- what torch's CPU cumsum does for float32
  (verified bit-equal in tests/test_oracle_scan.py, so this is the
  reference's own arithmetic, not an approximation of it).
* ``reverse_cumsum_f32``: the same in reverse (the backward).
* ``cumsum_i64``: int32 input summed exactly in int64 (torch.cumsum's result
  type for int32).  ``cumsum_i32_wrap``: the same truncated to int32
  (two's-complement wrap-around).
* ``torch_cpu_forward`` / ``torch_cpu_backward``: the reference path itself,
  op for op, used as the CPU baseline.

Pinned by tests/test_oracle_scan.py: known values and closed forms
(ones -> 1..D, arange -> triangular numbers, constant c -> c (i + 1)),
brute-force Python loops on small inputs, torch CPU cumsum (bit-equal) and
float64 autograd, the C restatement (oracle/csrc/oracle.c), the identity
reverse(x) = flip(cumsum(flip(x))), and planted mistakes (exclusive scan,
float32 accumulation, off-by-one reverse) that must fail.
"""

import numpy as np


def cumsum_f32(x):
    """reference.py:9 on a float32 array: float64 running sums, one rounding."""
    x = np.asarray(x, dtype=np.float32)
    return np.cumsum(x.astype(np.float64), axis=-1).astype(np.float32)


def reverse_cumsum_f32(dy):
    """Gradient of cumsum: dX[:, j] = sum_{i >= j} dY[:, i] (float64 sums)."""
    dy = np.asarray(dy, dtype=np.float32).astype(np.float64)
    return np.flip(np.cumsum(np.flip(dy, axis=-1), axis=-1), axis=-1).astype(np.float32)


def cumsum_i64(x):
    """torch.cumsum of int32 input: exact int64 running sums."""
    return np.cumsum(np.asarray(x, dtype=np.int32).astype(np.int64), axis=-1)


def cumsum_i32_wrap(x):
    """The exact sums truncated to int32 (modulo 2^32, two's complement)."""
    return cumsum_i64(x).astype(np.int32)


def cumsum_loops(x):
    """Brute force on small inputs: Python floats / ints, one row at a time."""
    x = np.asarray(x)
    out = np.zeros(x.shape, dtype=np.float64 if x.dtype.kind == "f" else np.int64)
    for r in range(x.shape[0]):
        acc = 0.0 if x.dtype.kind == "f" else 0
        for i in range(x.shape[1]):
            acc += x[r, i].item()
            out[r, i] = acc
    return out


def torch_cpu_forward(x):
    import torch
    return torch.cumsum(x, dim=-1)


def torch_cpu_backward(x, g):
    import torch
    xr = x.detach().clone().requires_grad_(True)
    torch.cumsum(xr, dim=-1).backward(g)
    return xr.grad
