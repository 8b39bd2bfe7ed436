"""LayerNorm oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Reference definition: cases/layernorm/reference.py:14-21 (two-pass mean,
biased variance, eps inside the square root), backward by autograd; the
reference kernels' backward formula (layernorm_backward.cu:74-93):
dx = rstd (g - mean(g) - xhat mean(g xhat)), g = dy w.

Pins (tests/test_oracle_layernorm.py): hand-computed values, torch float64
autograd of the restated reference, central finite differences (float64,
tiny shapes), the exact identity sum_d dx = 0, dbias = sum_b dy, the C
restatement (csrc/oracle.c oracle_layernorm_forward), and planted mistakes.
"""

import numpy as np


def forward_f64(x, w, b, eps):
    """(y, mean, rstd) in float64."""
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1)
    var = ((x - mean[:, None]) ** 2).mean(axis=-1)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = (x - mean[:, None]) * rstd[:, None]
    y = xhat * np.asarray(w, dtype=np.float64) + np.asarray(b, dtype=np.float64)
    return y, mean, rstd


def backward_f64(dy, x, w, eps):
    """(dx, dw, db) in float64 from the closed form."""
    x = np.asarray(x, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    _, mean, rstd = forward_f64(x, w, np.zeros_like(w), eps)
    xhat = (x - mean[:, None]) * rstd[:, None]
    g = dy * w
    dx = rstd[:, None] * (g - g.mean(axis=-1, keepdims=True)
                          - xhat * (g * xhat).mean(axis=-1, keepdims=True))
    return dx, (dy * xhat).sum(axis=0), dy.sum(axis=0)


def finite_difference_grads(x, w, b, dy, eps, h=1e-6):
    x = np.array(x, dtype=np.float64)
    w = np.array(w, dtype=np.float64)
    b = np.array(b, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)

    def loss(xx, ww, bb):
        return float(np.sum(dy * forward_f64(xx, ww, bb, eps)[0]))

    grads = []
    for arr in (x, w, b):
        g = np.zeros_like(arr)
        for idx in np.ndindex(*arr.shape):
            orig = arr[idx]
            arr[idx] = orig + h
            lp = loss(x, w, b)
            arr[idx] = orig - h
            lm = loss(x, w, b)
            arr[idx] = orig
            g[idx] = (lp - lm) / (2 * h)
        grads.append(g)
    return tuple(grads)


def torch_cpu_forward(x, w, b, eps):
    """Op-for-op restatement of reference.py:14-21 (CPU torch tensors)."""
    import torch
    mean = x.mean(dim=-1, keepdim=True)
    var = ((x - mean) ** 2).mean(dim=-1, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps) * w + b


def torch_cpu_backward(x, w, b, dy, eps):
    xr = x.detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    br = b.detach().clone().requires_grad_(True)
    torch_cpu_forward(xr, wr, br, eps).backward(dy)
    return xr.grad, wr.grad, br.grad
