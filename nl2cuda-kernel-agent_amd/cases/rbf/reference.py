"""PyTorch reference of the RBF kernel matrix (the case's golden reference).

Same operation order as the reference's cases/rbf/reference.py:14-20: the
natural broadcast form diff = X[:,None,:] - Y[None,:,:], squared and summed
over D, then exp(-gamma * .).  Autograd provides the backward.  It
materialises an [N, M, D] intermediate (1 GiB at N = M = 2048), which is the
point: it is the reference path, not an implementation.

``make_inputs`` draws X then Y from one seeded generator (reference:
reference.py:23-31).  The draw always happens on the host CPU generator and
the tensors are then moved to ``device``, so every device sees identical
inputs; ``scale`` multiplies the N(0,1) draws.
"""

import torch

from cases.rbf import config


def reference_forward(inputs, params):
    """inputs={"X":[N,D], "Y":[M,D]}, params={"gamma": float} -> K:[N,M]."""
    X, Y = inputs["X"], inputs["Y"]
    gamma = params["gamma"]
    diff = X.unsqueeze(1) - Y.unsqueeze(0)
    dist_sq = diff.pow(2).sum(dim=-1)
    return torch.exp(-gamma * dist_sq)


def make_inputs_for(n, m, d, scale):
    """Input generator for an N x M x D problem with N(0, scale^2) entries."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        g = torch.Generator(device="cpu").manual_seed(seed)
        X = torch.randn(n, d, dtype=torch.float32, generator=g)
        Y = torch.randn(m, d, dtype=torch.float32, generator=g)
        if scale != 1.0:
            X = X * scale
            Y = Y * scale
        X = X.to(device=device, dtype=dtype)
        Y = Y.to(device=device, dtype=dtype)
        if requires_grad:
            X.requires_grad_(True)
            Y.requires_grad_(True)
        return {"X": X, "Y": Y}

    return make_inputs


make_inputs = make_inputs_for(config.N, config.M, config.D, config.INPUT_SCALE)
