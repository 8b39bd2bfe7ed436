"""PyTorch reference of L2 normalisation with a per-dimension scale (the
case's golden reference).

Same expression as the reference's cases/l2norm_scale/reference.py:12-17:
norm = sqrt(sum(x * x) + eps) per row, then (x / norm) * g; autograd gives
the backward.  ``make_inputs`` draws X then g from one seeded generator
(reference.py:20-28) on the host CPU, then moves them to ``device``.
"""

import torch

from cases.l2norm_scale import config


def reference_forward(inputs, params):
    """inputs={"X":[N,D], "g":[D]}, params={"eps": float} -> Y:[N,D]."""
    x, g = inputs["X"], inputs["g"]
    norm = torch.sqrt((x * x).sum(dim=-1, keepdim=True) + params["eps"])
    return (x / norm) * g


def make_inputs_for(n, d):
    """Input generator for an N x D problem with N(0, 1) entries."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        gen = torch.Generator(device="cpu").manual_seed(seed)
        x = torch.randn(n, d, dtype=torch.float32, generator=gen).to(device=device, dtype=dtype)
        g = torch.randn(d, dtype=torch.float32, generator=gen).to(device=device, dtype=dtype)
        if requires_grad:
            x.requires_grad_(True)
            g.requires_grad_(True)
        return {"X": x, "g": g}

    return make_inputs


make_inputs = make_inputs_for(config.N, config.D)
