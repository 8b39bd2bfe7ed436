"""PyTorch reference of pairwise cosine similarity (the case's golden
reference).

Same expression as the reference's cases/cosine_sim/reference.py:13-20:
rows scaled by 1 / (norm + eps), then the broadcast product summed over D
(deliberately not a matmul).  Autograd provides the backward.
``make_inputs`` draws A then B from one seeded generator
(reference.py:23-30) on the host CPU, then moves them to ``device``, so
every device sees identical inputs.
"""

import torch

from cases.cosine_sim import config


def reference_forward(inputs, params):
    """inputs={"A":[N,D], "B":[M,D]}, params={"eps": float} -> S:[N,M]."""
    A, B = inputs["A"], inputs["B"]
    eps = params["eps"]
    Ah = A / (A.norm(dim=-1, keepdim=True) + eps)
    Bh = B / (B.norm(dim=-1, keepdim=True) + eps)
    return (Ah[:, None, :] * Bh[None, :, :]).sum(dim=-1)


def make_inputs_for(n, m, d):
    """Input generator for an N x M x D problem with N(0, 1) entries."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        g = torch.Generator(device="cpu").manual_seed(seed)
        A = torch.randn(n, d, dtype=torch.float32, generator=g).to(device=device, dtype=dtype)
        B = torch.randn(m, d, dtype=torch.float32, generator=g).to(device=device, dtype=dtype)
        if requires_grad:
            A.requires_grad_(True)
            B.requires_grad_(True)
        return {"A": A, "B": B}

    return make_inputs


make_inputs = make_inputs_for(config.N, config.M, config.D)
