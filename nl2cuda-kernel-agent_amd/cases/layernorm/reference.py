"""PyTorch reference of LayerNorm (the case's golden reference).

Same operations as the reference's cases/layernorm/reference.py:14-21:
mean over the last dim, biased variance of (X - mean), xhat = (X - mean) /
sqrt(var + eps), Y = xhat * gamma + beta; autograd provides the backward.
Inputs are drawn on the host CPU generator (X, then gamma, then beta, as in
reference.py:26-29) and moved to ``device``.
"""

import torch

from cases.layernorm import config


def reference_forward(inputs, params):
    """inputs={"X":[B,D], "gamma":[D], "beta":[D]}, params={"eps"} -> Y:[B,D]."""
    X, gamma, beta = inputs["X"], inputs["gamma"], inputs["beta"]
    eps = params["eps"]
    mean = X.mean(dim=-1, keepdim=True)
    var = ((X - mean) ** 2).mean(dim=-1, keepdim=True)
    xhat = (X - mean) / torch.sqrt(var + eps)
    return xhat * gamma + beta


def make_inputs_for(b, d, params="reference"):
    def make_inputs(seed, dtype, device, requires_grad=False):
        g = torch.Generator(device="cpu").manual_seed(seed)
        X = torch.randn(b, d, generator=g)
        gamma = torch.randn(d, generator=g)
        beta = torch.randn(d, generator=g)
        if params == "baseline":
            gamma = 1.0 + 0.1 * gamma
            beta = 0.1 * beta
        out = {"X": X, "gamma": gamma, "beta": beta}
        out = {k: v.to(device=device, dtype=dtype) for k, v in out.items()}
        if requires_grad:
            for v in out.values():
                v.requires_grad_(True)
        return out

    return make_inputs


make_inputs = make_inputs_for(config.B, config.D, config.PARAMS)
