"""PyTorch reference of the inclusive last-dimension scan.

Same operation as the reference's cases/scan/reference.py:8-9
(torch.cumsum(X, dim=-1)); autograd gives the backward (reverse cumsum).
Inputs are drawn on the host CPU generator and moved to ``device``, so the
reference and the candidate see identical tensors.  For int32 input torch
returns int64 (exact), which the int32 case keeps.
"""

import torch

from cases.scan import config


def reference_forward(inputs, params):
    return torch.cumsum(inputs["X"], dim=-1)


def make_inputs_for(b, d, dist="reference"):
    """fp32 inputs: N(0,1) ("reference") or U(-1, 1) ("baseline")."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        g = torch.Generator(device="cpu").manual_seed(seed)
        if dist == "baseline":
            x = torch.rand(b, d, generator=g, dtype=torch.float64) * 2 - 1
        else:
            x = torch.randn(b, d, generator=g)
        x = x.to(device=device, dtype=dtype)
        if requires_grad:
            x.requires_grad_(True)
        return {"X": x}

    return make_inputs


def make_int_inputs_for(b, d, low=config.INT_LOW, high=config.INT_HIGH):
    """int32 inputs ~ U[low, high] (inclusive); the dtype argument is ignored."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        g = torch.Generator(device="cpu").manual_seed(seed)
        x = torch.randint(low, high + 1, (b, d), generator=g, dtype=torch.int32)
        return {"X": x.to(device)}

    return make_inputs


make_inputs = make_inputs_for(config.B, config.D, config.DIST)
