"""PyTorch reference of the softmax cross-entropy loss (the case's golden
reference).

Same expression as the reference's cases/softmax_ce/reference.py:15-21:
logp = logits - logsumexp(logits) per row, loss = mean of -logp at the
labels, from basic operators (no F.cross_entropy); autograd gives the
backward.  ``make_inputs`` draws logits ~ N(0, 1) then labels uniform in
[0, C) from one seeded generator (reference.py:24-31) on the host CPU, then
moves them to ``device``.
"""

import torch

from cases.softmax_ce import config


def reference_forward(inputs, params):
    """inputs={"logits":[B,C], "labels":[B] int64} -> scalar loss."""
    logits, labels = inputs["logits"], inputs["labels"]
    logp = logits - torch.logsumexp(logits, dim=-1, keepdim=True)
    nll = -logp.gather(1, labels.unsqueeze(1)).squeeze(1)
    return nll.mean()


def make_inputs_for(b, c):
    """Input generator for a B x C problem."""

    def make_inputs(seed, dtype, device, requires_grad=False):
        gen = torch.Generator(device="cpu").manual_seed(seed)
        logits = torch.randn(b, c, dtype=torch.float32, generator=gen)
        labels = torch.randint(0, c, (b,), generator=gen)
        logits = logits.to(device=device, dtype=dtype)
        if requires_grad:
            logits.requires_grad_(True)
        return {"logits": logits, "labels": labels.to(device)}

    return make_inputs


make_inputs = make_inputs_for(config.B, config.C)
