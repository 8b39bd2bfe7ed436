"""CPU oracle of the softmax cross-entropy case -- TEST INFRASTRUCTURE ONLY.

Restates cases/softmax_ce/reference.py:15-21 in float64 with numpy:
  * ``lse_f64``: log sum_c exp(logits[b, c]) with the row max taken out
    first (the stable form torch.logsumexp computes);
  * ``forward_f64``: loss = mean_b (lse[b] - logits[b, labels[b]]), and lse;
  * ``backward_f64``: autograd of that expression for the upstream scalar
    gout, dlogits = gout / B (softmax - onehot(labels)) (the reference
    kernel's formula, cases/softmax_ce/kernels/softmax_ce_backward.cu:47-53);
  * ``forward_loops``: brute force with math.exp / math.log for tiny inputs.

Pinned by tests/test_oracle_softmax_ce.py: closed forms (equal logits give
log C; two classes give softplus of the margin), brute force, float64 torch
autograd of the reference expression, central finite differences, the
invariants (shift of a row, gradient rows summing to zero, softmax rows
summing to one), logits near the float32 limits, and planted mistakes that
must fail (no max shift, wrong sign of the one-hot, missing 1/B, sum in
place of mean, label off by one).
"""

import math

import numpy as np


def lse_f64(logits):
    x = np.asarray(logits, dtype=np.float64)
    m = x.max(axis=1)
    return m + np.log(np.exp(x - m[:, None]).sum(axis=1))


def forward_f64(logits, labels):
    """(loss, lse) of reference.py:15-21 in float64."""
    x = np.asarray(logits, dtype=np.float64)
    lab = np.asarray(labels, dtype=np.int64)
    lse = lse_f64(x)
    nll = lse - x[np.arange(x.shape[0]), lab]
    return float(nll.mean()) if x.shape[0] else float("nan"), lse


def backward_f64(logits, labels, gout=1.0):
    """dlogits: autograd of forward_f64's loss for the upstream scalar gout."""
    x = np.asarray(logits, dtype=np.float64)
    lab = np.asarray(labels, dtype=np.int64)
    B = x.shape[0]
    p = np.exp(x - lse_f64(x)[:, None])
    p[np.arange(B), lab] -= 1.0
    return p * (float(gout) / B)


def forward_loops(logits, labels):
    """Brute force, one element at a time."""
    total = 0.0
    rows = [[float(v) for v in r] for r in np.asarray(logits)]
    for r, lab in zip(rows, np.asarray(labels)):
        m = max(r)
        lse = m + math.log(sum(math.exp(v - m) for v in r))
        total += lse - r[int(lab)]
    return total / len(rows)
