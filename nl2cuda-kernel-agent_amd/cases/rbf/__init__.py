"""RBF case: exposes ``CASE`` (reference defaults, cases/rbf/__init__.py:16-24)
and ``make_case`` for other sizes and input distributions."""

import os

from framework.case import Case
from cases.rbf import config
from cases.rbf.reference import make_inputs, make_inputs_for, reference_forward


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(n=None, m=None, d=None, gamma=None, scale=None):
    """A Case for an N x M x D problem (defaults: the config module)."""
    n = config.N if n is None else n
    m = config.M if m is None else m
    d = config.D if d is None else d
    gamma = config.GAMMA if gamma is None else gamma
    scale = config.INPUT_SCALE if scale is None else scale
    return Case(
        name="rbf",
        description=_load_description(),
        params={"gamma": gamma},
        grad_inputs=["X", "Y"],
        dtype=config.DTYPE,
        make_inputs=make_inputs_for(n, m, d, scale),
        reference_forward=reference_forward,
    )


def baseline_case(size):
    """The acceptance workload at N = M = size: D = 64, gamma = 0.5, X, Y ~ N(0,1)/8."""
    return make_case(size, size, 64, config.BASELINE_GAMMA, config.BASELINE_SCALE)


CASE = Case(
    name="rbf",
    description=_load_description(),
    params={"gamma": config.GAMMA},
    grad_inputs=["X", "Y"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
