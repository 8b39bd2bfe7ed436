"""L2-norm-scale case: exposes ``CASE`` (reference defaults,
cases/l2norm_scale/__init__.py:16-24) and ``make_case`` for other shapes."""

import os

from framework.case import Case
from cases.l2norm_scale import config
from cases.l2norm_scale.reference import make_inputs, make_inputs_for, reference_forward


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(n=None, d=None, eps=None):
    """A Case for an N x D problem (defaults: the config module)."""
    return Case(
        name="l2norm_scale",
        description=_load_description(),
        params={"eps": config.EPS if eps is None else eps},
        grad_inputs=["X", "g"],
        dtype=config.DTYPE,
        make_inputs=make_inputs_for(config.N if n is None else n, config.D if d is None else d),
        reference_forward=reference_forward,
    )


CASE = Case(
    name="l2norm_scale",
    description=_load_description(),
    params={"eps": config.EPS},
    grad_inputs=["X", "g"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
