"""Cosine-similarity case: exposes ``CASE`` (reference defaults,
cases/cosine_sim/__init__.py:16-24) and ``make_case`` for other sizes."""

import os

from framework.case import Case
from cases.cosine_sim import config
from cases.cosine_sim.reference import make_inputs, make_inputs_for, reference_forward


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(n=None, m=None, d=None, eps=None):
    """A Case for an N x M x D problem (defaults: the config module)."""
    n = config.N if n is None else n
    m = config.M if m is None else m
    d = config.D if d is None else d
    return Case(
        name="cosine_sim",
        description=_load_description(),
        params={"eps": config.EPS if eps is None else eps},
        grad_inputs=["A", "B"],
        dtype=config.DTYPE,
        make_inputs=make_inputs_for(n, m, d),
        reference_forward=reference_forward,
    )


CASE = Case(
    name="cosine_sim",
    description=_load_description(),
    params={"eps": config.EPS},
    grad_inputs=["A", "B"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
