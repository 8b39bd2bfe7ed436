"""Softmax cross-entropy case: exposes ``CASE`` (reference defaults,
cases/softmax_ce/__init__.py:16-24) and ``make_case`` for other shapes."""

import os

from framework.case import Case
from cases.softmax_ce import config
from cases.softmax_ce.reference import make_inputs, make_inputs_for, reference_forward


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(b=None, c=None):
    """A Case for a B x C problem (defaults: the config module)."""
    return Case(
        name="softmax_ce",
        description=_load_description(),
        params={},
        grad_inputs=["logits"],
        dtype=config.DTYPE,
        make_inputs=make_inputs_for(config.B if b is None else b, config.C if c is None else c),
        reference_forward=reference_forward,
    )


CASE = Case(
    name="softmax_ce",
    description=_load_description(),
    params={},
    grad_inputs=["logits"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
