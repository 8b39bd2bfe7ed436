"""Scan case: ``CASE`` (reference defaults, cases/scan/__init__.py:14-22),
``make_case`` for other shapes, ``baseline_case`` (fp32 [64, 65536]
U(-1, 1)) and ``int_case`` (int32 U[-1000, 1000], forward only)."""

import os

from framework.case import Case
from cases.scan import config
from cases.scan.reference import (make_inputs, make_inputs_for, make_int_inputs_for,
                                  reference_forward)


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(b=None, d=None, dist=None):
    b = config.B if b is None else b
    d = config.D if d is None else d
    dist = config.DIST if dist is None else dist
    return Case(name="scan", description=_load_description(), params={}, grad_inputs=["X"],
                dtype=config.DTYPE, make_inputs=make_inputs_for(b, d, dist),
                reference_forward=reference_forward)


def baseline_case():
    return make_case(config.BASELINE_B, config.BASELINE_D, "baseline")


def int_case(b=None, d=None):
    b = config.BASELINE_B if b is None else b
    d = config.BASELINE_D if d is None else d
    return Case(name="scan_int32", description=_load_description(), params={}, grad_inputs=[],
                dtype="int32", make_inputs=make_int_inputs_for(b, d),
                reference_forward=reference_forward)


CASE = Case(
    name="scan",
    description=_load_description(),
    params={},
    grad_inputs=["X"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
