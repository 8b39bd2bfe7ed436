"""LayerNorm case: ``CASE`` (reference defaults, cases/layernorm/__init__.py:16-24)
and ``make_case`` / ``baseline_case`` for other sizes."""

import os

from framework.case import Case
from cases.layernorm import config
from cases.layernorm.reference import make_inputs, make_inputs_for, reference_forward


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(b=None, d=None, params=None, eps=None):
    b = config.B if b is None else b
    d = config.D if d is None else d
    params = config.PARAMS if params is None else params
    eps = config.EPS if eps is None else eps
    return Case(name="layernorm", description=_load_description(), params={"eps": eps},
                grad_inputs=["X", "gamma", "beta"], dtype=config.DTYPE,
                make_inputs=make_inputs_for(b, d, params), reference_forward=reference_forward)


def baseline_case():
    """The acceptance workload: x [8192, 4096], gamma = 1 + 0.1 N, beta = 0.1 N."""
    return make_case(config.BASELINE_B, config.BASELINE_D, "baseline")


CASE = Case(
    name="layernorm",
    description=_load_description(),
    params={"eps": config.EPS},
    grad_inputs=["X", "gamma", "beta"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
