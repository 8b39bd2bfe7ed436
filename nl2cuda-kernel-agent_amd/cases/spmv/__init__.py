"""SpMV case: ``CASE`` (reference defaults, cases/spmv/__init__.py:16-24),
``make_case`` for other uniform shapes and ``baseline_case`` (the power-law
2^20 x 2^20 SpMV with int32 indices)."""

import os

import torch

from framework.case import Case
from cases.spmv import config
from cases.spmv.reference import (make_inputs, make_inputs_for, make_zipf_inputs_for,
                                  reference_forward)


def _load_description():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "description.md")
    with open(path, encoding="utf-8") as f:
        return f.read()


def make_case(m=None, k=None, d=None, nnz_per_row=None):
    m = config.M if m is None else m
    k = config.K if k is None else k
    d = config.D if d is None else d
    nnz_per_row = config.NNZ_PER_ROW if nnz_per_row is None else nnz_per_row
    return Case(name="spmv", description=_load_description(), params={},
                grad_inputs=["vals", "X"], dtype=config.DTYPE,
                make_inputs=make_inputs_for(m, k, d, nnz_per_row),
                reference_forward=reference_forward)


def baseline_case(m=config.BASELINE_M, k=config.BASELINE_K, d=config.BASELINE_D,
                  index_dtype=torch.int32):
    return Case(name="spmv_zipf", description=_load_description(), params={},
                grad_inputs=["vals", "X"], dtype=config.DTYPE,
                make_inputs=make_zipf_inputs_for(m, k, d, index_dtype),
                reference_forward=reference_forward)


CASE = Case(
    name="spmv",
    description=_load_description(),
    params={},
    grad_inputs=["vals", "X"],
    dtype=config.DTYPE,
    make_inputs=make_inputs,
    reference_forward=reference_forward,
)
