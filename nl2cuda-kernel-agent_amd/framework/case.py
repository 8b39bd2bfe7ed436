"""The Case protocol: the only contract between the framework and a case.

Same seven fields as the reference's Case (framework/case.py:13-35).  A case
package exposes an instance as ``CASE`` in its ``__init__``; verify/bench only
rely on these fields, never on input counts, output shapes or parameter names.
"""

from dataclasses import dataclass
from typing import Callable


@dataclass
class Case:
    """Description of one algorithm case.

    name:              short name, e.g. "rbf".
    description:       natural-language description of the algorithm.
    params:            scalar parameters, e.g. {"gamma": 1/64}.
    grad_inputs:       names of the inputs that receive gradients.
    dtype:             acceptance dtype name, e.g. "float32".
    make_inputs:       (seed, dtype, device, requires_grad) -> dict[str, Tensor]
    reference_forward: (inputs: dict, params: dict) -> Tensor; the PyTorch
                       reference, whose backward autograd provides.
    """

    name: str
    description: str
    params: dict
    grad_inputs: list
    dtype: str
    make_inputs: Callable
    reference_forward: Callable
