"""Tolerances and timing constants shared by every case.

Field-for-field the reference's Protocol (framework/protocol.py:12-27) with
two changes required by this build's acceptance bar: atol = rtol = 1e-3
(the reference uses 1e-2), and ``flush_bytes`` -- the size of the buffer the
timing loop reads between timed iterations so that neither the L2 caches
(4 MiB per XCD) nor the 256 MiB Infinity Cache (MALL) of an MI355X hold the
operands of the next iteration.
"""

from dataclasses import dataclass


@dataclass(frozen=True)
class Protocol:
    # correctness
    atol: float = 1e-3
    rtol: float = 1e-3
    seeds: tuple = (0, 1, 2, 3, 4)

    # timing
    warmup: int = 10
    iters: int = 100
    repeats: int = 3
    cv_threshold: float = 0.05
    max_retries: int = 4
    flush_bytes: int = 512 << 20

    # candidate vs baseline acceptance (kept from the reference)
    speedup_target: float = 1.05


PROTOCOL = Protocol()


def dtype_of(name):
    """Map a dtype name to a torch dtype (reference: protocol.py:33-36)."""
    import torch
    return {"float32": torch.float32, "float64": torch.float64,
            "float16": torch.float16, "int32": torch.int32,
            "int64": torch.int64}[name]
