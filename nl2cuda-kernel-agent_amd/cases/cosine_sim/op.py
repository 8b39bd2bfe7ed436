"""Cosine-similarity candidate: autograd wrapper over the HIP library
(kernels/cosine_sim.hip).

Mirrors the reference's cases/cosine_sim/op.py:19-43: ``CosineSimFunction``
runs the forward once, saves what the backward needs and returns
(dA, dB, None); ``candidate`` and ``forward_only`` keep the dict interface.
The saved tensors differ: the reference saves the normalised copies Ah, Bh
and the inverse norms; here the backward scales rows as it stages them, so
A, B and the inverse norms are saved and no [N, D] / [M, D] copies are
written.  There is no CPU path: without a GPU the library refuses to load.
"""

import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "cosine_sim_hip"
SOURCES = ["cosine_sim.hip"]


def bind_library(lib):
    V, I64, F, S = capi.c_void_p, capi.c_int64, capi.c_float, capi.c_size_t
    capi.bind(lib, "cosine_sim_forward_f32", [V, V, V, V, V, I64, I64, I64, F, V])
    capi.bind(lib, "cosine_sim_backward_workspace_bytes", [I64, I64, I64], S)
    capi.bind(lib, "cosine_sim_backward_f32", [V, V, V, V, V, V, V, I64, I64, I64, V, S, V])
    capi.bind_last_error(lib, "cosine_sim_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _check_pair(A, B):
    capi.require(A.is_cuda and B.is_cuda, "A, B must be GPU tensors")
    capi.require(A.dtype == torch.float32 and B.dtype == torch.float32, "A, B must be float32")
    capi.require(A.dim() == 2 and B.dim() == 2, "A, B must be 2D")
    capi.require(A.size(1) == B.size(1), "A, B must share feature dim D")
    capi.require(A.size(1) > 0, "D must be positive")


def cos_forward(A, B, eps):
    """(S, inv_a, inv_b): S = (A_i . B_j) / ((|A_i| + eps)(|B_j| + eps)) and
    the inverse norms 1 / (|row| + eps) the backward reuses."""
    _check_pair(A, B)
    lib = _lib()
    A, B = A.contiguous(), B.contiguous()
    N, D = A.shape
    M = B.size(0)
    S = torch.empty((N, M), dtype=torch.float32, device=A.device)
    inv_a = torch.empty(N, dtype=torch.float32, device=A.device)
    inv_b = torch.empty(M, dtype=torch.float32, device=A.device)
    with torch.cuda.device(A.device):
        st = lib.cosine_sim_forward_f32(capi.ptr(A), capi.ptr(B), capi.ptr(S), capi.ptr(inv_a),
                                        capi.ptr(inv_b), N, M, D, float(eps),
                                        capi.stream_of(A))
    capi.check(st, lib.cosine_sim_last_error, "cos_forward")
    return S, inv_a, inv_b


def cos_backward(A, B, inv_a, inv_b, dS):
    """(dA, dB) from upstream dS = dL/dS and the forward's inverse norms."""
    _check_pair(A, B)
    N, M = A.size(0), B.size(0)
    capi.require(dS.is_cuda and dS.dtype == torch.float32 and tuple(dS.shape) == (N, M),
                 "dS must be a float32 GPU tensor of shape [N, M]")
    lib = _lib()
    A, B, dS = A.contiguous(), B.contiguous(), dS.contiguous()
    D = A.size(1)
    dA = torch.empty_like(A)
    dB = torch.empty_like(B)
    ws_bytes = lib.cosine_sim_backward_workspace_bytes(N, M, D)
    ws = torch.empty((max(ws_bytes, 4) + 3) // 4, dtype=torch.float32, device=A.device)
    with torch.cuda.device(A.device):
        st = lib.cosine_sim_backward_f32(capi.ptr(A), capi.ptr(B), capi.ptr(inv_a),
                                         capi.ptr(inv_b), capi.ptr(dS), capi.ptr(dA),
                                         capi.ptr(dB), N, M, D, capi.ptr(ws), ws_bytes,
                                         capi.stream_of(A))
    capi.check(st, lib.cosine_sim_last_error, "cos_backward")
    return dA, dB


class CosineSimFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, A, B, eps):
        A, B = A.contiguous(), B.contiguous()
        S, inv_a, inv_b = cos_forward(A, B, float(eps))
        ctx.save_for_backward(A, B, inv_a, inv_b)
        return S

    @staticmethod
    def backward(ctx, dS):
        A, B, inv_a, inv_b = ctx.saved_tensors
        dA, dB = cos_backward(A, B, inv_a, inv_b, dS.contiguous())
        return dA, dB, None


def candidate(inputs, params):
    """Framework candidate contract: inputs={"A","B"}, params={"eps"} -> S."""
    return CosineSimFunction.apply(inputs["A"], inputs["B"], params["eps"])


def forward_only(inputs, params):
    """Forward without autograd."""
    return cos_forward(inputs["A"], inputs["B"], float(params["eps"]))[0]
