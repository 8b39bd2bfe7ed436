"""L2-norm-scale candidate: autograd wrapper over the HIP library
(kernels/l2norm_scale.hip).

Mirrors the reference's cases/l2norm_scale/op.py:22-44:
``L2NormScaleFunction`` returns Y, saves (X, g, norm) and returns
(dX, dg, None); ``candidate`` and ``forward_only`` keep the dict interface.
There is no CPU path: without a GPU the library refuses to load.
"""

import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "l2norm_scale_hip"
SOURCES = ["l2norm_scale.hip"]


def bind_library(lib):
    V, I64, F, S = capi.c_void_p, capi.c_int64, capi.c_float, capi.c_size_t
    capi.bind(lib, "l2norm_scale_forward_f32", [V, V, V, V, I64, I64, F, V])
    capi.bind(lib, "l2norm_scale_backward_workspace_bytes", [I64, I64], S)
    capi.bind(lib, "l2norm_scale_backward_f32", [V, V, V, V, V, V, I64, I64, V, S, V])
    capi.bind_last_error(lib, "l2norm_scale_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _check(X, g):
    capi.require(X.is_cuda and g.is_cuda, "X, g must be GPU tensors")
    capi.require(X.dtype == torch.float32 and g.dtype == torch.float32, "X, g must be float32")
    capi.require(X.dim() == 2 and g.dim() == 1 and g.numel() == X.size(1),
                 "X must be [N, D] and g [D]")


def l2n_forward(X, g, eps):
    """(Y, norm): Y = X / sqrt(sum X^2 + eps) * g, norm = sqrt(sum X^2 + eps) per row."""
    _check(X, g)
    lib = _lib()
    X, g = X.contiguous(), g.contiguous()
    N, D = X.shape
    Y = torch.empty_like(X)
    norm = torch.empty(N, dtype=torch.float32, device=X.device)
    with torch.cuda.device(X.device):
        st = lib.l2norm_scale_forward_f32(capi.ptr(X), capi.ptr(g), capi.ptr(Y), capi.ptr(norm),
                                          N, D, float(eps), capi.stream_of(X))
    capi.check(st, lib.l2norm_scale_last_error, "l2n_forward")
    return Y, norm


def l2n_backward(X, g, G, norm):
    """(dX, dg) from upstream G = dL/dY and the forward's norm."""
    _check(X, g)
    capi.require(G.is_cuda and G.dtype == torch.float32 and G.shape == X.shape,
                 "G must be a float32 GPU tensor shaped like X")
    lib = _lib()
    X, g, G, norm = X.contiguous(), g.contiguous(), G.contiguous(), norm.contiguous()
    N, D = X.shape
    dX = torch.empty_like(X)
    dg = torch.empty_like(g)
    ws_bytes = lib.l2norm_scale_backward_workspace_bytes(N, D)
    ws = torch.empty((max(ws_bytes, 4) + 3) // 4, dtype=torch.float32, device=X.device)
    with torch.cuda.device(X.device):
        st = lib.l2norm_scale_backward_f32(capi.ptr(G), capi.ptr(X), capi.ptr(g), capi.ptr(norm),
                                           capi.ptr(dX), capi.ptr(dg), N, D, capi.ptr(ws),
                                           ws_bytes, capi.stream_of(X))
    capi.check(st, lib.l2norm_scale_last_error, "l2n_backward")
    return dX, dg


class L2NormScaleFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, X, g, eps):
        X, g = X.contiguous(), g.contiguous()
        Y, norm = l2n_forward(X, g, float(eps))
        ctx.save_for_backward(X, g, norm)
        return Y

    @staticmethod
    def backward(ctx, G):
        X, g, norm = ctx.saved_tensors
        dX, dg = l2n_backward(X, g, G.contiguous(), norm)
        return dX, dg, None


def candidate(inputs, params):
    """Framework candidate contract: inputs={"X","g"}, params={"eps"} -> Y."""
    return L2NormScaleFunction.apply(inputs["X"], inputs["g"], params["eps"])


def forward_only(inputs, params):
    """Forward without autograd."""
    return l2n_forward(inputs["X"], inputs["g"], float(params["eps"]))[0]
