"""RBF candidate: autograd wrapper over the HIP library (kernels/rbf.hip).

Mirrors the reference's cases/rbf/op.py:17-49: ``RBFFunction`` saves
(X, Y, K) in forward and returns (dX, dY, None) from backward; ``candidate``
and ``forward_only`` keep the dict interface.  ``rbf_forward`` and
``rbf_backward`` are the Python faces of the C entry points
``rbf_forward_f32`` / ``rbf_backward_f32`` (include/rbf.h), with the
reference's argument checks (cases/rbf/kernels/rbf_forward.cu:95-98,
rbf_backward.cu:61-64).  There is no CPU path: without a GPU the library
refuses to load.
"""

import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "rbf_hip"
SOURCES = ["rbf.hip"]


def bind_library(lib):
    V, I64, F, S = capi.c_void_p, capi.c_int64, capi.c_float, capi.c_size_t
    capi.bind(lib, "rbf_forward_f32", [V, V, V, I64, I64, I64, F, V])
    capi.bind(lib, "rbf_backward_workspace_bytes", [I64, I64, I64], S)
    capi.bind(lib, "rbf_backward_f32", [V, V, V, V, V, V, I64, I64, I64, F, V, S, V])
    capi.bind(lib, "rbf_backward_f32_noalloc", [V, V, V, V, V, V, I64, I64, I64, F, V])
    capi.bind(lib, "rbf_backward_noalloc_max_bytes", [], S)
    capi.bind_last_error(lib, "rbf_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def rbf_forward(X, Y, gamma):
    """K = exp(-gamma * ||X_i - Y_j||^2) on the GPU (fp32)."""
    capi.require(X.is_cuda and Y.is_cuda, "X, Y must be GPU tensors")
    capi.require(X.dtype == torch.float32 and Y.dtype == torch.float32, "X, Y must be float32")
    capi.require(X.dim() == 2 and Y.dim() == 2, "X, Y must be 2D")
    capi.require(X.size(1) == Y.size(1), "X, Y must share feature dim D")
    lib = _lib()
    X = X.contiguous()
    Y = Y.contiguous()
    N, D = X.shape
    M = Y.size(0)
    K = torch.empty((N, M), dtype=torch.float32, device=X.device)
    with torch.cuda.device(X.device):
        st = lib.rbf_forward_f32(capi.ptr(X), capi.ptr(Y), capi.ptr(K), N, M, D,
                                 float(gamma), capi.stream_of(X))
    capi.check(st, lib.rbf_last_error, "rbf_forward")
    return K


def rbf_backward(X, Y, G, K, gamma):
    """(dX, dY) from upstream G = dL/dK and the saved forward output K."""
    capi.require(X.is_cuda and Y.is_cuda and G.is_cuda and K.is_cuda, "inputs must be GPU tensors")
    capi.require(all(t.dtype == torch.float32 for t in (X, Y, G, K)), "inputs must be float32")
    capi.require(X.dim() == 2 and Y.dim() == 2 and X.size(1) == Y.size(1),
                 "X, Y must be 2D with a shared feature dim D")
    capi.require(tuple(G.shape) == (X.size(0), Y.size(0)) and tuple(K.shape) == tuple(G.shape),
                 "G and K must have shape [N, M]")
    lib = _lib()
    X, Y, G, K = X.contiguous(), Y.contiguous(), G.contiguous(), K.contiguous()
    N, D = X.shape
    M = Y.size(0)
    dX = torch.empty_like(X)
    dY = torch.empty_like(Y)
    ws_bytes = lib.rbf_backward_workspace_bytes(N, M, D)
    ws = torch.empty((max(ws_bytes, 4) + 3) // 4, dtype=torch.float32, device=X.device)
    with torch.cuda.device(X.device):
        st = lib.rbf_backward_f32(capi.ptr(X), capi.ptr(Y), capi.ptr(G), capi.ptr(K),
                                  capi.ptr(dX), capi.ptr(dY), N, M, D, float(gamma),
                                  capi.ptr(ws), ws_bytes, capi.stream_of(X))
    capi.check(st, lib.rbf_last_error, "rbf_backward")
    return dX, dY


class RBFFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, X, Y, gamma):
        X = X.contiguous()
        Y = Y.contiguous()
        K = rbf_forward(X, Y, float(gamma))
        ctx.save_for_backward(X, Y, K)  # K is reused by backward
        ctx.gamma = float(gamma)
        return K

    @staticmethod
    def backward(ctx, G):
        X, Y, K = ctx.saved_tensors
        dX, dY = rbf_backward(X, Y, G.contiguous(), K, ctx.gamma)
        return dX, dY, None


def candidate(inputs, params):
    """Framework candidate contract: inputs={"X","Y"}, params={"gamma"} -> K."""
    return RBFFunction.apply(inputs["X"], inputs["Y"], params["gamma"])


def forward_only(inputs, params):
    """Forward without autograd."""
    return rbf_forward(inputs["X"], inputs["Y"], float(params["gamma"]))
