"""LayerNorm candidate: autograd wrapper over liblayernorm_hip.so.

Mirrors the reference's cases/layernorm/op.py:26-64: forward returns y and
saves (x, gamma, mean, inv_std); backward returns (dx, dgamma, dbeta, None);
``candidate(inputs, params)`` reads params["eps"] (default 1e-5).  The
argument checks follow layernorm_forward.cu:214-227 and
layernorm_backward.cu:147-171.  No CPU path: the library refuses to load
without a GPU.
"""

import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "layernorm_hip"
SOURCES = ["layernorm.hip"]


def bind_library(lib):
    V, I64, F, S = capi.c_void_p, capi.c_int64, capi.c_float, capi.c_size_t
    capi.bind(lib, "layernorm_forward_f32", [V, V, V, V, V, V, I64, I64, F, V])
    capi.bind(lib, "layernorm_backward_workspace_bytes", [I64, I64], S)
    capi.bind(lib, "layernorm_backward_f32", [V, V, V, V, V, V, V, V, I64, I64, V, S, V])
    capi.bind_last_error(lib, "layernorm_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _check_inputs(x, gamma, beta):
    capi.require(x.is_cuda and gamma.is_cuda and beta.is_cuda, "X, gamma, beta must be GPU tensors")
    capi.require(all(t.dtype == torch.float32 for t in (x, gamma, beta)),
                 "X, gamma, beta must be float32")
    capi.require(x.dim() == 2, "X must have shape [B, D]")
    capi.require(gamma.dim() == 1 and beta.dim() == 1, "gamma, beta must have shape [D]")
    capi.require(gamma.size(0) == x.size(1), "gamma length must equal D")
    capi.require(beta.size(0) == x.size(1), "beta length must equal D")


def layernorm_forward(x, gamma, beta, eps):
    """Returns (y, mean, inv_std) like the reference extension."""
    _check_inputs(x, gamma, beta)
    lib = _lib()
    x, gamma, beta = x.contiguous(), gamma.contiguous(), beta.contiguous()
    B, D = x.shape
    y = torch.empty_like(x)
    mean = torch.empty(B, dtype=torch.float32, device=x.device)
    rstd = torch.empty(B, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        st = lib.layernorm_forward_f32(capi.ptr(x), capi.ptr(gamma), capi.ptr(beta), capi.ptr(y),
                                       capi.ptr(mean), capi.ptr(rstd), B, D, float(eps),
                                       capi.stream_of(x))
    capi.check(st, lib.layernorm_last_error, "layernorm_forward")
    return y, mean, rstd


def layernorm_backward(grad_y, x, gamma, mean, inv_std):
    """Returns (grad_x, grad_gamma, grad_beta) like the reference extension."""
    capi.require(all(t.is_cuda for t in (grad_y, x, gamma, mean, inv_std)), "inputs must be GPU tensors")
    capi.require(all(t.dtype == torch.float32 for t in (grad_y, x, gamma, mean, inv_std)),
                 "inputs must be float32")
    capi.require(grad_y.shape == x.shape and x.dim() == 2, "grad_y and X must have shape [B, D]")
    capi.require(gamma.dim() == 1 and gamma.size(0) == x.size(1), "gamma length must equal D")
    capi.require(mean.shape == (x.size(0),) and inv_std.shape == (x.size(0),),
                 "mean and inv_std must have shape [B]")
    lib = _lib()
    grad_y, x, gamma = grad_y.contiguous(), x.contiguous(), gamma.contiguous()
    mean, inv_std = mean.contiguous(), inv_std.contiguous()
    B, D = x.shape
    dx = torch.empty_like(x)
    dgamma = torch.empty(D, dtype=torch.float32, device=x.device)
    dbeta = torch.empty(D, dtype=torch.float32, device=x.device)
    ws_bytes = lib.layernorm_backward_workspace_bytes(B, D)
    ws = torch.empty((max(ws_bytes, 16) + 3) // 4, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        st = lib.layernorm_backward_f32(capi.ptr(grad_y), capi.ptr(x), capi.ptr(gamma),
                                        capi.ptr(mean), capi.ptr(inv_std), capi.ptr(dx),
                                        capi.ptr(dgamma), capi.ptr(dbeta), B, D, capi.ptr(ws),
                                        ws_bytes, capi.stream_of(x))
    capi.check(st, lib.layernorm_last_error, "layernorm_backward")
    return dx, dgamma, dbeta


class _LayerNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gamma, beta, eps):
        x_c, gamma_c, beta_c = x.contiguous(), gamma.contiguous(), beta.contiguous()
        y, mean, inv_std = layernorm_forward(x_c, gamma_c, beta_c, float(eps))
        ctx.save_for_backward(x_c, gamma_c, mean, inv_std)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, gamma, mean, inv_std = ctx.saved_tensors
        grad_x, grad_gamma, grad_beta = layernorm_backward(grad_y.contiguous(), x, gamma, mean,
                                                           inv_std)
        return grad_x, grad_gamma, grad_beta, None


def candidate(inputs, params):
    """Framework candidate: inputs={"X","gamma","beta"}, params={"eps"} -> Y."""
    eps = float(params.get("eps", 1.0e-5))
    return _LayerNormFunction.apply(inputs["X"], inputs["gamma"], inputs["beta"], eps)


def forward_only(inputs, params):
    return candidate(inputs, params)
