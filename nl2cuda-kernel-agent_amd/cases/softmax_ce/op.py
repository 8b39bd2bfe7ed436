"""Softmax cross-entropy candidate: autograd wrapper over the HIP library
(kernels/softmax_ce.hip).

Mirrors the reference's cases/softmax_ce/op.py:27-46: ``SoftmaxCEFunction``
returns the scalar loss and returns (dlogits, None); the upstream gradient
is handed to the kernel as a one-element device tensor.  Unlike the
reference, the forward also saves each row's log-sum-exp, so the backward
is one streaming pass.  ``candidate`` and ``forward_only`` keep the dict
interface.  There is no CPU path: without a GPU the library refuses to load.
With ``NL2K_CHECK=1`` the forward also zeroes and reads back the
workspace's trip counter (a synchronisation) and raises if workgroup 0's
wait for the partial losses hit its spin cap.
"""

import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "softmax_ce_hip"
SOURCES = ["softmax_ce.hip"]


def bind_library(lib):
    V, I64, S = capi.c_void_p, capi.c_int64, capi.c_size_t
    capi.bind(lib, "softmax_ce_forward_workspace_bytes", [I64, I64], S)
    capi.bind(lib, "softmax_ce_status_offset", [], S)
    capi.bind(lib, "softmax_ce_forward_f32", [V, V, V, V, I64, I64, V, S, V])
    capi.bind(lib, "softmax_ce_backward_f32", [V, V, V, V, V, I64, I64, V])
    capi.bind_last_error(lib, "softmax_ce_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _check(logits, labels):
    capi.require(logits.is_cuda and labels.is_cuda, "logits, labels must be GPU tensors")
    capi.require(logits.dtype == torch.float32, "logits must be float32")
    capi.require(labels.dtype == torch.int64, "labels must be int64")
    capi.require(logits.dim() == 2 and labels.dim() == 1 and labels.numel() == logits.size(0),
                 "logits must be [B, C] and labels [B]")


def sce_forward(logits, labels):
    """(loss, lse): loss = mean_b (lse[b] - logits[b, labels[b]]), lse per row."""
    _check(logits, labels)
    lib = _lib()
    logits, labels = logits.contiguous(), labels.contiguous()
    B, C = logits.shape
    loss = torch.empty((), dtype=torch.float32, device=logits.device)
    lse = torch.empty(B, dtype=torch.float32, device=logits.device)
    ws_bytes = lib.softmax_ce_forward_workspace_bytes(B, C)
    ws = torch.empty((ws_bytes + 7) // 8, dtype=torch.int64, device=logits.device)
    status = None
    if capi.checking() and not torch.cuda.is_current_stream_capturing():
        off = lib.softmax_ce_status_offset() // 8
        status = ws[off:off + 1]
        status.zero_()
    with torch.cuda.device(logits.device):
        st = lib.softmax_ce_forward_f32(capi.ptr(logits), capi.ptr(labels), capi.ptr(loss),
                                        capi.ptr(lse), B, C, capi.ptr(ws), ws_bytes,
                                        capi.stream_of(logits))
    capi.check(st, lib.softmax_ce_last_error, "sce_forward")
    if status is not None:
        trips = int(status.item()) & 0xFFFFFFFF
        capi.require(trips == 0, "sce_forward: the partial-loss wait hit its spin cap")
    return loss, lse


def sce_backward(logits, labels, lse, gout):
    """dlogits = gout / B * (softmax - onehot(labels)), gout a one-element tensor."""
    _check(logits, labels)
    capi.require(gout.is_cuda and gout.dtype == torch.float32 and gout.numel() == 1,
                 "gout must be a one-element float32 GPU tensor")
    lib = _lib()
    logits, labels, lse = logits.contiguous(), labels.contiguous(), lse.contiguous()
    g = gout.reshape(1).contiguous()
    B, C = logits.shape
    dlogits = torch.empty_like(logits)
    with torch.cuda.device(logits.device):
        st = lib.softmax_ce_backward_f32(capi.ptr(logits), capi.ptr(labels), capi.ptr(lse),
                                         capi.ptr(g), capi.ptr(dlogits), B, C,
                                         capi.stream_of(logits))
    capi.check(st, lib.softmax_ce_last_error, "sce_backward")
    return dlogits


class SoftmaxCEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels):
        logits, labels = logits.contiguous(), labels.contiguous()
        loss, lse = sce_forward(logits, labels)
        ctx.save_for_backward(logits, labels, lse)
        return loss

    @staticmethod
    def backward(ctx, gout):
        logits, labels, lse = ctx.saved_tensors
        return sce_backward(logits, labels, lse, gout), None


def candidate(inputs, params):
    """Framework candidate contract: inputs={"logits","labels"} -> scalar loss."""
    return SoftmaxCEFunction.apply(inputs["logits"], inputs["labels"])


def forward_only(inputs, params):
    """Forward without autograd."""
    return sce_forward(inputs["logits"], inputs["labels"])[0]
