"""Scan candidate: autograd wrapper over libscan_hip.so (kernels/scan.hip).

Mirrors the reference's cases/scan/op.py:22-37: ``_ScanFunction`` returns
the forward scan and backward returns the reverse scan of the upstream
gradient; ``candidate`` and ``forward_only`` keep the dict interface.  The
argument checks follow scan.cu:67-80 (GPU tensor, 2-D, at least one row),
widened to any D >= 1 and to int32 input (-> int64 output, as torch.cumsum).
There is no CPU path: without a GPU the library refuses to load.

With ``NL2K_CHECK=1`` in the environment every call also zeroes the
workspace's trip counter first and reads it after (a synchronisation), and
raises if a chunk's wait for its predecessors hit the kernel's spin cap.
"""

import ctypes
import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "scan_hip"
SOURCES = ["scan.hip"]
SIZE_MAX = ctypes.c_size_t(-1).value


def bind_library(lib):
    V, I64, S = capi.c_void_p, capi.c_int64, capi.c_size_t
    capi.bind(lib, "scan_workspace_bytes", [I64, I64], S)
    capi.bind(lib, "scan_status_offset", [I64, I64], S)
    capi.bind(lib, "scan_launch_grid", [I64, I64, I64], I64)
    for name in ("scan_forward_f32", "scan_backward_f32", "scan_forward_i32_i64",
                 "scan_forward_i32"):
        capi.bind(lib, name, [V, V, I64, I64, V, S, V])
    capi.bind_last_error(lib, "scan_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _check(x, what, dtypes):
    capi.require(x.is_cuda, f"{what} expects a GPU tensor")
    capi.require(x.dtype in dtypes, f"{what} only supports " + " / ".join(str(d) for d in dtypes))
    capi.require(x.dim() == 2, f"{what} expects a 2D tensor")
    capi.require(x.size(0) > 0, f"{what} expects at least one row")
    capi.require(x.size(1) > 0, f"{what} expects a non-empty last dimension")


_WORKSPACES = {}


def _workspace(device, stream, nbytes):
    """The workspace kept for (device, stream), allocated only when a larger
    one is needed (the kernels need no initial contents).  While the stream
    is being captured into a graph every call gets a fresh workspace, which
    the graph's memory pool then owns: a graph keeps the address it was
    captured with, so it must not share one that a later eager call could
    replace and free, nor one with another graph captured on the same
    (shared capture) stream."""
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max((nbytes + 7) // 8, 1), dtype=torch.int64, device=device)
    key = (device.index, stream.value)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() * 8 < nbytes:
        ws = torch.empty(max((nbytes + 7) // 8, 1), dtype=torch.int64, device=device)
        _WORKSPACES[key] = ws
    return ws


def _call(fn_name, x, out_dtype, what):
    lib = _lib()
    x = x.contiguous()
    rows, d = x.shape
    y = torch.empty((rows, d), dtype=out_dtype, device=x.device)
    ws_bytes = lib.scan_workspace_bytes(rows, d)
    ws = _workspace(x.device, capi.stream_of(x), ws_bytes)
    status = None
    if capi.checking() and not torch.cuda.is_current_stream_capturing():
        off = lib.scan_status_offset(rows, d)
        if off != SIZE_MAX:
            status = ws[off // 8:off // 8 + 1]
            status.zero_()
    with torch.cuda.device(x.device):
        st = getattr(lib, fn_name)(capi.ptr(x), capi.ptr(y), rows, d, capi.ptr(ws),
                                   ws.numel() * 8, capi.stream_of(x))
    capi.check(st, lib.scan_last_error, what)
    if status is not None:
        trips = int(status.item()) & 0xFFFFFFFF
        capi.require(trips == 0, f"{what}: {trips} chunk(s) hit the carry-wait spin cap "
                                 "(fewer workgroups resident than the device reports)")
    return y


def scan_forward(x):
    """Inclusive scan over the last dim: float32 -> float32, int32 -> int64."""
    _check(x, "scan_forward", (torch.float32, torch.int32))
    if x.dtype == torch.int32:
        return _call("scan_forward_i32_i64", x, torch.int64, "scan_forward")
    return _call("scan_forward_f32", x, torch.float32, "scan_forward")


def scan_forward_int32(x):
    """int32 -> int32 inclusive scan, wrapping modulo 2^32."""
    _check(x, "scan_forward_int32", (torch.int32,))
    return _call("scan_forward_i32", x, torch.int32, "scan_forward_int32")


def scan_backward(grad_output):
    """Reverse inclusive scan (the gradient of scan_forward), float32."""
    _check(grad_output, "scan_backward", (torch.float32,))
    return _call("scan_backward_f32", grad_output, torch.float32, "scan_backward")


class _ScanFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return scan_forward(x.contiguous())

    @staticmethod
    def backward(ctx, grad_out):
        return scan_backward(grad_out.contiguous())


def candidate(inputs, params):
    return _ScanFunction.apply(inputs["X"])


def forward_only(inputs, params):
    return scan_forward(inputs["X"].contiguous())
