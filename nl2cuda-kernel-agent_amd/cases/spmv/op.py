"""CSR SpMM / SpMV candidate: autograd wrapper over libspmv_hip.so.

Mirrors the reference's cases/spmv/op.py:24-57: ``_CSRSpMMFunction`` saves
exactly (row_ptr, col_idx, vals, X) and returns (None, None, grad_vals,
grad_X); ``candidate`` / ``forward_only`` keep the dict interface.  The
argument checks follow spmv.cu:167-197 (GPU tensors, fp32 values, 1-D
structure of matching lengths, rank-2 X with positive sizes), with int32
indices accepted beside int64 (row_ptr and col_idx must share the type).
There is no CPU path: without a GPU the library refuses to load.

Opt-in (``params["keep_gather"] = True`` or ``NL2K_SPMV_KEEP_GATHER=1``):
at D == 1 with vals requiring grad, ``_CSRSpMMKeepGatherFunction`` also
saves the gathered X[col_idx] the forward read (nnz floats), so the
backward's dvals streams it instead of gathering X again; gradients are
bit-identical, the forward writes nnz * 4 more bytes.

With ``NL2K_CHECK=1`` every call first checks the CSR structure on the
device and reads the report back (a synchronisation): a column outside
[0, K) raises IndexError, as the reference path's ``X.index_select(0,
col_idx)`` does (cases/spmv/reference.py:19), and a malformed row_ptr
raises RuntimeError; the backward also zeroes and reads back the
workspace's trip counter on shapes that build the column-major copy of A.
"""

import ctypes
import functools
import os

import torch

from framework import capi
from framework.loader import load_kernel

KERNEL_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels")
LIB_NAME = "spmv_hip"
SOURCES = ["spmv.hip"]
SIZE_MAX = ctypes.c_size_t(-1).value


def bind_library(lib):
    V, I64 = capi.c_void_p, capi.c_int64
    for t in ("i32", "i64"):
        capi.bind(lib, f"spmv_forward_f32_{t}", [V, V, V, V, V, I64, I64, I64, I64, V])
        capi.bind(lib, f"spmv_forward_gather_f32_{t}", [V, V, V, V, V, V, I64, I64, I64, I64, V])
        capi.bind(lib, f"spmv_backward_f32_{t}",
                  [V, V, V, V, V, V, V, I64, I64, I64, I64, V, capi.c_size_t, V])
        capi.bind(lib, f"spmv_backward_gathered_f32_{t}",
                  [V, V, V, V, V, V, V, V, I64, I64, I64, I64, V, capi.c_size_t, V])
        capi.bind(lib, f"spmv_check_structure_{t}", [V, V, I64, I64, I64, V, V])
    capi.bind(lib, "spmv_backward_workspace_bytes", [I64, I64, I64, I64], restype=capi.c_size_t)
    capi.bind(lib, "spmv_status_offset", [I64, I64, I64, I64], restype=capi.c_size_t)
    capi.bind_last_error(lib, "spmv_last_error")
    return lib


@functools.lru_cache(maxsize=1)
def _lib():
    return bind_library(load_kernel(LIB_NAME, SOURCES, base_dir=KERNEL_DIR))


def _suffix(row_ptr, col_idx):
    capi.require(row_ptr.dtype == col_idx.dtype, "row_ptr and col_idx must share a dtype")
    capi.require(row_ptr.dtype in (torch.int32, torch.int64), "row_ptr must be int64 or int32")
    return "i32" if row_ptr.dtype == torch.int32 else "i64"


def _validate(row_ptr, col_idx, vals, X):
    for name, t in (("row_ptr", row_ptr), ("col_idx", col_idx), ("vals", vals), ("X", X)):
        capi.require(t.is_cuda, f"{name} must be a GPU tensor")
    capi.require(vals.dtype == torch.float32, "vals must be float32")
    capi.require(X.dtype == torch.float32, "X must be float32")
    capi.require(X.dim() == 2, "X must be a rank-2 tensor")
    capi.require(X.size(0) > 0 and X.size(1) > 0, "X dimensions must be positive")
    capi.require(row_ptr.dim() == 1 and row_ptr.numel() >= 1, "row_ptr must have shape [M + 1]")
    capi.require(col_idx.dim() == 1, "col_idx must have shape [nnz]")
    capi.require(vals.dim() == 1, "vals must have shape [nnz]")
    capi.require(col_idx.numel() == vals.numel(), "col_idx and vals must have the same length")
    return _suffix(row_ptr, col_idx)


def check_structure(row_ptr, col_idx, K):
    """Checks the CSR structure on the device (one read-back) and raises
    what the reference path would: IndexError for a column outside [0, K),
    RuntimeError for a row_ptr that does not start at 0, decreases or does
    not end at nnz."""
    t = _suffix(row_ptr, col_idx)
    lib = _lib()
    M, nnz = row_ptr.numel() - 1, col_idx.numel()
    report = torch.empty(4, dtype=torch.int64, device=row_ptr.device)
    with torch.cuda.device(row_ptr.device):
        st = getattr(lib, f"spmv_check_structure_{t}")(
            capi.ptr(row_ptr), capi.ptr(col_idx), M, K, nnz, capi.ptr(report),
            capi.stream_of(row_ptr))
    capi.check(st, lib.spmv_last_error, "spmv_check_structure")
    flags, bad_pos, bad_row, _ = (v & 0xFFFFFFFFFFFFFFFF for v in report.cpu().tolist())
    if flags & 8:
        c = int(col_idx[bad_pos].item())
        raise IndexError(f"spmv: index out of range: col_idx[{bad_pos}] = {c} is not in "
                         f"[0, {K}) (X has {K} rows)")
    if flags:
        what = []
        if flags & 1:
            what.append("row_ptr[0] != 0")
        if flags & 2:
            what.append("row_ptr decreases or leaves [0, nnz]")
        if flags & 4:
            what.append(f"row_ptr[M] != nnz ({nnz})")
        raise RuntimeError(f"spmv: malformed CSR structure: {', '.join(what)} "
                           f"(first at row_ptr[{bad_row}])")


def spmv_forward(row_ptr, col_idx, vals, X, keep_gather=False):
    """Y = A X.  keep_gather=True (D == 1 only) also returns Xg [nnz] =
    X[col_idx] as the kernel read it, for spmv_backward(..., X_gathered=Xg)."""
    t = _validate(row_ptr, col_idx, vals, X)
    lib = _lib()
    row_ptr, col_idx, vals, X = (a.contiguous() for a in (row_ptr, col_idx, vals, X))
    M = row_ptr.numel() - 1
    K, D = X.shape
    if capi.checking() and not torch.cuda.is_current_stream_capturing():
        check_structure(row_ptr, col_idx, K)
    Y = torch.empty((M, D), dtype=torch.float32, device=X.device)
    if keep_gather:
        capi.require(D == 1, "keep_gather needs D == 1")
        Xg = torch.empty_like(vals)
    with torch.cuda.device(X.device):
        if keep_gather:
            st = getattr(lib, f"spmv_forward_gather_f32_{t}")(
                capi.ptr(row_ptr), capi.ptr(col_idx), capi.ptr(vals), capi.ptr(X), capi.ptr(Y),
                capi.ptr(Xg), M, K, D, vals.numel(), capi.stream_of(X))
        else:
            st = getattr(lib, f"spmv_forward_f32_{t}")(
                capi.ptr(row_ptr), capi.ptr(col_idx), capi.ptr(vals), capi.ptr(X), capi.ptr(Y),
                M, K, D, vals.numel(), capi.stream_of(X))
    capi.check(st, lib.spmv_last_error, "spmv_forward")
    return (Y, Xg) if keep_gather else Y


def spmv_backward(row_ptr, col_idx, vals, X, grad_Y, need_vals=True, need_X=True,
                  X_gathered=None):
    """(grad_vals, grad_X).  X_gathered: the Xg spmv_forward(...,
    keep_gather=True) returned for the same inputs; dvals then reads it
    instead of gathering X (bit-identical results)."""
    t = _validate(row_ptr, col_idx, vals, X)
    if X_gathered is not None:
        capi.require(X.size(1) == 1, "X_gathered needs D == 1")
        capi.require(X_gathered.is_cuda and X_gathered.dtype == torch.float32 and
                     X_gathered.shape == vals.shape, "X_gathered must be a float32 GPU [nnz] tensor")
        X_gathered = X_gathered.contiguous()
    capi.require(grad_Y.is_cuda and grad_Y.dtype == torch.float32, "grad_Y must be a float32 GPU tensor")
    M = row_ptr.numel() - 1
    capi.require(grad_Y.dim() == 2 and grad_Y.size(0) == M and grad_Y.size(1) == X.size(1),
                 "grad_Y must have shape [M, D]")
    lib = _lib()
    row_ptr, col_idx, vals, X, grad_Y = (a.contiguous() for a in (row_ptr, col_idx, vals, X, grad_Y))
    K, D = X.shape
    if capi.checking() and not torch.cuda.is_current_stream_capturing():
        check_structure(row_ptr, col_idx, K)
    grad_vals = torch.empty_like(vals) if need_vals else None
    grad_X = torch.empty_like(X) if need_X else None
    ws_bytes = lib.spmv_backward_workspace_bytes(M, K, D, vals.numel()) if need_X else 0
    ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=X.device)  # scratch
    status = None
    if need_X and capi.checking() and not torch.cuda.is_current_stream_capturing():
        off = lib.spmv_status_offset(M, K, D, vals.numel())
        if off != SIZE_MAX:
            status = ws[off:off + 8].view(torch.int64)
            status.zero_()
    outs = (capi.ptr(grad_vals) if need_vals else None, capi.ptr(grad_X) if need_X else None)
    with torch.cuda.device(X.device):
        if X_gathered is not None:
            st = getattr(lib, f"spmv_backward_gathered_f32_{t}")(
                capi.ptr(row_ptr), capi.ptr(col_idx), capi.ptr(vals), capi.ptr(X),
                capi.ptr(X_gathered), capi.ptr(grad_Y), *outs, M, K, D, vals.numel(),
                capi.ptr(ws), ws_bytes, capi.stream_of(X))
        else:
            st = getattr(lib, f"spmv_backward_f32_{t}")(
                capi.ptr(row_ptr), capi.ptr(col_idx), capi.ptr(vals), capi.ptr(X),
                capi.ptr(grad_Y), *outs, M, K, D, vals.numel(), capi.ptr(ws), ws_bytes,
                capi.stream_of(X))
    capi.check(st, lib.spmv_last_error, "spmv_backward")
    if status is not None:
        trips = int(status.item()) & 0xFFFFFFFF
        capi.require(trips == 0, "spmv_backward: a column-total wait hit its spin cap")
    return grad_vals, grad_X


class _CSRSpMMFunction(torch.autograd.Function):
    """The reference's autograd contract (cases/spmv/op.py:24-40): saves
    (row_ptr, col_idx, vals, X); backward returns (None, None, grad_vals,
    grad_X)."""

    @staticmethod
    def forward(ctx, row_ptr, col_idx, vals, X):
        row_ptr = row_ptr.contiguous()
        col_idx = col_idx.contiguous()
        vals = vals.contiguous()
        X = X.contiguous()
        Y = spmv_forward(row_ptr, col_idx, vals, X)
        ctx.save_for_backward(row_ptr, col_idx, vals, X)
        return Y

    @staticmethod
    def backward(ctx, grad_output):
        row_ptr, col_idx, vals, X = ctx.saved_tensors
        grad_vals, grad_X = spmv_backward(row_ptr, col_idx, vals, X, grad_output.contiguous(),
                                          need_vals=ctx.needs_input_grad[2],
                                          need_X=ctx.needs_input_grad[3])
        return None, None, grad_vals, grad_X


class _CSRSpMMKeepGatherFunction(torch.autograd.Function):
    """Opt-in variant (no counterpart in the reference): at D == 1 with vals
    requiring grad the forward also saves Xg = X[col_idx] as it read it, a
    fifth saved tensor of nnz floats, and the backward's dvals streams Xg
    instead of gathering X; gradients are bit-identical to
    _CSRSpMMFunction's.  Other shapes save the reference's four tensors."""

    @staticmethod
    def forward(ctx, row_ptr, col_idx, vals, X):
        row_ptr = row_ptr.contiguous()
        col_idx = col_idx.contiguous()
        vals = vals.contiguous()
        X = X.contiguous()
        keep = X.dim() == 2 and X.size(1) == 1 and ctx.needs_input_grad[2] and vals.numel() > 0
        if keep:
            Y, Xg = spmv_forward(row_ptr, col_idx, vals, X, keep_gather=True)
            ctx.save_for_backward(row_ptr, col_idx, vals, X, Xg)
        else:
            Y = spmv_forward(row_ptr, col_idx, vals, X)
            ctx.save_for_backward(row_ptr, col_idx, vals, X)
        return Y

    @staticmethod
    def backward(ctx, grad_output):
        row_ptr, col_idx, vals, X, *kept = ctx.saved_tensors
        grad_vals, grad_X = spmv_backward(row_ptr, col_idx, vals, X, grad_output.contiguous(),
                                          need_vals=ctx.needs_input_grad[2],
                                          need_X=ctx.needs_input_grad[3],
                                          X_gathered=kept[0] if kept else None)
        return None, None, grad_vals, grad_X


def keep_gather_requested(params=None):
    """The opt-in of _CSRSpMMKeepGatherFunction: params["keep_gather"], else
    NL2K_SPMV_KEEP_GATHER=1 in the environment."""
    if params and "keep_gather" in params:
        return bool(params["keep_gather"])
    return os.environ.get("NL2K_SPMV_KEEP_GATHER", "") == "1"


def candidate(inputs, params):
    fn = _CSRSpMMKeepGatherFunction if keep_gather_requested(params) else _CSRSpMMFunction
    return fn.apply(inputs["row_ptr"], inputs["col_idx"], inputs["vals"], inputs["X"])


def forward_only(inputs, params):
    del params
    return spmv_forward(inputs["row_ptr"], inputs["col_idx"], inputs["vals"], inputs["X"])
