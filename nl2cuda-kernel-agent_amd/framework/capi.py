"""ctypes plumbing shared by the case ``op`` modules.

Each case library exports plain C functions (see the headers in include/):
device pointers as ``void*``, sizes as ``int64_t``, the HIP stream as a
pointer, and an ``int`` status (0 = success).  ``bind`` attaches argument
and result types; ``check`` turns a non-zero status into the RuntimeError
the reference's TORCH_CHECK failures would have raised.
"""

import ctypes
import os

import torch

c_void_p = ctypes.c_void_p
c_int64 = ctypes.c_int64
c_int = ctypes.c_int
c_float = ctypes.c_float
c_size_t = ctypes.c_size_t
c_double = ctypes.c_double


def bind(lib, name, argtypes, restype=ctypes.c_int):
    fn = getattr(lib, name)
    fn.argtypes = argtypes
    fn.restype = restype
    return fn


def bind_last_error(lib, name):
    fn = getattr(lib, name)
    fn.argtypes = []
    fn.restype = ctypes.c_char_p
    return fn


def check(status, last_error, what):
    if status != 0:
        msg = last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (status {status})")


def ptr(t):
    """Device address of a tensor (0 for an empty tensor)."""
    return ctypes.c_void_p(t.data_ptr() if t.numel() else 0)


def stream_of(t):
    """The current torch stream of the tensor's device, as a HIP stream handle."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require(cond, msg):
    """TORCH_CHECK equivalent for the Python boundary."""
    if not cond:
        raise RuntimeError(msg)


def checking():
    """True when NL2K_CHECK=1: ops then also read the status words their
    kernels leave in the workspace (a synchronisation per call)."""
    return os.environ.get("NL2K_CHECK", "") == "1"
