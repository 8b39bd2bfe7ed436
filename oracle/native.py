"""ctypes bindings of the oracle's C code (TEST INFRASTRUCTURE ONLY).

* ``lib()``     -> oracle/lib/liboracle.so   (csrc/oracle.c, built by `make -C oracle`)
* ``ref_lib()`` -> oracle/_ref/librbf_ref.so (the reference's own CPU loops,
  cases/rbf/delivery/rbf_test.cu:24-52, built by `make -C oracle ref` in the
  container that holds /root/reference; the .so travels with the tree).
Both return None when the library has not been built.
"""

import ctypes
import functools
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
REF_PATH = os.path.join(_HERE, "_ref", "librbf_ref.so")
REF_ROOT = os.environ.get("NL2K_REFERENCE_ROOT", "/root/reference")

_P = ctypes.c_void_p
_I = ctypes.c_int64
_D = ctypes.c_double


def build(with_reference=True):
    """Compile liboracle.so, and librbf_ref.so when the reference is present."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if with_reference and os.path.exists(
            os.path.join(REF_ROOT, "cases/rbf/delivery/rbf_test.cu")):
        subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REF_ROOT={REF_ROOT}"], check=True)
    lib.cache_clear()
    ref_lib.cache_clear()


@functools.lru_cache(maxsize=1)
def lib():
    if not os.path.exists(LIB_PATH):
        return None
    L = ctypes.CDLL(LIB_PATH)
    L.oracle_rbf_forward.argtypes = [_P, _P, _P, _I, _I, _I, _D]
    L.oracle_rbf_backward.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _D]
    L.oracle_scan_i32.argtypes = [_P, _P, _I, _I, ctypes.c_int]
    L.oracle_scan_f32.argtypes = [_P, _P, _I, _I, ctypes.c_int]
    L.oracle_spmm_csr.argtypes = [_P, _P, _P, _P, _P, _I, _I]
    L.oracle_spmm_csr_backward.argtypes = [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I]
    L.oracle_layernorm_forward.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _D]
    return L


@functools.lru_cache(maxsize=1)
def ref_lib():
    if not os.path.exists(REF_PATH):
        return None
    L = ctypes.CDLL(REF_PATH)
    c_int, c_float = ctypes.c_int, ctypes.c_float
    L.ref_rbf_cpu_forward.argtypes = [_P, _P, _P, c_int, c_int, c_int, c_float]
    L.ref_rbf_cpu_backward.argtypes = [_P, _P, _P, _P, _P, _P, c_int, c_int, c_int, c_float]
    return L


def _p(a):
    return a.ctypes.data_as(_P)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def rbf_forward(X, Y, gamma):
    X, Y = _c(X, np.float32), _c(Y, np.float32)
    K = np.empty((X.shape[0], Y.shape[0]), dtype=np.float64)
    lib().oracle_rbf_forward(_p(X), _p(Y), _p(K), X.shape[0], Y.shape[0], X.shape[1], gamma)
    return K


def rbf_backward(X, Y, G, K, gamma):
    X, Y, G = _c(X, np.float32), _c(Y, np.float32), _c(G, np.float32)
    K = _c(K, np.float64)
    dX = np.empty(X.shape, dtype=np.float64)
    dY = np.empty(Y.shape, dtype=np.float64)
    lib().oracle_rbf_backward(_p(X), _p(Y), _p(G), _p(K), _p(dX), _p(dY),
                              X.shape[0], Y.shape[0], X.shape[1], gamma)
    return dX, dY


def scan_i32(x, reverse=False):
    x = _c(x, np.int32)
    y = np.empty(x.shape, dtype=np.int64)
    lib().oracle_scan_i32(_p(x), _p(y), x.shape[0], x.shape[1], int(reverse))
    return y


def scan_f32(x, reverse=False):
    x = _c(x, np.float32)
    y = np.empty(x.shape, dtype=np.float32)
    lib().oracle_scan_f32(_p(x), _p(y), x.shape[0], x.shape[1], int(reverse))
    return y


def spmm_csr(row_ptr, col, vals, X):
    rp, cl = _c(row_ptr, np.int64), _c(col, np.int64)
    v, X = _c(vals, np.float32), _c(X, np.float32)
    M = rp.shape[0] - 1
    Y = np.empty((M, X.shape[1]), dtype=np.float64)
    lib().oracle_spmm_csr(_p(rp), _p(cl), _p(v), _p(X), _p(Y), M, X.shape[1])
    return Y


def spmm_csr_backward(row_ptr, col, vals, X, dY):
    rp, cl = _c(row_ptr, np.int64), _c(col, np.int64)
    v, X, dY = _c(vals, np.float32), _c(X, np.float32), _c(dY, np.float32)
    M = rp.shape[0] - 1
    dX = np.empty(X.shape, dtype=np.float64)
    dv = np.empty(v.shape, dtype=np.float64)
    lib().oracle_spmm_csr_backward(_p(rp), _p(cl), _p(v), _p(X), _p(dY), _p(dX), _p(dv),
                                   M, X.shape[0], X.shape[1])
    return dX, dv


def layernorm_forward(x, w, b, eps):
    x, w, b = _c(x, np.float32), _c(w, np.float32), _c(b, np.float32)
    B, D = x.shape
    y = np.empty((B, D), dtype=np.float64)
    mean = np.empty(B, dtype=np.float64)
    rstd = np.empty(B, dtype=np.float64)
    lib().oracle_layernorm_forward(_p(x), _p(w), _p(b), _p(y), _p(mean), _p(rstd), B, D, eps)
    return y, mean, rstd


def ref_rbf_forward(X, Y, gamma):
    """The reference's cpu_forward (fp32 loops), via oracle/_ref."""
    X, Y = _c(X, np.float32), _c(Y, np.float32)
    K = np.empty((X.shape[0], Y.shape[0]), dtype=np.float32)
    ref_lib().ref_rbf_cpu_forward(_p(X), _p(Y), _p(K), X.shape[0], Y.shape[0], X.shape[1], gamma)
    return K


def ref_rbf_backward(X, Y, G, K, gamma):
    """The reference's cpu_backward (fp32 loops), via oracle/_ref."""
    X, Y, G, K = (_c(a, np.float32) for a in (X, Y, G, K))
    dX = np.empty(X.shape, dtype=np.float32)
    dY = np.empty(Y.shape, dtype=np.float32)
    ref_lib().ref_rbf_cpu_backward(_p(X), _p(Y), _p(G), _p(K), _p(dX), _p(dY),
                                   X.shape[0], Y.shape[0], X.shape[1], gamma)
    return dX, dY
