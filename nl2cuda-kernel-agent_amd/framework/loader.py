"""Builds HIP sources into an in-tree C-ABI shared library and loads it.

Replaces the reference's JIT torch-extension loader (framework/loader.py:39-74,
``torch.utils.cpp_extension.load`` driving nvcc).  Here every case ships a
plain ``extern "C"`` library with no torch headers: ``hipcc
--offload-arch=gfx950 -O3 -shared -fPIC`` writes ``lib<name>.so`` next to the
sources, and ``ctypes`` loads it.  Keeping the library free of the torch C++
ABI means the torch build and the ROCm toolchain can move independently.

Precision policy (same as the reference, loader.py:6-8): no fast-math flags.
Packed fp32 instructions are disabled (``-packed-fp32-ops``).

Build policy: ``build_library`` always compiles.  ``load_kernel`` loads the
library that is already built and compiles only when it is missing.  A
stale library (its recorded fingerprint of sources, shared headers and
flags differs from the current one) is refused with a RuntimeError, so a
run never measures or tests code other than the committed source; setting
``NL2K_ALLOW_STALE=1`` loads it anyway, with a warning on stderr.
"""

import ctypes
import hashlib
import os
import shutil
import subprocess
import sys

FRAMEWORK_DIR = os.path.dirname(os.path.abspath(__file__))
PACKAGE_DIR = os.path.dirname(FRAMEWORK_DIR)
CSRC_DIR = os.path.join(PACKAGE_DIR, "csrc")
INCLUDE_DIR = os.path.join(os.path.dirname(PACKAGE_DIR), "include")

OFFLOAD_ARCH = os.environ.get("NL2K_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

DEFAULT_HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _resolve(sources, base_dir):
    base = base_dir if base_dir is not None else FRAMEWORK_DIR
    out = []
    for s in sources:
        p = s if os.path.isabs(s) else os.path.join(base, s)
        if not os.path.exists(p):
            raise FileNotFoundError(f"source file not found: {p}")
        out.append(p)
    return out


def _fingerprint(paths, flags):
    """Hash of the sources, the shared headers and the flags."""
    h = hashlib.sha256()
    deps = list(paths)
    for d in (CSRC_DIR, INCLUDE_DIR):
        if os.path.isdir(d):
            deps += sorted(os.path.join(d, f) for f in os.listdir(d)
                           if f.endswith((".h", ".hpp")))
    for p in deps:
        h.update(os.path.basename(p).encode())
        with open(p, "rb") as f:
            h.update(f.read())
    h.update(" ".join(f for f in flags if not os.path.isabs(f)).encode())
    return h.hexdigest()


def library_path(name, base_dir):
    return os.path.join(base_dir, f"lib{name}.so")


def _flags(extra_cuda_cflags, extra_cflags):
    flags = list(DEFAULT_HIP_FLAGS) + ["-I", INCLUDE_DIR, "-I", CSRC_DIR]
    if extra_cuda_cflags:
        flags += list(extra_cuda_cflags)
    if extra_cflags:
        flags += list(extra_cflags)
    return flags


def build_library(name, sources, base_dir=None, extra_cuda_cflags=None,
                  extra_cflags=None, verbose=False):
    """Compile ``sources`` into ``<base_dir>/lib<name>.so``; returns the path.

    Raises RuntimeError when hipcc is missing or fails.
    """
    base = base_dir if base_dir is not None else FRAMEWORK_DIR
    paths = _resolve(sources, base)
    flags = _flags(extra_cuda_cflags, extra_cflags)
    out = library_path(name, base)
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}; cannot build lib{name}.so")
    tmp = out + f".tmp{os.getpid()}"
    cmd = [HIPCC] + flags + paths + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise RuntimeError(f"hipcc failed for lib{name}.so:\n{proc.stderr[-4000:]}")
    os.replace(tmp, out)
    with open(out + ".stamp", "w") as f:
        f.write(_fingerprint(paths, flags))
    return out


def is_stale(name, sources, base_dir=None, extra_cuda_cflags=None, extra_cflags=None):
    base = base_dir if base_dir is not None else FRAMEWORK_DIR
    out = library_path(name, base)
    stamp = out + ".stamp"
    if not (os.path.exists(out) and os.path.exists(stamp)):
        return True
    with open(stamp) as f:
        recorded = f.read().strip()
    return recorded != _fingerprint(_resolve(sources, base),
                                    _flags(extra_cuda_cflags, extra_cflags))


def load_library(name, sources, base_dir=None, extra_cuda_cflags=None,
                 extra_cflags=None, verbose=False):
    """Load ``lib<name>.so`` (building it only if it does not exist).

    Does not require a GPU: the HIP runtime initialises lazily, so loading and
    symbol lookup work on a CPU-only host.
    """
    base = base_dir if base_dir is not None else FRAMEWORK_DIR
    out = library_path(name, base)
    if not os.path.exists(out):
        build_library(name, sources, base, extra_cuda_cflags, extra_cflags, verbose)
    elif is_stale(name, sources, base, extra_cuda_cflags, extra_cflags):
        msg = (f"lib{name}.so was built from other sources or flags than the ones in "
               f"{base}; run __graft_entry__.build() to rebuild")
        if os.environ.get("NL2K_ALLOW_STALE", "") != "1":
            raise RuntimeError(msg + " (or set NL2K_ALLOW_STALE=1 to load it anyway)")
        print(f"[loader] warning: {msg}", file=sys.stderr)
    return ctypes.CDLL(out)


def load_kernel(name, sources, base_dir=None, extra_cuda_cflags=None,
                extra_cflags=None, verbose=False):
    """Load a case's HIP library for use on the GPU.

    Same call shape as the reference's ``load_kernel`` (loader.py:39-74) and,
    like it, refuses to run without a GPU -- there is no CPU fallback.
    """
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError(f"lib{name}.so needs an MI355X (gfx950) GPU; "
                           "torch.cuda.is_available() is False")
    return load_library(name, sources, base_dir, extra_cuda_cflags, extra_cflags, verbose)
