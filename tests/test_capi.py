"""C-ABI checks that need no GPU: every library loads, exports every symbol
its header in include/ declares, and rejects bad arguments with the right
NL2K_* status before touching the device."""

import ctypes
import os
import re

import pytest

from framework import loader

import __graft_entry__ as entry

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")

# header -> op module that loads the library implementing it
HEADERS = {"rbf.h": "cases.rbf.op", "layernorm.h": "cases.layernorm.op",
           "scan.h": "cases.scan.op", "spmv.h": "cases.spmv.op",
           "cosine_sim.h": "cases.cosine_sim.op", "l2norm_scale.h": "cases.l2norm_scale.op",
           "softmax_ce.h": "cases.softmax_ce.op"}

STATUS = {}
with open(os.path.join(INCLUDE, "nl2k_status.h")) as _f:
    for _name, _val in re.findall(r"#define\s+(NL2K_\w+)\s+\(?(-?\d+)\)?", _f.read()):
        STATUS[_name] = int(_val)


def declared_functions(header):
    with open(os.path.join(INCLUDE, header)) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"#[^\n]*", "", text)
    return sorted(set(re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{)]*(?:\([^)]*\)[^;{)]*)*\)\s*;", text)))


def _load(modname):
    import importlib
    mod = importlib.import_module(modname)
    lib = loader.load_library(mod.LIB_NAME, mod.SOURCES, mod.KERNEL_DIR,
                              extra_cuda_cflags=getattr(mod, "EXTRA_CUDA_CFLAGS", None))
    return mod.bind_library(lib)


def test_every_op_module_has_a_header():
    assert sorted(HEADERS.values()) == sorted(entry.OP_MODULES)


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_library_exports_every_declared_symbol(header):
    names = declared_functions(header)
    assert names, f"no declarations parsed from {header}"
    lib = _load(HEADERS[header])
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{header}: not exported: {missing}"


def test_rbf_argument_validation_without_gpu():
    lib = _load("cases.rbf.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    null = None
    st = lib.rbf_forward_f32(fake, fake, fake, -1, 4, 64, 0.5, null)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"N >= 0" in lib.rbf_last_error()
    st = lib.rbf_forward_f32(fake, fake, fake, 4, 4, 0, 0.5, null)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.rbf_forward_f32(null, fake, fake, 4, 4, 64, 0.5, null)
    assert st == STATUS["NL2K_ERR_NULL"]
    st = lib.rbf_forward_f32(fake, fake, fake, 1 << 40, 4, 64, 0.5, null)
    assert st == STATUS["NL2K_ERR_OVERFLOW"]
    # empty problem: nothing to do, success without any launch
    assert lib.rbf_forward_f32(null, null, null, 0, 5, 64, 0.5, null) == 0
    assert lib.rbf_last_error() == b""
    # backward: workspace too small is reported before any launch
    need = lib.rbf_backward_workspace_bytes(4096, 4096, 64)
    assert need == (16 * 4096 + 16 * 4096) * 65 * 4
    st = lib.rbf_backward_f32(fake, fake, fake, fake, fake, fake, 4096, 4096, 64, 0.5,
                              null, 0, null)
    assert st == STATUS["NL2K_ERR_WORKSPACE"] and b"workspace" in lib.rbf_last_error()
    st = lib.rbf_backward_f32(null, fake, fake, fake, fake, fake, 8, 8, 64, 0.5, null, 0, null)
    assert st == STATUS["NL2K_ERR_NULL"]


def test_rbf_noalloc_rejects_shapes_beyond_its_scratch_without_gpu():
    """The no-alloc backward serves shapes whose workspace fits the 64 MiB
    scratch compiled into the library; larger ones fail before any HIP call."""
    lib = _load("cases.rbf.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    cap = lib.rbf_backward_noalloc_max_bytes()
    assert cap == 64 << 20
    assert lib.rbf_backward_workspace_bytes(4096, 4096, 64) <= cap
    assert lib.rbf_backward_workspace_bytes(8192, 8192, 64) > cap
    st = lib.rbf_backward_f32_noalloc(fake, fake, fake, fake, fake, fake, 8192, 8192, 64, 0.5,
                                      None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"] and b"scratch" in lib.rbf_last_error()
    st = lib.rbf_backward_f32_noalloc(fake, fake, fake, fake, fake, fake, -1, 8, 64, 0.5, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]


def test_rbf_workspace_plan():
    lib = _load("cases.rbf.op")
    # Per region slot: a [rows, 64] partial contraction plus a [rows] partial
    # row/column sum of W.  2048: 128-edge regions -> 16 x 16 slots;
    # 8192: 256-edge regions -> 32 x 32; 64 x 64: a single region.
    assert lib.rbf_backward_workspace_bytes(2048, 2048, 64) == 2 * 16 * 2048 * 65 * 4
    assert lib.rbf_backward_workspace_bytes(8192, 8192, 64) == 2 * 32 * 8192 * 65 * 4
    assert lib.rbf_backward_workspace_bytes(64, 64, 64) == 2 * 64 * 65 * 4
    # other feature widths use the generic kernels: each side's walk in
    # slices, 64-aligned, about 1024 workgroups a side.  4096^2, D = 32: 64
    # row tiles x 1 feature pass -> 16 slices of 256, each a [rows, D]
    # partial plus a [rows] partial sum, for both sides
    assert lib.rbf_backward_workspace_bytes(4096, 4096, 32) == 2 * 16 * 4096 * 33 * 4
    # 100 x 70, D = 200: 2 x 4 tiles, 2 slices of 64 columns for dX; 2 x 4
    # tiles, 2 slices of 64 rows for dY
    assert lib.rbf_backward_workspace_bytes(100, 70, 200) == (2 * 100 + 2 * 70) * 201 * 4


def test_loader_refuses_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from cases.rbf import op
    op._lib.cache_clear()
    with pytest.raises(RuntimeError, match="needs an MI355X"):
        op._lib()


def test_scan_argument_validation_and_plan_without_gpu():
    lib = _load("cases.scan.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    st = lib.scan_forward_f32(fake, fake, -1, 16, None, 0, None)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"rows" in lib.scan_last_error()
    st = lib.scan_backward_f32(fake, fake, 4, 0, None, 0, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.scan_forward_i32_i64(fake, fake, 2, 2**31, None, 0, None)
    assert st == STATUS["NL2K_ERR_OVERFLOW"]
    st = lib.scan_forward_f32(None, fake, 4, 16, None, 0, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    # rows of one 4096-element chunk need no workspace; longer rows need one
    # two-word (16-byte) slot per chunk and one word
    assert lib.scan_workspace_bytes(4096, 4096) == 0
    assert lib.scan_workspace_bytes(64, 65536) == 64 * 16 * 16 + 8
    # 2^21 + 5 elements: 513 tiles -> 171 chunks of 3
    assert lib.scan_workspace_bytes(2, 2**21 + 5) == 2 * 171 * 16 + 8
    need = lib.scan_workspace_bytes(64, 65536)
    st = lib.scan_forward_f32(fake, fake, 64, 65536, fake, need - 8, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"]
    assert lib.scan_forward_f32(fake, fake, 0, 65536, None, 0, None) == 0  # nothing to do
    # the trip counter sits in the word after the slots
    SIZE_MAX = ctypes.c_size_t(-1).value
    assert lib.scan_status_offset(64, 65536) == 64 * 16 * 16
    assert lib.scan_status_offset(2, 2**21 + 5) == 2 * 171 * 16
    assert lib.scan_status_offset(4096, 4096) == SIZE_MAX  # single-chunk rows: no workspace
    assert lib.scan_status_offset(-1, 4) == SIZE_MAX


@pytest.mark.parametrize("resident", [1, 3, 64, 1024, 4096])
def test_scan_launch_grid_never_exceeds_residency(resident):
    """Multi-chunk rows wait on their predecessors, so their grid may not
    exceed the resident workgroup count (a device with fewer CUs, or lower
    occupancy, gets a smaller grid and a persistent loop); single-chunk rows
    never wait and take one workgroup per row."""
    lib = _load("cases.scan.op")
    for rows, d in [(64, 65536), (128, 65536), (1, 1 << 20), (2, (1 << 21) + 5), (700, 8192)]:
        nchunk = -(-d // 4096)
        if nchunk > 256:
            nchunk = -(-nchunk // -(-nchunk // 256))
        total = rows * nchunk
        assert lib.scan_launch_grid(rows, d, resident) == min(total, resident), (rows, d)
    assert lib.scan_launch_grid(4096, 4096, resident) == 4096  # single chunks: uncapped
    assert lib.scan_launch_grid(3, 100, resident) == 3
    assert lib.scan_launch_grid(0, 65536, resident) == 0
    assert lib.scan_launch_grid(64, 65536, 0) == -1
    assert lib.scan_launch_grid(-1, 65536, resident) == -1


def test_spmv_argument_validation_without_gpu():
    lib = _load("cases.spmv.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    st = lib.spmv_forward_f32_i32(fake, fake, fake, fake, fake, -1, 4, 1, 0, None)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"M >= 0" in lib.spmv_last_error()
    st = lib.spmv_forward_f32_i64(fake, fake, fake, fake, fake, 4, 0, 1, 0, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.spmv_forward_f32_i32(fake, fake, fake, fake, fake, 4, 4, 1, 2**31, None)
    assert st == STATUS["NL2K_ERR_OVERFLOW"]
    st = lib.spmv_forward_f32_i64(None, fake, fake, fake, fake, 4, 4, 1, 8, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    st = lib.spmv_backward_f32_i32(fake, None, fake, fake, fake, fake, fake, 4, 4, 1, 8, fake,
                                   1 << 20, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    assert lib.spmv_forward_f32_i32(fake, fake, fake, fake, fake, 0, 4, 1, 0, None) == 0
    # dX at D == 1 is summed by column bucket in a workspace: contributions
    # (4 B) and low column bits (2 B) per nonzero, then nb + 1 int64 segment
    # offsets per 8192-position tile, each 256-byte aligned, then one int64
    # row per tile boundary; 2^20 columns -> 256 buckets of 4096
    nnz, K = 16 * 2**20, 2**20
    tiles = nnz // 8192
    assert lib.spmv_backward_workspace_bytes(K, K, 1, nnz) == (
        4 * nnz + 2 * nnz + tiles * 257 * 8 + (tiles + 1) * 8)
    # 1 bucket, 1 tile
    assert lib.spmv_backward_workspace_bytes(100, 7, 1, 10) == 256 + 256 + 256 + 2 * 8
    assert lib.spmv_backward_workspace_bytes(K, K, 64, nnz) == 0  # D > 1, K > 16384: atomics
    # D > 1 with K <= 16384: the column-major copy of A (trip counter and look-back
    # slots first, then chunk offsets, colptr, 16-byte {row, position, value} records)
    n2 = 64 * 4096
    ws2 = lib.spmv_backward_workspace_bytes(4096, 4096, 64, n2)
    def a256(b):
        return (b + 255) // 256 * 256
    chunks = n2 // 1024  # 1024 positions per chunk, int32 chunk counts; 8-byte indices
    assert ws2 == 256 + a256(256 * 16) + a256(chunks * 4096 * 4) + a256(4097 * 8) \
        + a256(n2 * 16)
    assert lib.spmv_status_offset(4096, 4096, 64, n2) == 0
    SIZE_MAX = ctypes.c_size_t(-1).value
    assert lib.spmv_status_offset(K, K, 1, nnz) == SIZE_MAX  # D == 1: bucket route
    assert lib.spmv_status_offset(4096, 20000, 8, 1000) == SIZE_MAX  # > 16384 columns
    assert lib.spmv_backward_workspace_bytes(4096, 20000, 8, 1000) == 0
    assert lib.spmv_backward_workspace_bytes(K, K, 1, 0) == 0
    assert lib.spmv_backward_workspace_bytes(4, 2**25, 1, 8) == 0  # > 1024 buckets of 16384
    need = lib.spmv_backward_workspace_bytes(4, 4, 1, 8)
    st = lib.spmv_backward_f32_i32(fake, fake, fake, fake, fake, fake, fake, 4, 4, 1, 8, fake,
                                   need - 1, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"]
    st = lib.spmv_backward_f32_i64(fake, fake, fake, fake, fake, fake, fake, 4, 4, 1, 8,
                                   ctypes.c_void_p((1 << 20) + 16), need, None)
    assert st == STATUS["NL2K_ERR_ALIGN"]


def test_spmv_gathered_entry_points_validate_without_gpu():
    lib = _load("cases.spmv.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    # the gathered copy of X exists only at D == 1
    st = lib.spmv_forward_gather_f32_i32(fake, fake, fake, fake, fake, fake, 4, 4, 2, 8, None)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"D == 1" in lib.spmv_last_error()
    st = lib.spmv_backward_gathered_f32_i64(fake, fake, fake, fake, fake, fake, fake, fake, 4, 4,
                                            3, 8, fake, 1 << 20, None)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"D == 1" in lib.spmv_last_error()
    # a null Xg is refused when there are nonzeros
    st = lib.spmv_forward_gather_f32_i64(fake, fake, fake, fake, fake, None, 4, 4, 1, 8, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    st = lib.spmv_backward_gathered_f32_i32(fake, fake, fake, fake, None, fake, fake, fake, 4, 4,
                                            1, 8, fake, 1 << 20, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    # shape checks come first, as in the plain entry points
    st = lib.spmv_forward_gather_f32_i32(fake, fake, fake, fake, fake, fake, -1, 4, 1, 0, None)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"M >= 0" in lib.spmv_last_error()
    # same workspace contract as spmv_backward_f32_*
    need = lib.spmv_backward_workspace_bytes(4, 4, 1, 8)
    st = lib.spmv_backward_gathered_f32_i32(fake, fake, fake, fake, fake, fake, fake, fake, 4, 4,
                                            1, 8, fake, need - 1, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"]
    # nothing to do: no rows
    assert lib.spmv_forward_gather_f32_i32(fake, fake, fake, fake, fake, fake, 0, 4, 1, 0,
                                           None) == 0


def test_cosine_sim_argument_validation_without_gpu():
    lib = _load("cases.cosine_sim.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    st = lib.cosine_sim_forward_f32(fake, fake, fake, fake, fake, -1, 4, 64, 1e-8, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.cosine_sim_forward_f32(fake, fake, fake, fake, fake, 4, 4, 64, -1.0, None)
    assert st == STATUS["NL2K_ERR_VALUE"] and b"eps" in lib.cosine_sim_last_error()
    st = lib.cosine_sim_forward_f32(None, fake, fake, fake, fake, 4, 4, 64, 1e-8, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    # D = 64 fast path: partial (dS . bh) [nRJ][N][64] + (dS^T . ah) [nRI][M][64], no sums;
    # 4096^2 -> 16 x 16 regions of 256
    assert lib.cosine_sim_backward_workspace_bytes(4096, 4096, 64) == 2 * 16 * 4096 * 64 * 4
    assert lib.cosine_sim_backward_workspace_bytes(10, 20, 100) == (10 + 20) * 100 * 4  # generic
    assert lib.cosine_sim_backward_workspace_bytes(0, 20, 64) == 0
    need = lib.cosine_sim_backward_workspace_bytes(64, 64, 64)
    st = lib.cosine_sim_backward_f32(fake, fake, fake, fake, fake, fake, fake, 64, 64, 64, fake,
                                     need - 4, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"]


def test_layernorm_argument_validation_without_gpu():
    lib = _load("cases.layernorm.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    st = lib.layernorm_forward_f32(fake, fake, fake, fake, fake, fake, -1, 64, 1e-5, None)
    assert st == STATUS["NL2K_ERR_SHAPE"] and b"B >= 0" in lib.layernorm_last_error()
    st = lib.layernorm_forward_f32(fake, fake, fake, fake, fake, fake, 4, 0, 1e-5, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.layernorm_forward_f32(fake, fake, fake, fake, fake, fake, 1 << 31, 64, 1e-5, None)
    assert st == STATUS["NL2K_ERR_OVERFLOW"]
    st = lib.layernorm_forward_f32(fake, fake, fake, fake, fake, fake, 4, 64, -1.0, None)
    assert st == STATUS["NL2K_ERR_VALUE"] and b"eps" in lib.layernorm_last_error()
    st = lib.layernorm_forward_f32(fake, fake, fake, fake, fake, fake, 4, 64, float("nan"), None)
    assert st == STATUS["NL2K_ERR_VALUE"]
    st = lib.layernorm_forward_f32(fake, None, fake, fake, fake, fake, 4, 64, 1e-5, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    assert lib.layernorm_forward_f32(None, None, None, None, None, None, 0, 64, 1e-5, None) == 0
    need = lib.layernorm_backward_workspace_bytes(8192, 4096)
    assert need > 0 and lib.layernorm_backward_workspace_bytes(-1, 4096) == 0
    st = lib.layernorm_backward_f32(fake, fake, fake, fake, fake, fake, None, fake, 8192, 4096,
                                    fake, need, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    st = lib.layernorm_backward_f32(fake, fake, fake, fake, fake, fake, fake, fake, 8192, 4096,
                                    fake, need - 4, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"] and b"workspace" in lib.layernorm_last_error()
    odd = ctypes.c_void_p((1 << 20) + 4)
    st = lib.layernorm_backward_f32(fake, fake, fake, fake, fake, fake, fake, fake, 8192, 4096,
                                    odd, need, None)
    assert st == STATUS["NL2K_ERR_ALIGN"]
    st = lib.layernorm_backward_f32(fake, fake, fake, fake, fake, fake, fake, fake, 8, 0,
                                    fake, need, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]


def test_l2norm_scale_argument_validation_without_gpu():
    lib = _load("cases.l2norm_scale.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    st = lib.l2norm_scale_forward_f32(fake, fake, fake, fake, -1, 64, 1e-6, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.l2norm_scale_forward_f32(fake, fake, fake, fake, 4, 64, float("nan"), None)
    assert st == STATUS["NL2K_ERR_VALUE"]
    st = lib.l2norm_scale_forward_f32(fake, None, fake, fake, 4, 64, 1e-6, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    # one partial dg row per backward block (512 blocks at 16384 rows) plus the
    # first column-sum pass's rows; no bias rows
    need = lib.l2norm_scale_backward_workspace_bytes(16384, 1024)
    ln = _load("cases.layernorm.op")
    assert 2 * need == ln.layernorm_backward_workspace_bytes(16384, 1024)
    st = lib.l2norm_scale_backward_f32(fake, fake, fake, fake, fake, fake, 16384, 1024, fake,
                                       need - 4, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"]


def test_softmax_ce_argument_validation_without_gpu():
    lib = _load("cases.softmax_ce.op")
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation
    # one 16-byte slot pair (a partial loss) for each of at most 1024
    # workgroups, then the 8-byte trip-counter word
    assert lib.softmax_ce_forward_workspace_bytes(8192, 1024) == 16 * 1024 + 8
    assert lib.softmax_ce_forward_workspace_bytes(0, 1024) == 16 * 1024 + 8
    assert lib.softmax_ce_forward_workspace_bytes(-1, 1024) == 0
    assert lib.softmax_ce_status_offset() == 16 * 1024
    need = 16 * 1024 + 8
    st = lib.softmax_ce_forward_f32(fake, fake, fake, fake, -1, 1024, fake, need, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.softmax_ce_forward_f32(fake, fake, fake, fake, 8, 0, fake, need, None)
    assert st == STATUS["NL2K_ERR_SHAPE"]
    st = lib.softmax_ce_forward_f32(fake, None, fake, fake, 8, 16, fake, need, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    st = lib.softmax_ce_forward_f32(fake, fake, fake, fake, 8192, 1024, fake, need - 4, None)
    assert st == STATUS["NL2K_ERR_WORKSPACE"] and b"workspace" in lib.softmax_ce_last_error()
    odd = ctypes.c_void_p((1 << 20) + 4)  # 4-byte aligned; the slots need 8
    st = lib.softmax_ce_forward_f32(fake, fake, fake, fake, 8192, 1024, odd, need, None)
    assert st == STATUS["NL2K_ERR_ALIGN"]
    st = lib.softmax_ce_backward_f32(fake, fake, fake, None, fake, 8, 16, None)
    assert st == STATUS["NL2K_ERR_NULL"]
    st = lib.softmax_ce_backward_f32(fake, fake, fake, fake, fake, 1 << 31, 16, None)
    assert st == STATUS["NL2K_ERR_OVERFLOW"]
    assert lib.softmax_ce_backward_f32(None, None, None, None, None, 0, 16, None) == 0


DELIVERY = os.path.join(REPO, "nl2cuda-kernel-agent_amd", "cases", "rbf", "delivery")


def test_delivery_archive_exports_every_declared_symbol():
    """librbf.a (built by __graft_entry__.build) defines every function of
    include/rbf_delivery.h and of include/rbf.h."""
    import subprocess
    archive = os.path.join(DELIVERY, "librbf.a")
    if not os.path.exists(archive):
        pytest.skip("delivery not built")
    out = subprocess.run(["nm", "--defined-only", archive], capture_output=True, text=True,
                         check=True).stdout
    defined = set(re.findall(r" T (\w+)", out))
    for header in ("rbf_delivery.h", "rbf.h"):
        missing = [n for n in declared_functions(header) if n not in defined]
        assert not missing, f"{header}: not in librbf.a: {missing}"
