"""CSR SpMV / SpMM parity on the GPU (libspmv_hip.so) against the float64
oracle at atol = rtol = 1e-3: the acceptance workload (2^20 x 2^20 power-law,
int32 and int64 indices, D = 1, forward and backward), the reference's
default case through verify_all, structures with empty rows, runs of empty
rows longer than the staged window, long rows, K = 1, nnz = 0, feature
widths across every SpMM lane class, misaligned value arrays, determinism
(also under a different split of the rows between waves) and the adjoint
identities."""

import numpy as np
import pytest
import torch

from conftest import announce
from framework.verify import verify_all
from oracle import spmv as osp

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _read_trip_counter(monkeypatch):
    """Every backward through op.py on a column-major (D > 1) route zeroes
    the workspace's trip counter first and reads it after, raising if a
    column-total wait hit its spin cap."""
    monkeypatch.setenv("NL2K_CHECK", "1")


def _close(name, got, ref, atol=1e-3, rtol=1e-3):
    got = got.detach().cpu().double().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    print(f"  {name}: max_abs={max_abs:.3e}")
    assert np.all(err <= atol + rtol * np.abs(ref)), f"{name}: max_abs {max_abs:.3e}"


def _csr(lens, k, d, seed, index_dtype=torch.int64):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    ptr = np.zeros(lens.size + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    col = rng.integers(0, k, int(ptr[-1]))
    g = torch.Generator().manual_seed(seed)
    vals = torch.randn(int(ptr[-1]), generator=g)
    X = torch.randn(k, d, generator=g)
    return (torch.from_numpy(ptr).to(index_dtype), torch.from_numpy(col).to(index_dtype), vals, X)


def _check(ptr, col, vals, X, seed=0, check_bwd=True):
    from cases.spmv import op
    M = ptr.numel() - 1
    dY = torch.randn(M, X.shape[1], generator=torch.Generator().manual_seed(seed + 10_000))
    y = op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda())
    torch.cuda.synchronize()
    _close("y", y, osp.forward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy()))
    if check_bwd:
        dv, dX = op.spmv_backward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda(), dY.cuda())
        torch.cuda.synchronize()
        rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
        _close("dvals", dv, rdv)
        _close("dX", dX, rdX)
        if X.shape[1] == 1 and vals.numel() > 0:
            _check_gathered(ptr, col, vals, X, dY, y, dv, rdX)
    return y


def _check_gathered(ptr, col, vals, X, dY, y, dv, rdX):
    """D == 1: the forward that keeps X[col] gives the same y bit for bit
    and an exact copy of the gathered x; the backward reading that copy gives
    the same dvals bit for bit (dX is summed in a varying order, so it is
    checked against the oracle)."""
    from cases.spmv import op
    args = [ptr.cuda(), col.cuda(), vals.cuda(), X.cuda()]
    y2, xg = op.spmv_forward(*args, keep_gather=True)
    dv2, dX2 = op.spmv_backward(*args, dY.cuda(), X_gathered=xg)
    dv3, _ = op.spmv_backward(*args, dY.cuda(), need_X=False, X_gathered=xg)
    torch.cuda.synchronize()
    assert torch.equal(y2, y), "gathered forward changed y"
    assert torch.equal(xg.cpu(), X[:, 0][col.long()]), "Xg is not X[col]"
    assert torch.equal(dv2, dv) and torch.equal(dv3, dv), "gathered dvals differ"
    _close("dX (gathered walk)", dX2, rdX)


@pytest.fixture(scope="module")
def zipf_inputs():
    from cases.spmv import reference as ref
    return ref.make_zipf_inputs(1 << 20, 1 << 20, 1, 0, torch.int32)


@pytest.mark.parametrize("seed", [1, 2])
def test_spmv_zipf_other_seeds(seed):
    """The acceptance recipe at further seeds: other row lengths, columns,
    values, x and dy (seed 0 runs below, with determinism checks)."""
    announce(f"spmv zipf 2^20 int32 D=1 fwd+bwd seed={seed}")
    from cases.spmv import reference as ref
    t = ref.make_zipf_inputs(1 << 20, 1 << 20, 1, seed, torch.int32)
    _check(t["row_ptr"], t["col_idx"], t["vals"], t["X"], seed=seed)


def test_spmv_zipf_baseline_int32(zipf_inputs):
    announce("spmv zipf 2^20 int32 D=1 fwd+bwd")
    t = zipf_inputs
    y = _check(t["row_ptr"], t["col_idx"], t["vals"], t["X"])
    from cases.spmv import op
    y2 = op.spmv_forward(t["row_ptr"].cuda(), t["col_idx"].cuda(), t["vals"].cuda(), t["X"].cuda())
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "forward is not deterministic"


def test_spmv_zipf_int64_matches_int32(zipf_inputs):
    announce("spmv zipf 2^20 int64 == int32")
    from cases.spmv import op
    t = zipf_inputs
    args32 = [t["row_ptr"].cuda(), t["col_idx"].cuda(), t["vals"].cuda(), t["X"].cuda()]
    args64 = [t["row_ptr"].long().cuda(), t["col_idx"].long().cuda()] + args32[2:]
    y32 = op.spmv_forward(*args32)
    y64 = op.spmv_forward(*args64)
    dY = torch.randn(y32.shape, generator=torch.Generator().manual_seed(3)).cuda()
    dv32, _ = op.spmv_backward(*args32, dY, need_X=False)
    dv64, dX64 = op.spmv_backward(*args64, dY)
    torch.cuda.synchronize()
    assert torch.equal(y32, y64)
    assert torch.equal(dv32, dv64)
    # adjoint identities at full size: <A x, dy> = <x, A^T dy> = sum vals * dvals
    lhs = float((y64.double() * dY.double()).sum())
    assert np.isclose(lhs, float((args32[3].double() * dX64.double()).sum()), rtol=1e-4)
    assert np.isclose(lhs, float((args32[2].double() * dv64.double()).sum()), rtol=1e-4)


@pytest.mark.parametrize("pad", [(777, 0), (0, 1234), (5, 300_001)])
def test_spmv_d1_forward_independent_of_wave_split(zipf_inputs, pad):
    """Empty rows before and after the matrix move every boundary of the
    merge-path split between waves (and the wave count) but no nonzero: the
    real rows must come out bit-identical and the padding rows 0."""
    announce(f"spmv zipf 2^20 forward with {pad} empty rows around it")
    from cases.spmv import op
    t = zipf_inputs
    ptr, col, vals, X = (t[k].cuda() for k in ("row_ptr", "col_idx", "vals", "X"))
    before, after = pad
    nnz = int(ptr[-1])
    ptr_p = torch.cat([torch.zeros(before, dtype=ptr.dtype, device=ptr.device), ptr,
                       torch.full((after,), nnz, dtype=ptr.dtype, device=ptr.device)])
    y = op.spmv_forward(ptr, col, vals, X)
    y_p = op.spmv_forward(ptr_p, col, vals, X)
    torch.cuda.synchronize()
    M = ptr.numel() - 1
    assert torch.equal(y_p[before:before + M], y)
    assert not torch.any(y_p[:before]) and not torch.any(y_p[before + M:])


@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
def test_spmm_reference_default_backward_deterministic(idx):
    """The reference's default SpMM (M = K = 4096, D = 64, 64 nonzeros per
    row, sorted unique columns): dX = A^T dY is summed in a fixed order, so
    two backward calls give identical dX and dvals bit for bit, and both
    match the float64 oracle."""
    announce(f"spmm reference default backward determinism {idx}")
    from cases.spmv import op, reference as ref
    t = ref.make_inputs(0, torch.float32, "cpu")
    ptr, col, vals, X = (t[k] for k in ("row_ptr", "col_idx", "vals", "X"))
    ptr, col = ptr.to(idx), col.to(idx)
    M = ptr.numel() - 1
    dY = torch.randn(M, X.shape[1], generator=torch.Generator().manual_seed(10_000))
    args = [ptr.cuda(), col.cuda(), vals.cuda(), X.cuda()]
    dv1, dX1 = op.spmv_backward(*args, dY.cuda())
    dv2, dX2 = op.spmv_backward(*args, dY.cuda())
    _, dX3 = op.spmv_backward(*args, dY.cuda(), need_vals=False)
    torch.cuda.synchronize()
    assert torch.equal(dX1, dX2) and torch.equal(dX1, dX3), "dX is not bitwise repeatable"
    assert torch.equal(dv1, dv2), "dvals is not bitwise repeatable"
    rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
    _close("dvals", dv1, rdv)
    _close("dX", dX1, rdX)


def test_spmv_verify_all_reference_defaults():
    announce("spmv verify_all (reference defaults M=K=4096 D=64 int64)")
    from cases.spmv import CASE, op
    ok, report = verify_all(CASE, op.candidate, device="cuda")
    print(report)
    assert ok, report


def _lens(kind, m, k, rng):
    if kind == "small":
        return rng.integers(0, 10, m)
    if kind == "mostly_empty":
        return np.where(rng.random(m) < 0.9, 0, rng.integers(0, min(k, 2000) + 1, m))
    if kind == "ones":
        return np.ones(m, np.int64)
    if kind == "one_long":
        lens = np.zeros(m, np.int64)
        lens[m // 3] = k
        return lens
    if kind == "ends_only":  # runs of empty rows far longer than the staged window
        lens = np.zeros(m, np.int64)
        lens[1] = 5
        lens[m - 2] = 300
        return lens
    if kind == "zipf":
        return np.minimum(rng.zipf(1.5, m), k)
    if kind == "sparse_rows":  # rows of 0-1 nonzeros: sort tiles span more rows than their LDS copy
        return (rng.random(m) < 0.15).astype(np.int64)
    if kind == "ragged_long":  # SpMM rows split between lane groups: long, empty and 1-entry rows
        lens = rng.integers(0, 300, m)
        lens[::7] = 0
        lens[1::11] = 1
        return lens
    if kind == "long":
        return rng.integers(100, 400, m)
    if kind == "mid":
        return rng.integers(0, 48, m)
    if kind == "tile_edges":  # rows starting on 8192-position sort-tile edges, empty ones too
        lens = np.full(m, 8, np.int64)
        lens[1024] = 0  # rows 1024 and 1025 both start at position 8192
        lens[3000] = 13  # later edges fall inside rows
        lens[5000:5003] = 0
        return lens
    raise ValueError(kind)


@pytest.mark.parametrize("kind,m,k,d", [
    ("small", 1000, 500, 1), ("mostly_empty", 3000, 3000, 1), ("ones", 257, 100, 1),
    ("one_long", 2000, 60000, 1), ("ends_only", 5000, 400, 1), ("zipf", 20000, 5000, 1),
    ("small", 4000, 1, 1), ("small", 1, 10, 1), ("small", 500, 300, 3), ("small", 500, 300, 4),
    ("zipf", 300, 200, 17), ("zipf", 300, 200, 64), ("small", 100, 100, 100),
    ("small", 100, 50, 256), ("one_long", 64, 64, 300), ("ends_only", 700, 90, 8),
    ("small", 300, 20000, 4), ("small", 300, 16384, 8), ("mostly_empty", 2000, 1500, 32), ("one_long", 50, 3000, 16),
    ("sparse_rows", 200000, 5000, 1), ("tile_edges", 6000, 3000, 1),
    ("ragged_long", 333, 500, 3), ("ragged_long", 333, 500, 8), ("ragged_long", 333, 500, 20),
    ("ragged_long", 333, 500, 64), ("ragged_long", 129, 700, 100), ("long", 77, 900, 8),
    ("long", 77, 900, 5), ("mid", 1001, 300, 12), ("mid", 1001, 300, 64)])
def test_spmv_structures(kind, m, k, d):
    announce(f"spmv {kind} M={m} K={k} D={d}")
    rng = np.random.default_rng(m + k + d)
    lens = _lens(kind, m, k, rng)
    for idx in (torch.int64, torch.int32):
        _check(*_csr(lens, k, d, m + d, idx))


@pytest.mark.parametrize("d", [1, 64])
def test_spmv_nan_propagates(d):
    """A NaN in one row of X reaches exactly the rows of Y that use that
    column and the dvals of those positions; a NaN in one row of dY reaches
    exactly the dX rows of that row's columns (through the D = 1 sort and sum,
    or the SpMM column gather) and its dvals.  Everything else matches the
    oracle."""
    announce(f"spmv NaN propagation D={d}")
    from cases.spmv import op
    rng = np.random.default_rng(41)
    m, k = 3000, 2500
    lens = np.minimum(rng.zipf(1.5, m), 300)
    ptr, col, vals, X = _csr(lens, k, d, 41, torch.int32)
    rows = np.repeat(np.arange(m), lens)
    c0 = int(col[len(col) // 2])
    r0 = int(rows[len(col) // 3])
    X[c0, 0] = float("nan")
    dY = torch.randn(m, d, generator=torch.Generator().manual_seed(42))
    dY[r0, 0] = float("nan")
    y = op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda())
    dv, dX = op.spmv_backward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda(), dY.cuda())
    torch.cuda.synchronize()
    coln = col.numpy()
    hit_rows = np.unique(rows[coln == c0])
    hit_cols = np.unique(coln[rows == r0])
    ynan = torch.isnan(y.cpu()).any(dim=1).numpy()
    assert np.array_equal(np.nonzero(ynan)[0], hit_rows)
    xnan = torch.isnan(dX.cpu()).any(dim=1).numpy()
    assert np.array_equal(np.nonzero(xnan)[0], hit_cols)
    vnan = torch.isnan(dv.cpu()).numpy()
    assert np.array_equal(vnan, (coln == c0) | (rows == r0))
    Xc = X.clone()
    Xc[c0, 0] = 0.0
    dYc = dY.clone()
    dYc[r0, 0] = 0.0
    ry = osp.forward_f64(ptr.numpy(), coln, vals.numpy(), Xc.numpy())
    rdv, rdX = osp.backward_f64(ptr.numpy(), coln, vals.numpy(), Xc.numpy(), dYc.numpy())
    keep_r, keep_c = ~ynan, ~xnan
    _close("y (other rows)", y.cpu()[keep_r], ry[keep_r])
    _close("dX (other rows)", dX.cpu()[keep_c], rdX[keep_c])
    _close("dvals (other positions)", dv.cpu()[~vnan], rdv[~vnan])


def test_spmv_d1_beyond_the_bucket_sort():
    """More columns than the bucket sort covers (1024 buckets of 16384
    columns, 2^24): dX at D == 1 takes the zero-fill plus fp32 atomics route
    from the walk, with and without the kept copy of X[col]."""
    k = (1 << 24) + 4099
    announce(f"spmv D=1 K={k} (atomic dX route)")
    lens = np.random.default_rng(21).integers(0, 40, 800)
    for idx in (torch.int32, torch.int64):
        _check(*_csr(lens, k, 1, 21, idx))


def test_spmv_no_nonzeros():
    announce("spmv nnz = 0")
    from cases.spmv import op
    ptr = torch.zeros(101, dtype=torch.int64)
    col = torch.zeros(0, dtype=torch.int64)
    vals = torch.zeros(0)
    X = torch.randn(7, 1)
    y = op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda())
    dv, dX = op.spmv_backward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda(), torch.ones(100, 1).cuda())
    torch.cuda.synchronize()
    assert torch.all(y == 0) and y.shape == (100, 1)
    assert dv.numel() == 0 and torch.all(dX == 0)


def test_spmv_misaligned_values():
    announce("spmv misaligned vals / X (scalar paths)")
    from cases.spmv import op
    ptr, col, vals, X = _csr(np.random.default_rng(1).integers(0, 20, 900), 700, 1, 9)
    buf = torch.empty(vals.numel() + 1, device="cuda")
    buf[1:].copy_(vals.cuda())
    y = op.spmv_forward(ptr.cuda(), col.cuda(), buf[1:], X.cuda())
    torch.cuda.synchronize()
    _close("y (misaligned vals)", y, osp.forward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy()))
    ptr, col, vals, X = _csr(np.random.default_rng(2).integers(0, 20, 300), 200, 64, 10)
    xb = torch.empty(X.numel() + 1, device="cuda")
    xb[1:].copy_(X.reshape(-1).cuda())
    y = op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), xb[1:].view(200, 64))
    torch.cuda.synchronize()
    _close("y (misaligned X)", y, osp.forward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy()))


def _backward_twice(ptr, col, vals, X, dY, X_dev=None, dY_dev=None):
    """Two backward calls; asserts they agree bit for bit and returns one."""
    from cases.spmv import op
    args = [ptr.cuda(), col.cuda(), vals.cuda(), X.cuda() if X_dev is None else X_dev]
    g = dY.cuda() if dY_dev is None else dY_dev
    dv1, dX1 = op.spmv_backward(*args, g)
    dv2, dX2 = op.spmv_backward(*args, g)
    torch.cuda.synchronize()
    assert torch.equal(dX1, dX2), "dX is not bitwise repeatable"
    assert torch.equal(dv1, dv2), "dvals is not bitwise repeatable"
    return dv1, dX1


@pytest.mark.parametrize("k,d", [(20, 64), (20, 8), (40, 16)])
def test_spmm_column_block_rounds(k, d):
    """Few columns, many nonzeros: one column block holds tens of thousands
    of entries, which the column-block gather takes in several rounds of at
    most 2048 (K = 20 at D = 8: one block of 64 columns holds every entry).
    dX matches the oracle and repeats bit for bit."""
    announce(f"spmm column-block rounds K={k} D={d}")
    for idx in (torch.int64, torch.int32):
        ptr, col, vals, X = _csr(np.full(4000, 10), k, d, 77, idx)
        dY = torch.randn(4000, d, generator=torch.Generator().manual_seed(78))
        dv, dX = _backward_twice(ptr, col, vals, X, dY)
        rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
        _close("dvals", dv, rdv)
        _close("dX", dX, rdX)


@pytest.mark.parametrize("d", [64, 16])
def test_spmm_column_block_many_chunks(d):
    """More 1024-position sort chunks (563) than one gather round reads
    (512 per window): the window moves on, and rows with zero to 128
    entries cross chunk edges."""
    announce(f"spmm column-block chunk windows D={d}")
    lens = np.random.default_rng(90).integers(0, 129, 9000)
    ptr, col, vals, X = _csr(lens, 4096, d, 91, torch.int32)
    assert vals.numel() > 512 * 1024
    dY = torch.randn(9000, d, generator=torch.Generator().manual_seed(92))
    dv, dX = _backward_twice(ptr, col, vals, X, dY)
    rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
    _close("dvals", dv, rdv)
    _close("dX", dX, rdX)


def test_spmm_backward_routes_agree():
    """The reference default shape through both D > 1 routes: 16-byte
    aligned X and dY take the column-block kernels, an X that starts one
    float past an aligned address takes the column-major copy.  Each is
    bitwise repeatable and matches the oracle, and they agree with each
    other to rounding."""
    announce("spmm backward: column-block route vs column-major copy")
    from cases.spmv import reference as ref
    t = ref.make_inputs(3, torch.float32, "cpu")
    ptr, col, vals, X = (t[k] for k in ("row_ptr", "col_idx", "vals", "X"))
    K, D = X.shape
    dY = torch.randn(ptr.numel() - 1, D, generator=torch.Generator().manual_seed(93))
    dv_a, dX_a = _backward_twice(ptr, col, vals, X, dY)
    xb = torch.empty(X.numel() + 1, device="cuda")
    xb[1:].copy_(X.reshape(-1).cuda())
    dv_b, dX_b = _backward_twice(ptr, col, vals, X, dY, X_dev=xb[1:].view(K, D))
    rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
    for name, dv, dX in (("blocks", dv_a, dX_a), ("column-major", dv_b, dX_b)):
        _close(f"dvals ({name})", dv, rdv)
        _close(f"dX ({name})", dX, rdX)
    assert torch.allclose(dX_a, dX_b, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("opt_in", ["default", "params", "env"])
def test_spmv_autograd_saved_tensors_and_gathered_opt_in(opt_in, monkeypatch):
    """The reference's save list (cases/spmv/op.py:28-33) by default: exactly
    (row_ptr, col_idx, vals, X).  With the opt-in (params["keep_gather"] or
    NL2K_SPMV_KEEP_GATHER=1) at D == 1 with vals requiring grad the forward
    also keeps X[col] and the backward streams it.  Either way both
    gradients match the oracle and dvals equals the plain C-ABI backward's
    bit for bit."""
    announce(f"spmv autograd D=1 save list ({opt_in})")
    from cases.spmv import op
    params = {"keep_gather": True} if opt_in == "params" else {}
    if opt_in == "env":
        monkeypatch.setenv("NL2K_SPMV_KEEP_GATHER", "1")
    ptr, col, vals, X = _csr(np.minimum(np.random.default_rng(6).zipf(1.5, 5000), 3000), 3000, 1, 12)
    vd = vals.cuda().requires_grad_(True)
    Xd = X.cuda().requires_grad_(True)
    y = op.candidate({"row_ptr": ptr.cuda(), "col_idx": col.cuda(), "vals": vd, "X": Xd}, params)
    saved = y.grad_fn.saved_tensors
    if opt_in == "default":
        assert len(saved) == 4  # row_ptr, col_idx, vals, X
    else:
        assert len(saved) == 5  # row_ptr, col_idx, vals, X, Xg
        assert torch.equal(saved[4].cpu(), X[:, 0][col.long()])
    dY = torch.randn(y.shape, generator=torch.Generator().manual_seed(7))
    y.backward(dY.cuda())
    dv, _ = op.spmv_backward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda(), dY.cuda(), need_X=False)
    torch.cuda.synchronize()
    rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
    _close("dvals", vd.grad, rdv)
    _close("dX", Xd.grad, rdX)
    assert torch.equal(vd.grad, dv)


def test_spmv_opt_in_keeps_four_tensors_where_it_does_not_apply():
    """The opt-in saves the reference's four tensors when vals needs no
    gradient or D > 1."""
    announce("spmv autograd opt-in outside D=1 with vals grad")
    from cases.spmv import op
    ptr, col, vals, X = _csr(np.random.default_rng(2).integers(0, 20, 300), 200, 1, 3)
    Xd = X.cuda().requires_grad_(True)
    y = op.candidate({"row_ptr": ptr.cuda(), "col_idx": col.cuda(), "vals": vals.cuda(), "X": Xd},
                     {"keep_gather": True})
    assert len(y.grad_fn.saved_tensors) == 4
    ptr, col, vals, X = _csr(np.random.default_rng(2).integers(0, 20, 300), 200, 8, 3)
    y = op.candidate({"row_ptr": ptr.cuda(), "col_idx": col.cuda(),
                      "vals": vals.cuda().requires_grad_(True), "X": X.cuda()},
                     {"keep_gather": True})
    assert len(y.grad_fn.saved_tensors) == 4


@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_spmv_malformed_structure_raises_under_check(idx, monkeypatch):
    """NL2K_CHECK=1 (set for every test here): the device-side structure
    check raises before any product kernel runs: IndexError for a column
    outside [0, K), as the reference path's X.index_select(0, col_idx) does
    (cases/spmv/reference.py:19), RuntimeError for a bad row_ptr.  Without
    NL2K_CHECK the kernels clamp the index into range (no error, no fault)."""
    announce(f"spmv structure check ({idx})")
    from cases.spmv import op
    ptr, col, vals, X = _csr([3, 0, 2, 4], 10, 1, 5, index_dtype=idx)
    dY = torch.ones(4, 1, device="cuda")
    for bad, what in ((10, "= 10 is not in"), (-1, "= -1 is not in")):
        c = col.clone()
        c[5] = bad
        with pytest.raises(IndexError, match=f"col_idx\\[5\\] {what}"):
            op.spmv_forward(ptr.cuda(), c.cuda(), vals.cuda(), X.cuda())
        with pytest.raises(IndexError, match="index out of range"):
            op.spmv_backward(ptr.cuda(), c.cuda(), vals.cuda(), X.cuda(), dY)
        Xd = X.cuda().requires_grad_(True)
        with pytest.raises(IndexError):
            op.candidate({"row_ptr": ptr.cuda(), "col_idx": c.cuda(), "vals": vals.cuda(),
                          "X": Xd}, {})
    for r, v, what in ((0, 1, "row_ptr\\[0\\] != 0"), (2, 1, "decreases"),
                       (4, 8, "row_ptr\\[M\\] != nnz")):
        p = ptr.clone()
        p[r] = v
        with pytest.raises(RuntimeError, match=what):
            op.spmv_forward(p.cuda(), col.cuda(), vals.cuda(), X.cuda())
    op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda())  # well formed: no error
    monkeypatch.delenv("NL2K_CHECK")
    c = col.clone()
    c[5] = 10
    y = op.spmv_forward(ptr.cuda(), c.cuda(), vals.cuda(), X.cuda())
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()


def test_spmv_gathered_misaligned():
    """Scalar (unaligned) forms of the gathered forward and walk."""
    announce("spmv gathered copy of X, misaligned vals / Xg")
    from cases.spmv import op
    ptr, col, vals, X = _csr(np.random.default_rng(3).integers(0, 40, 1200), 900, 1, 13)
    buf = torch.empty(vals.numel() + 1, device="cuda")
    buf[1:].copy_(vals.cuda())
    args = [ptr.cuda(), col.cuda(), buf[1:], X.cuda()]
    y, xg = op.spmv_forward(*args, keep_gather=True)
    xb = torch.empty(vals.numel() + 1, device="cuda")
    xb[1:].copy_(xg)
    dY = torch.randn(y.shape, generator=torch.Generator().manual_seed(8))
    dv, dX = op.spmv_backward(*args, dY.cuda(), X_gathered=xb[1:])
    torch.cuda.synchronize()
    assert torch.equal(xg.cpu(), X[:, 0][col.long()])
    rdv, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
    _close("y", y, osp.forward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy()))
    _close("dvals", dv, rdv)
    _close("dX", dX, rdX)


def test_spmv_autograd_partial_grads():
    announce("spmv autograd, X only")
    from cases.spmv import op
    ptr, col, vals, X = _csr(np.random.default_rng(4).integers(1, 30, 400), 300, 16, 11)
    Xd = X.cuda().requires_grad_(True)
    y = op.candidate({"row_ptr": ptr.cuda(), "col_idx": col.cuda(), "vals": vals.cuda(), "X": Xd}, {})
    dY = torch.randn(y.shape, generator=torch.Generator().manual_seed(5))
    y.backward(dY.cuda())
    torch.cuda.synchronize()
    _, rdX = osp.backward_f64(ptr.numpy(), col.numpy(), vals.numpy(), X.numpy(), dY.numpy())
    _close("dX", Xd.grad, rdX)


def test_spmv_rejects_bad_arguments():
    announce("spmv argument checks")
    from cases.spmv import op
    ptr, col, vals, X = _csr([1, 2], 4, 1, 0)
    with pytest.raises(RuntimeError, match="share a dtype"):
        op.spmv_forward(ptr.cuda(), col.int().cuda(), vals.cuda(), X.cuda())
    with pytest.raises(RuntimeError, match="same length"):
        op.spmv_forward(ptr.cuda(), col.cuda(), vals[:1].cuda(), X.cuda())
    with pytest.raises(RuntimeError, match="rank-2"):
        op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), X.reshape(-1).cuda())
    with pytest.raises(RuntimeError, match="D == 1"):
        op.spmv_forward(ptr.cuda(), col.cuda(), vals.cuda(), X.repeat(1, 2).cuda(), keep_gather=True)
    with pytest.raises(RuntimeError, match="X_gathered must be"):
        op.spmv_backward(ptr.cuda(), col.cuda(), vals.cuda(), X.cuda(), torch.ones(2, 1).cuda(),
                         X_gathered=vals[:1].cuda())
