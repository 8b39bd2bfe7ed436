"""RBF parity on the GPU: the HIP library (through its C-ABI and through the
autograd op) against the float64 oracle, at atol = rtol = 1e-3.

Workloads follow the acceptance configs (X, Y ~ N(0,1)/8, gamma = 0.5,
dK ~ N(0,1)): N = M = 2048, 4096 and 8192 for seeds 0-4 (the reference
protocol's seeds), with size-independent identities at 8192; then ragged and edge shapes, the
generic (D != 64, misaligned) path, empty inputs, gamma = 0, NaN inputs, the committed
fixtures written by the reference's own CPU loops, and the framework's
verify_all against the case's reference.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from conftest import announce
from framework import capi
from framework.verify import verify_all
from oracle import rbf as orbf

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rbf_ref_small.npz")


def _op():
    from cases.rbf import op
    return op


def _inputs(n, m, d, seed, scale=0.125):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n, d, generator=g) * scale
    Y = torch.randn(m, d, generator=g) * scale
    G = torch.randn(n, m, generator=torch.Generator().manual_seed(seed + 10_000))
    return X, Y, G


def _close(name, got, ref, atol=ATOL, rtol=RTOL):
    got = got.detach().cpu().double().numpy() if torch.is_tensor(got) else np.asarray(got)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    max_abs = float(err.max()) if err.size else 0.0
    print(f"  {name}: max_abs={max_abs:.3e} max_rel={float((err / np.maximum(np.abs(ref), 1e-30)).max()) if err.size else 0:.3e}")
    assert not bad.any(), f"{name}: {int(bad.sum())} entries outside tolerance (max_abs {max_abs:.3e})"


def _run_autograd(X, Y, G, gamma):
    op = _op()
    Xd = X.cuda().requires_grad_(True)
    Yd = Y.cuda().requires_grad_(True)
    K = op.candidate({"X": Xd, "Y": Yd}, {"gamma": gamma})
    K.backward(G.cuda())
    torch.cuda.synchronize()
    return K.detach(), Xd.grad, Yd.grad


def _check_full(X, Y, G, gamma):
    K, dX, dY = _run_autograd(X, Y, G, gamma)
    Xn, Yn, Gn = X.numpy(), Y.numpy(), G.numpy()
    Kr = orbf.forward_f64(Xn, Yn, gamma)
    _close("K", K, Kr)
    dXr, dYr = orbf.backward_f64(Xn, Yn, Gn, Kr, gamma)
    _close("dX", dX, dXr)
    _close("dY", dY, dYr)
    return K, dX, dY


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_rbf_2048_parity(seed):
    announce(f"rbf 2048 seed={seed}")
    _check_full(*_inputs(2048, 2048, 64, seed), 0.5)


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_rbf_4096_parity(seed):
    announce(f"rbf 4096 seed={seed}")
    _check_full(*_inputs(4096, 4096, 64, seed), 0.5)


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_rbf_8192_parity_and_identities(seed):
    announce(f"rbf 8192 seed={seed}")
    X, Y, G = _inputs(8192, 8192, 64, seed)
    K, dX, dY = _check_full(X, Y, G, 0.5)
    # translation identity: sum_i dX_i + sum_j dY_j = 0 (relative to the scale of dX)
    s = (dX.double().sum(0) + dY.double().sum(0)).abs().max().item()
    assert s <= 1e-3 * dX.double().abs().sum().item() / dX.shape[0]
    assert float(K.max()) <= 1.0 and float(K.min()) >= 0.0


@pytest.mark.parametrize("n,m", [(1, 1), (3, 5), (65, 130), (127, 129), (300, 17),
                                 (128, 4100), (1000, 999), (513, 2049),
                                 # multiples of 64: the full-tile (buffer-load) backward
                                 # at every region width, square and not
                                 (64, 192), (256, 640), (1088, 960), (3072, 1024),
                                 # 192-wide regions (ragged, full tiles, scalar loads, two
                                 # rounds); forward units spread unevenly, 128 or 256 rows
                                 (3000, 3000), (3008, 2944), (2999, 3001), (5000, 5000)])
def test_rbf_ragged_shapes(n, m):
    announce(f"rbf ragged n={n} m={m}")
    _check_full(*_inputs(n, m, 64, n + m), 0.5)


@pytest.mark.parametrize("d", [1, 3, 32, 100])
def test_rbf_generic_feature_dims(d):
    announce(f"rbf generic D={d}")
    _check_full(*_inputs(70, 45, d, d, scale=1.0 / np.sqrt(d)), 0.5)


# the tiled generic kernels: ragged tile edges on both sides, feature chunks
# of 16 (forward) and passes of 64 (backward) with ragged ends
@pytest.mark.parametrize("n,m,d", [(130, 200, 16), (257, 65, 128), (1000, 1000, 32),
                                   (64, 64, 65), (300, 129, 200)])
def test_rbf_generic_tiled_shapes(n, m, d):
    announce(f"rbf generic n={n} m={m} D={d}")
    _check_full(*_inputs(n, m, d, n + m + d, scale=1.0 / np.sqrt(d)), 0.5)


def test_rbf_reference_default_distribution():
    announce("rbf gamma=1/64 unscaled inputs (reference defaults)")
    _check_full(*_inputs(512, 384, 64, 11, scale=1.0), 1.0 / 64.0)


def test_rbf_gamma_zero_and_self_kernel():
    announce("rbf gamma=0 / X==Y")
    X, Y, G = _inputs(200, 150, 64, 3)
    K, dX, dY = _run_autograd(X, Y, G, 0.0)
    assert torch.all(K == 1.0)
    assert torch.all(dX == 0) and torch.all(dY == 0)
    K2, _, _ = _run_autograd(X, X.clone(), torch.zeros(200, 200), 0.5)
    _close("diag(K(X,X))", torch.diagonal(K2), np.ones(200))


@pytest.mark.parametrize("n,m", [(256, 256), (200, 150)])
def test_rbf_nan_rows_propagate(n, m):
    """A NaN in row i of X (column j of Y) makes K[i, :] (K[:, j]) NaN, as the
    reference's exp(-gamma * sum((x - y)^2)) does: the distance clamp is a
    compare and select, which passes NaN through (v_min / v_med3 would map it
    to 0 and give K = 1).  Every other entry matches the oracle.  256 x 256
    takes the full-tile kernel, 200 x 150 the ragged one."""
    announce(f"rbf NaN rows {n}x{m}")
    X, Y, _ = _inputs(n, m, 64, 11)
    X[3, 5] = float("nan")
    Y[7, 0] = float("nan")
    K = _op().candidate({"X": X.cuda(), "Y": Y.cuda()}, {"gamma": 0.5})
    torch.cuda.synchronize()
    Kc = K.cpu()
    nan_mask = torch.zeros(n, m, dtype=torch.bool)
    nan_mask[3, :] = True
    nan_mask[:, 7] = True
    assert torch.equal(torch.isnan(Kc), nan_mask)
    Kr = orbf.forward_f64(X.numpy(), Y.numpy(), 0.5)
    assert np.array_equal(np.isnan(Kr), nan_mask.numpy())
    keep = ~nan_mask.numpy()
    _close("K (finite part)", Kc.numpy()[keep], Kr[keep])


def test_rbf_empty_inputs():
    announce("rbf empty")
    op = _op()
    X = torch.zeros(0, 64, device="cuda")
    Y = torch.randn(5, 64, device="cuda")
    K = op.rbf_forward(X, Y, 0.5)
    assert K.shape == (0, 5)
    dX, dY = op.rbf_backward(X, Y, torch.zeros(0, 5, device="cuda"), K, 0.5)
    torch.cuda.synchronize()
    assert dX.shape == (0, 64) and torch.all(dY == 0)
    dX, dY = op.rbf_backward(Y, X, torch.zeros(5, 0, device="cuda"),
                             torch.zeros(5, 0, device="cuda"), 0.5)
    torch.cuda.synchronize()
    assert torch.all(dX == 0) and dY.shape == (0, 64)


def test_rbf_misaligned_inputs_use_generic_path():
    announce("rbf misaligned")
    X, Y, G = _inputs(40, 24, 64, 5)
    buf = torch.empty(40 * 64 + 1, device="cuda")
    buf[1:].copy_(X.reshape(-1).cuda())
    Xmis = buf[1:].view(40, 64)  # contiguous but 4 bytes off 16-byte alignment
    K = _op().rbf_forward(Xmis, Y.cuda(), 0.5)
    torch.cuda.synchronize()
    _close("K(misaligned)", K, orbf.forward_f64(X.numpy(), Y.numpy(), 0.5))


def test_rbf_against_reference_loop_fixtures():
    announce("rbf vs committed fixtures of the reference's CPU loops")
    z = np.load(GOLDEN)
    for name in ("tiny", "small", "ragged", "refdefault"):
        X, Y, G = (torch.from_numpy(z[f"{name}_{k}"]) for k in ("X", "Y", "G"))
        gamma = float(z[f"{name}_gamma"])
        K, dX, dY = _run_autograd(X, Y, G, gamma)
        _close(f"{name} K", K, z[f"{name}_K"])
        _close(f"{name} dX", dX, z[f"{name}_dX"])
        _close(f"{name} dY", dY, z[f"{name}_dY"])


def test_rbf_c_abi_direct():
    """Calls rbf_forward_f32 / rbf_backward_f32 with raw device pointers."""
    announce("rbf C-ABI direct, 1024 x 768")
    op = _op()
    lib = op._lib()
    X, Y, G = _inputs(1024, 768, 64, 21)
    Xd, Yd, Gd = X.cuda(), Y.cuda(), G.cuda()
    K = torch.empty(1024, 768, device="cuda")
    dX = torch.empty_like(Xd)
    dY = torch.empty_like(Yd)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = lib.rbf_forward_f32(capi.ptr(Xd), capi.ptr(Yd), capi.ptr(K), 1024, 768, 64, 0.5, stream)
    assert st == 0, lib.rbf_last_error()
    ws_bytes = lib.rbf_backward_workspace_bytes(1024, 768, 64)
    ws = torch.empty(max(ws_bytes // 4, 1), device="cuda")
    st = lib.rbf_backward_f32(capi.ptr(Xd), capi.ptr(Yd), capi.ptr(Gd), capi.ptr(K),
                              capi.ptr(dX), capi.ptr(dY), 1024, 768, 64, 0.5,
                              capi.ptr(ws), ws_bytes, stream)
    assert st == 0, lib.rbf_last_error()
    torch.cuda.synchronize()
    Kr = orbf.forward_f64(X.numpy(), Y.numpy(), 0.5)
    _close("K", K, Kr)
    dXr, dYr = orbf.backward_f64(X.numpy(), Y.numpy(), G.numpy(), Kr, 0.5)
    _close("dX", dX, dXr)
    _close("dY", dY, dYr)
    # a too-small workspace is rejected with a message, nothing launched
    if ws_bytes:
        st = lib.rbf_backward_f32(capi.ptr(Xd), capi.ptr(Yd), capi.ptr(Gd), capi.ptr(K),
                                  capi.ptr(dX), capi.ptr(dY), 1024, 768, 64, 0.5,
                                  capi.ptr(ws), ws_bytes - 4, stream)
        assert st != 0 and b"workspace" in lib.rbf_last_error()


def test_rbf_generic_backward_split_and_whole():
    """D != 64: the generic backward cuts its walks into slices when the
    workspace holds their partial sums, and runs them whole with no
    workspace; both match the oracle."""
    announce("rbf generic backward, sliced and whole, 1500 x 700, D=32")
    lib = _op()._lib()
    n, m, d = 1500, 700, 32
    X, Y, G = _inputs(n, m, d, 5, scale=1.0 / np.sqrt(d))
    Xd, Yd, Gd = X.cuda(), Y.cuda(), G.cuda()
    K = torch.empty(n, m, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.rbf_forward_f32(capi.ptr(Xd), capi.ptr(Yd), capi.ptr(K), n, m, d, 0.5, stream) == 0
    ws_bytes = lib.rbf_backward_workspace_bytes(n, m, d)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes // 4, device="cuda")
    Kr = orbf.forward_f64(X.numpy(), Y.numpy(), 0.5)
    dXr, dYr = orbf.backward_f64(X.numpy(), Y.numpy(), G.numpy(), Kr, 0.5)
    for name, ptr, nbytes in (("sliced", capi.ptr(ws), ws_bytes), ("whole", None, 0)):
        dX = torch.empty_like(Xd)
        dY = torch.empty_like(Yd)
        st = lib.rbf_backward_f32(capi.ptr(Xd), capi.ptr(Yd), capi.ptr(Gd), capi.ptr(K),
                                  capi.ptr(dX), capi.ptr(dY), n, m, d, 0.5, ptr, nbytes, stream)
        assert st == 0, lib.rbf_last_error()
        torch.cuda.synchronize()
        _close(f"dX ({name})", dX, dXr)
        _close(f"dY ({name})", dY, dYr)


def test_rbf_repeatable():
    announce("rbf run-to-run determinism")
    X, Y, G = _inputs(1024, 1024, 64, 9)
    a = _run_autograd(X, Y, G, 0.5)
    b = _run_autograd(X, Y, G, 0.5)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("size", [2048, 4096])
def test_rbf_verify_all_framework(size):
    """The framework's parity harness (the reference's verify.py protocol:
    five seeds, the case's own reference.py through autograd, here run by
    torch on the device, 4 GiB of broadcast intermediate at 4096) at config
    sizes 1 and 2."""
    announce(f"rbf verify_all {size} (case reference.py path)")
    from cases.rbf import baseline_case, op
    ok, report = verify_all(baseline_case(size), op.candidate, device="cuda")
    print(report)
    assert ok, report
