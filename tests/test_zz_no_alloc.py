"""The allocation-free RBF backward (rbf_backward_f32_noalloc) against the
workspace entry point rbf_backward_f32 through the C-ABI: bit-identical dX
and dY (same kernels, same order of additions), both within atol = rtol =
1e-3 of the float64 oracle, on calls in a row whose later shapes are smaller
(the library's scratch keeps the previous call's partials), on the vector
and the scalar tile paths; a tile-path shape beyond the scratch rejected,
and a generic-path call beyond it run without scratch."""

import numpy as np
import pytest
import torch

from conftest import announce
from framework import capi
from oracle import rbf as orbf

pytestmark = pytest.mark.gpu


def _inputs(n, m, seed):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n, 64, generator=g) / 8
    Y = torch.randn(m, 64, generator=g) / 8
    G = torch.randn(n, m, generator=torch.Generator().manual_seed(seed + 10_000))
    return X, Y, G


def test_noalloc_backward_matches_workspace_entry():
    from cases.rbf import op
    lib = op._lib()
    gamma = 0.5
    for k, (n, m) in enumerate(((4096, 4096), (1000, 2052), (513, 2049))):
        announce(f"rbf noalloc call {k}: n={n} m={m}")
        X, Y, G = _inputs(n, m, 40 + k)
        Xd, Yd, Gd = X.cuda(), Y.cuda(), G.cuda()
        K = op.rbf_forward(Xd, Yd, gamma)
        s = capi.stream_of(Xd)
        P = capi.ptr
        need = lib.rbf_backward_workspace_bytes(n, m, 64)
        assert 0 < need <= lib.rbf_backward_noalloc_max_bytes()
        ws = torch.empty(need // 4, device="cuda")
        dX_ref, dY_ref = torch.empty_like(Xd), torch.empty_like(Yd)
        st = lib.rbf_backward_f32(P(Xd), P(Yd), P(Gd), P(K), P(dX_ref), P(dY_ref), n, m, 64, gamma,
                                  P(ws), need, s)
        capi.check(st, lib.rbf_last_error, "rbf_backward_f32")
        dX, dY = torch.full_like(Xd, float("nan")), torch.full_like(Yd, float("nan"))
        st = lib.rbf_backward_f32_noalloc(P(Xd), P(Yd), P(Gd), P(K), P(dX), P(dY), n, m, 64, gamma,
                                          s)
        capi.check(st, lib.rbf_last_error, "rbf_backward_f32_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(dX, dX_ref) and torch.equal(dY, dY_ref), f"call {k} differs"
        Kr = orbf.forward_f64(X.numpy(), Y.numpy(), gamma)
        dXr, dYr = orbf.backward_f64(X.numpy(), Y.numpy(), G.numpy(), Kr, gamma)
        for name, got, ref in (("dX", dX, dXr), ("dY", dY, dYr)):
            got = got.cpu().double().numpy()
            err = np.abs(got - ref)
            print(f"  {name}: max_abs={err.max():.3e}")
            assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref)), f"call {k}: {name}"


def test_noalloc_backward_rejects_a_shape_beyond_its_scratch():
    announce("rbf noalloc 8192 rejected")
    from cases.rbf import op
    lib = op._lib()
    x = torch.zeros(8, 64, device="cuda")
    P = capi.ptr
    st = lib.rbf_backward_f32_noalloc(P(x), P(x), P(x), P(x), P(x), P(x), 8192, 8192, 64, 0.5,
                                      capi.stream_of(x))
    assert st != 0 and b"scratch" in lib.rbf_last_error()


def test_noalloc_backward_generic_path_needs_no_scratch():
    """A misaligned X takes the generic kernels, which use no scratch: the
    no-alloc entry runs it even where the tile path's partials would not fit
    (N = M = 6000 needs about 100 MB of them), bit-identical to the workspace
    entry."""
    n = m = 6000
    announce(f"rbf noalloc, misaligned X, n={n} m={m} (generic kernels)")
    from cases.rbf import op
    lib = op._lib()
    gamma = 0.5
    assert lib.rbf_backward_workspace_bytes(n, m, 64) > lib.rbf_backward_noalloc_max_bytes()
    X, Y, G = _inputs(n, m, 3)
    buf = torch.empty(n * 64 + 1, device="cuda")
    Xd = buf[1:].view(n, 64)
    Xd.copy_(X.cuda())
    Yd, Gd = Y.cuda(), G.cuda()
    K = op.rbf_forward(Xd, Yd, gamma)
    P = capi.ptr
    dX0, dY0 = torch.empty(n, 64, device="cuda"), torch.empty(m, 64, device="cuda")
    ws = torch.empty(8, dtype=torch.uint8, device="cuda")
    st = lib.rbf_backward_f32(P(Xd), P(Yd), P(Gd), P(K), P(dX0), P(dY0), n, m, 64, gamma, P(ws),
                              0, capi.stream_of(Xd))
    capi.check(st, lib.rbf_last_error, "rbf_backward_f32 (misaligned X)")
    dX1, dY1 = torch.empty_like(dX0), torch.empty_like(dY0)
    st = lib.rbf_backward_f32_noalloc(P(Xd), P(Yd), P(Gd), P(K), P(dX1), P(dY1), n, m, 64, gamma,
                                      capi.stream_of(Xd))
    capi.check(st, lib.rbf_last_error, "rbf_backward_f32_noalloc (misaligned X)")
    torch.cuda.synchronize()
    assert torch.equal(dX0, dX1) and torch.equal(dY0, dY1)
    sub = slice(0, 48)  # the oracle on a row block: dX rows need all of Y and G's rows
    Kr = orbf.forward_f64(X.numpy()[sub], Y.numpy(), gamma)
    dXr, _ = orbf.backward_f64(X.numpy()[sub], Y.numpy(), G.numpy()[sub], Kr, gamma)
    err = np.abs(dX1[sub].cpu().double().numpy() - dXr)
    print(f"  dX rows 0-47: max_abs={err.max():.3e}")
    assert np.all(err <= 1e-3 + 1e-3 * np.abs(dXr))
