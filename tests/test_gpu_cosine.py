"""Cosine-similarity parity on the GPU: the HIP library (through its C-ABI
and through the autograd op) against the float64 oracle, at
atol = rtol = 1e-3.

Workloads: A, B ~ N(0,1), dS ~ N(0,1); N = M = 2048 (the reference default)
for two seeds and 4096 for one, forward S, the inverse norms and backward
dA, dB; ragged shapes, the generic path (D != 64, misaligned rows), zero
rows, a large eps, empty inputs, invariants (|S| <= 1, S(A, A) has a unit
diagonal), argument checks, and the framework's verify_all at the
reference defaults.
"""

import numpy as np
import pytest
import torch

from conftest import announce
from framework import capi
from framework.verify import verify_all
from oracle import cosine_sim as oc

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-3


def _op():
    from cases.cosine_sim import op
    return op


def _inputs(n, m, d, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(n, d, generator=g)
    B = torch.randn(m, d, generator=g)
    dS = torch.randn(n, m, generator=torch.Generator().manual_seed(seed + 10_000))
    return A, B, dS


def _close(name, got, ref, atol=ATOL, rtol=RTOL):
    got = got.detach().cpu().double().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    max_rel = float((err / np.maximum(np.abs(ref), 1e-30)).max()) if err.size else 0.0
    print(f"  {name}: max_abs={max_abs:.3e} max_rel={max_rel:.3e}")
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {int(bad.sum())} entries outside tolerance (max_abs {max_abs:.3e})"


def _check(A, B, dS, eps=1e-8, a_dev=None):
    op = _op()
    Ad = (A.cuda() if a_dev is None else a_dev).requires_grad_(True)
    Bd = B.cuda().requires_grad_(True)
    S = op.candidate({"A": Ad, "B": Bd}, {"eps": eps})
    S.backward(dS.cuda())
    _, inv_a, inv_b = op.cos_forward(Ad.detach(), Bd.detach(), eps)
    torch.cuda.synchronize()
    An, Bn, dSn = A.double().numpy(), B.double().numpy(), dS.double().numpy()
    _close("S", S, oc.forward_f64(An, Bn, eps))
    _close("inv_a", inv_a, oc.inv_norms(An, eps))
    _close("inv_b", inv_b, oc.inv_norms(Bn, eps))
    rA, rB = oc.backward_f64(An, Bn, dSn, eps)
    _close("dA", Ad.grad, rA)
    _close("dB", Bd.grad, rB)
    return S


@pytest.mark.parametrize("n,seed", [(2048, 0), (2048, 1), (4096, 2)])
def test_cosine_square_vs_oracle(n, seed):
    announce(f"cosine_sim N=M={n} D=64 seed={seed}")
    A, B, dS = _inputs(n, n, 64, seed)
    S = _check(A, B, dS)
    assert float(S.abs().max()) <= 1.0 + 1e-6


@pytest.mark.parametrize("n,m,d", [(1000, 3000, 64), (1, 1, 64), (5, 7, 64), (300, 257, 64),
                                   (129, 65, 32), (200, 150, 100), (64, 64, 1), (3000, 3008, 64),
                                   # tiled generic kernels: ragged tiles, feature chunks and
                                   # passes, the backward's walks in several slices
                                   (1000, 1000, 32), (257, 65, 128), (300, 129, 200), (70, 1500, 3)])
def test_cosine_shapes(n, m, d):
    announce(f"cosine_sim N={n} M={m} D={d}")
    A, B, dS = _inputs(n, m, d, n + m + d)
    _check(A, B, dS)


def test_cosine_generic_zero_rows():
    announce("cosine_sim generic path, zero rows, D=48")
    A, B, dS = _inputs(500, 400, 48, 9)
    A[3] = 0.0
    B[17] = 0.0
    _check(A, B, dS)


def test_cosine_zero_rows_and_large_eps():
    announce("cosine_sim zero rows, eps = 0.5")
    A, B, dS = _inputs(300, 200, 64, 7)
    A[3] = 0.0
    B[17] = 0.0
    _check(A, B, dS)
    _check(A, B, dS, eps=0.5)


def test_cosine_misaligned_rows():
    announce("cosine_sim misaligned A (generic path)")
    A, B, dS = _inputs(130, 90, 64, 8)
    buf = torch.empty(A.numel() + 1, device="cuda")
    buf[1:].copy_(A.reshape(-1).cuda())
    _check(A, B, dS, a_dev=buf[1:].view(130, 64))


def test_cosine_self_similarity_diagonal():
    announce("cosine_sim S(A, A) diagonal")
    A, _, _ = _inputs(512, 1, 64, 9)
    S = _op().forward_only({"A": A.cuda(), "B": A.cuda()}, {"eps": 1e-8})
    torch.cuda.synchronize()
    assert torch.allclose(torch.diagonal(S).cpu(), torch.ones(512), atol=1e-5)


def test_cosine_empty_inputs():
    announce("cosine_sim N = 0 / M = 0")
    op = _op()
    A, B, _ = _inputs(0, 5, 64, 10)
    S, inv_a, inv_b = op.cos_forward(A.cuda(), B.cuda(), 1e-8)
    dA, dB = op.cos_backward(A.cuda(), B.cuda(), inv_a, inv_b, torch.zeros(0, 5, device="cuda"))
    torch.cuda.synchronize()
    assert S.shape == (0, 5) and torch.all(dB == 0)
    _close("inv_b", inv_b, oc.inv_norms(B.double().numpy(), 1e-8))


def test_cosine_rejects_bad_arguments():
    announce("cosine_sim argument checks")
    op = _op()
    A, B, _ = _inputs(4, 4, 64, 11)
    with pytest.raises(RuntimeError, match="eps"):
        op.cos_forward(A.cuda(), B.cuda(), -1.0)
    with pytest.raises(RuntimeError, match="feature dim"):
        op.cos_forward(A.cuda(), B[:, :32].cuda(), 1e-8)


def test_cosine_verify_all_reference_defaults():
    announce("cosine_sim verify_all (reference defaults 2048 x 2048 x 64)")
    from cases.cosine_sim import CASE, op
    ok, report = verify_all(CASE, op.candidate, device="cuda")
    print(report)
    assert ok, report
