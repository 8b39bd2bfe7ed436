"""Scan parity on the GPU (libscan_hip.so) against the oracle: fp32 forward and
backward within atol = rtol = 1e-3 (and, since both accumulate in float64,
equal to torch's CPU cumsum in all but a few rounding-tie elements), int32
bit-exact.  Shapes: the acceptance workload [64, 65536], the reference's
default [4096, 4096], ragged widths (scalar path), rows longer than 256
chunks (multi-tile chunks), more chunks than resident workgroups (persistent
loop), misaligned pointers, empty inputs, NaN inputs, and full-size identities."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import announce
from framework import capi
from framework.verify import verify_all
from oracle import scan as osc

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _read_trip_counter(monkeypatch):
    """Every scan call through op.py zeroes the workspace's trip counter
    first and reads it after, raising if a chunk's carry wait hit the spin
    cap (so every test below also asserts the counter stays 0)."""
    monkeypatch.setenv("NL2K_CHECK", "1")


def _u(rows, d, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(rows, d, generator=g, dtype=torch.float64) * 2 - 1).float()


def _ints(rows, d, seed, low=-1000, high=1000):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(low, high + 1, (rows, d), generator=g, dtype=torch.int32)


def _close(name, got, ref, atol=1e-3, rtol=1e-3, min_equal=None):
    got = got.detach().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape
    err = np.abs(got - ref)
    max_abs = float(err.max()) if err.size else 0.0
    eq = float(np.mean(got == ref)) if err.size else 1.0
    print(f"  {name}: max_abs={max_abs:.3e} bit-equal fraction={eq:.6f}")
    assert np.all(err <= atol + rtol * np.abs(ref)), f"{name}: max_abs {max_abs:.3e}"
    if min_equal is not None:
        assert eq >= min_equal, f"{name}: only {eq:.6f} of elements equal the fp64-sum reference"


def _op():
    from cases.scan import op
    return op


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_scan_f32_baseline_64x65536(seed):
    announce(f"scan f32 [64, 65536] seed={seed}")
    op = _op()
    x = _u(64, 65536, seed)
    dy = torch.randn(64, 65536, generator=torch.Generator().manual_seed(seed + 10_000))
    xd = x.cuda().requires_grad_(True)
    y = op.candidate({"X": xd}, {})
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    _close("y", y, osc.cumsum_f32(x.numpy()), min_equal=0.999)
    _close("dx", xd.grad, osc.reverse_cumsum_f32(dy.numpy()), min_equal=0.999)


def test_scan_nan_propagates_across_chunks():
    """A NaN makes every later element of its row NaN, as torch's cumsum
    does, also in the row's later chunks (the NaN reaches them through the
    published chunk totals); rows without one match the oracle, and the
    reverse scan of the backward carries it towards the row's start."""
    announce("scan f32 NaN across chunks")
    op = _op()
    x = _u(4, 65536, 21)
    x[1, 5000] = float("nan")   # inside the second 4096-element chunk
    x[2, 65535] = float("nan")  # the last element
    dy = torch.randn(4, 65536, generator=torch.Generator().manual_seed(22))
    dy[3, 30000] = float("nan")
    xd = x.cuda().requires_grad_(True)
    y = op.candidate({"X": xd}, {})
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    yc, gc = y.detach().cpu(), xd.grad.cpu()
    ref_y = torch.cumsum(x.double(), dim=1)
    ref_g = torch.flip(torch.cumsum(torch.flip(dy.double(), [1]), dim=1), [1])
    assert torch.equal(torch.isnan(yc), torch.isnan(ref_y))
    assert torch.equal(torch.isnan(gc), torch.isnan(ref_g))
    assert torch.isnan(yc[1, 5000:]).all() and not torch.isnan(yc[1, :5000]).any()
    assert torch.isnan(gc[3, :30001]).all() and not torch.isnan(gc[3, 30001:]).any()
    _close("y (rows 0, 3)", yc[[0, 3]], osc.cumsum_f32(x[[0, 3]].numpy()))
    _close("dx (rows 0-2)", gc[:3], osc.reverse_cumsum_f32(dy[:3].numpy()))


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4])
def test_scan_i32_to_i64_bit_exact(seed):
    announce(f"scan int32 -> int64 [64, 65536] seed={seed}")
    x = _ints(64, 65536, seed)
    y = _op().scan_forward(x.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.int64
    assert np.array_equal(y.cpu().numpy(), osc.cumsum_i64(x.numpy()))
    assert torch.equal(y.cpu(), torch.cumsum(x, -1))


@pytest.mark.parametrize("rows,d", [(8, 70001), (300, 64), (70, 999)])
def test_scan_i32_wrapping_variant(rows, d):
    announce(f"scan int32 -> int32 wrap [{rows}, {d}]")
    x = _ints(rows, d, 5, -(2**31), 2**31 - 1)
    y = _op().scan_forward_int32(x.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.int32
    assert np.array_equal(y.cpu().numpy(), osc.cumsum_i32_wrap(x.numpy()))
    y64 = _op().scan_forward(x.cuda())  # extreme values: exact in int64
    torch.cuda.synchronize()
    assert np.array_equal(y64.cpu().numpy(), osc.cumsum_i64(x.numpy()))


@pytest.mark.parametrize("rows,d", [(1, 1), (3, 3), (2, 5), (5, 4095), (4, 4096), (3, 4097),
                                    (7, 8191), (2, 65537), (3, 100003), (1, 1 << 20),
                                    (2, (1 << 21) + 5), (128, 65536), (700, 8192),
                                    (65536, 64), (1000, 16), (333, 100), (257, 7), (4097, 256),
                                    (129, 300), (77, 1000), (1025, 1024), (5, 513), (3, 1025),
                                    (33, 2000), (1025, 1537), (7, 2048), (2, 2049)])
def test_scan_shapes(rows, d):
    announce(f"scan rows={rows} d={d}")
    op = _op()
    x = _u(rows, d, rows * 7 + d)
    xi = _ints(rows, d, rows + d)
    y = op.scan_forward(x.cuda())
    yb = op.scan_backward(x.cuda())
    yi = op.scan_forward(xi.cuda())
    torch.cuda.synchronize()
    _close("fwd", y, osc.cumsum_f32(x.numpy()))
    _close("bwd", yb, osc.reverse_cumsum_f32(x.numpy()))
    assert np.array_equal(yi.cpu().numpy(), osc.cumsum_i64(xi.numpy()))


def test_scan_misaligned_and_strided_input():
    announce("scan misaligned / non-contiguous")
    op = _op()
    x = _u(6, 20000, 3)
    buf = torch.empty(6 * 20000 + 1, device="cuda")
    buf[1:].copy_(x.reshape(-1).cuda())
    xm = buf[1:].view(6, 20000)  # 4-byte offset: scalar path
    _close("misaligned fwd", op.scan_forward(xm), osc.cumsum_f32(x.numpy()))
    _close("misaligned bwd", op.scan_backward(xm), osc.reverse_cumsum_f32(x.numpy()))
    xt = x.t().contiguous().cuda().t()  # non-contiguous view: op makes it contiguous
    _close("strided fwd", op.scan_forward(xt), osc.cumsum_f32(x.numpy()))


def test_scan_rejects_bad_arguments():
    announce("scan argument checks")
    op = _op()
    with pytest.raises(RuntimeError, match="2D"):
        op.scan_forward(torch.zeros(4, device="cuda"))
    with pytest.raises(RuntimeError, match="float32"):
        op.scan_backward(torch.zeros(2, 4, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="at least one row"):
        op.scan_forward(torch.zeros(0, 4, device="cuda"))


def test_scan_full_size_identities():
    """At the acceptance size: the last column equals the float64 row sums,
    the reverse scan equals flip(scan(flip)) bit for bit, repeated calls are
    bitwise identical, a workspace needs no initial contents (zeros, random
    bits, and what the previous call left all give the same results), and
    the C-ABI's hang-guard counter stays zero."""
    announce("scan identities [64, 65536]")
    op = _op()
    lib = op._lib()
    x = _u(64, 65536, 9).cuda()
    y1 = op.scan_forward(x)
    y2 = op.scan_forward(x)
    rb = op.scan_backward(x)
    fl = op.scan_forward(torch.flip(x, dims=[1])).flip(dims=[1])
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(rb, fl)
    rowsum = x.double().sum(dim=1).float()
    assert torch.allclose(y1[:, -1], rowsum, atol=1e-3, rtol=1e-3)
    assert torch.allclose(rb[:, 0], rowsum, atol=1e-3, rtol=1e-3)
    # direct C-ABI calls on one workspace, first zero-filled, then random
    # bits (all but the last word, which counts hang-guard trips and must
    # stay 0), then reused as the previous calls left it
    rows, d = x.shape
    nbytes = lib.scan_workspace_bytes(rows, d)
    ws = torch.zeros(nbytes // 8, dtype=torch.int64, device="cuda")
    junk = torch.randint(-2**62, 2**62, (nbytes // 8 - 1,), generator=torch.Generator().manual_seed(5))
    for k, fn in enumerate((lib.scan_forward_f32, lib.scan_backward_f32, lib.scan_forward_f32,
                            lib.scan_forward_f32)):
        if k == 1:
            ws[:-1].copy_(junk.cuda())
        y3 = torch.empty_like(x)
        st = fn(capi.ptr(x), capi.ptr(y3), rows, d, capi.ptr(ws), nbytes, capi.stream_of(x))
        assert st == 0, lib.scan_last_error()
        torch.cuda.synchronize()
        assert torch.equal(y3, y1 if fn is lib.scan_forward_f32 else rb)
        assert int(ws[lib.scan_status_offset(rows, d) // 8]) == 0, "hang guard tripped"


def test_scan_verify_all_reference_defaults():
    announce("scan verify_all (reference defaults [4096, 4096] N(0,1))")
    from cases.scan import CASE, op
    ok, report = verify_all(CASE, op.candidate, device="cuda")
    print(report)
    assert ok, report


def test_scan_verify_int_case():
    announce("scan verify_all int32 [64, 65536]")
    from cases.scan import int_case, op
    ok, report = verify_all(int_case(), op.forward_only, device="cuda", backward=False)
    print(report)
    assert ok, report
