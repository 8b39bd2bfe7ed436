"""Graph capture of the launches that hand values between workgroups
through nonce-tagged slots (the long-row scan, the softmax CE forward and
the column offsets of the SpMM backward), and of the SpMV D = 1 forward and
sorted backward, the RBF forward and backward, and LayerNorm.
A captured launch keeps the nonce it was captured with, so the libraries
clear the slots with a fill kernel captured ahead of it.  Each test replays
one graph several times on new inputs, with eager calls and
synchronisations between the replays, and checks every replay against the
oracle and against an eager call on the same inputs."""

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import scan as oscan
from oracle import softmax_ce as osce

pytestmark = pytest.mark.gpu


def _capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


@pytest.mark.parametrize("rows,d", [(64, 65536), (3, 100003)])
def test_scan_graph_replays_with_new_inputs(rows, d):
    announce(f"scan graph capture rows={rows} d={d}")
    from cases.scan import op
    x_static = torch.zeros(rows, d, device="cuda")
    g, y_static = _capture(lambda: op.scan_forward(x_static))
    for seed in range(4):
        gen = torch.Generator().manual_seed(100 + seed)
        x = (torch.rand(rows, d, generator=gen, dtype=torch.float64) * 2 - 1).float()
        x_static.copy_(x.cuda())
        g.replay()
        torch.cuda.synchronize()
        got = y_static.cpu().numpy().astype(np.float64)
        ref = oscan.cumsum_f32(x.numpy()).astype(np.float64)
        err = np.abs(got - ref)
        print(f"  replay {seed}: max_abs={err.max():.3e}")
        assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref)), f"replay {seed}"
        eager = op.scan_forward(x_static.clone())  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager, y_static), f"replay {seed} differs from the eager call"


def test_scan_graphs_keep_their_own_workspaces():
    """Two graphs, each holding a multi-chunk scan, captured on the shared
    capture stream, replayed alternately with a larger eager scan between
    the replays (which replaces the eagerly cached workspace): every replay
    still matches the oracle."""
    announce("scan: two captured graphs and eager calls in between")
    from cases.scan import op
    xa = torch.zeros(8, 40000, device="cuda")
    xb = torch.zeros(5, 70001, device="cuda")
    ga, ya = _capture(lambda: op.scan_forward(xa))
    gb, yb = _capture(lambda: op.scan_forward(xb))
    for seed in range(3):
        gen = torch.Generator().manual_seed(300 + seed)
        a = (torch.rand(8, 40000, generator=gen, dtype=torch.float64) * 2 - 1).float()
        b = (torch.rand(5, 70001, generator=gen, dtype=torch.float64) * 2 - 1).float()
        xa.copy_(a.cuda())
        xb.copy_(b.cuda())
        ga.replay()
        gb.replay()
        big = op.scan_forward(torch.ones(16 + seed, 300000, device="cuda"))
        torch.cuda.synchronize()
        assert float(big[0, -1]) == 300000.0
        for name, y, x in (("a", ya, a), ("b", yb, b)):
            ref = oscan.cumsum_f32(x.numpy()).astype(np.float64)
            err = np.abs(y.cpu().numpy().astype(np.float64) - ref)
            print(f"  replay {seed} graph {name}: max_abs={err.max():.3e}")
            assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref)), f"replay {seed} graph {name}"


def test_scan_int_graph_replays_bit_exact():
    announce("scan int32 -> int64 graph capture [64, 65536]")
    from cases.scan import op
    x_static = torch.zeros(64, 65536, dtype=torch.int32, device="cuda")
    g, y_static = _capture(lambda: op.scan_forward(x_static))
    for seed in range(3):
        gen = torch.Generator().manual_seed(200 + seed)
        x = torch.randint(-1000, 1001, (64, 65536), generator=gen, dtype=torch.int32)
        x_static.copy_(x.cuda())
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y_static.cpu().numpy(), oscan.cumsum_i64(x.numpy())), seed


def test_softmax_ce_forward_graph_replays_with_new_inputs():
    announce("softmax_ce forward graph capture [8192, 1024]")
    from cases.softmax_ce import op
    b, c = 8192, 1024
    x_static = torch.zeros(b, c, device="cuda")
    lab_static = torch.zeros(b, dtype=torch.int64, device="cuda")
    g, (loss_static, lse_static) = _capture(lambda: op.sce_forward(x_static, lab_static))
    for seed in range(4):
        gen = torch.Generator().manual_seed(300 + seed)
        x = torch.randn(b, c, generator=gen)
        lab = torch.randint(0, c, (b,), generator=gen)
        x_static.copy_(x.cuda())
        lab_static.copy_(lab.cuda())
        g.replay()
        torch.cuda.synchronize()
        rloss, rlse = osce.forward_f64(x.double().numpy(), lab.numpy())
        got = float(loss_static.item())
        print(f"  replay {seed}: loss={got:.6f} ref={rloss:.6f}")
        assert abs(got - rloss) <= 1e-3 + 1e-3 * abs(rloss), f"replay {seed}"
        assert np.allclose(lse_static.cpu().numpy(), rlse, atol=1e-3, rtol=1e-3)
        eager, _ = op.sce_forward(x_static.clone(), lab_static.clone())
        torch.cuda.synchronize()
        assert torch.equal(eager, loss_static), f"replay {seed} differs from the eager call"


def _wide_spmm_inputs(m=2048, k=16384, d=8, per_row=64, seed=0):
    """M x K CSR with per_row sorted unique random columns per row, X [K, D]."""
    rng = np.random.default_rng(seed)
    cols = np.sort(np.stack([rng.choice(k, per_row, replace=False) for _ in range(m)]), axis=1)
    ptr = np.arange(m + 1, dtype=np.int64) * per_row
    g = torch.Generator().manual_seed(seed)
    return {"row_ptr": torch.from_numpy(ptr), "col_idx": torch.from_numpy(cols.reshape(-1)),
            "vals": torch.randn(m * per_row, generator=g), "X": torch.randn(k, d, generator=g)}


@pytest.mark.parametrize("shape", ["reference default M=K=4096 D=64 (column blocks)",
                                   "K=16384 D=8 (column blocks of 64)",
                                   "K=16384 D=32 (column-major copy, 80 KB of scatter LDS)"])
def test_spmm_backward_graph_replays_with_new_inputs(shape):
    """Both D > 1 dX routes captured once and replayed on new dY: every
    replay matches the float64 oracle and an eager call bit for bit."""
    announce(f"spmm backward graph capture ({shape})")
    from cases.spmv import op, reference as ref
    from oracle import spmv as osp
    t = ref.make_inputs(0, torch.float32, "cpu") if shape.startswith("reference") \
        else _wide_spmm_inputs(d=int(shape.split("D=")[1].split()[0]))
    ptr, col, vals, X = (t[k].cuda() for k in ("row_ptr", "col_idx", "vals", "X"))
    M, D = ptr.numel() - 1, X.shape[1]
    dy_static = torch.zeros(M, D, device="cuda")
    g, (dv_static, dx_static) = _capture(lambda: op.spmv_backward(ptr, col, vals, X, dy_static))
    hp, hc, hv, hx = (t[k].numpy() for k in ("row_ptr", "col_idx", "vals", "X"))
    for seed in range(3):
        dy = torch.randn(M, D, generator=torch.Generator().manual_seed(400 + seed))
        dy_static.copy_(dy.cuda())
        g.replay()
        torch.cuda.synchronize()
        rdv, rdx = osp.backward_f64(hp, hc, hv, hx, dy.numpy())
        for name, got, ref_ in (("dvals", dv_static, rdv), ("dX", dx_static, rdx)):
            err = np.abs(got.cpu().double().numpy() - ref_)
            print(f"  replay {seed} {name}: max_abs={err.max():.3e}")
            assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref_)), f"replay {seed}: {name}"
        edv, edx = op.spmv_backward(ptr, col, vals, X, dy_static.clone())
        torch.cuda.synchronize()
        assert torch.equal(edx, dx_static) and torch.equal(edv, dv_static), f"replay {seed}"


def test_spmv_d1_graph_replays_with_new_inputs():
    """The D = 1 forward (one resident round of walk waves) and the sorted dX
    backward (row table, sort, bucket sums over a workspace with no initial
    contents) captured once and replayed on new x and dy."""
    announce("spmv D=1 forward + backward graph capture (Zipf 2^16)")
    from cases.spmv import op, reference as ref
    from oracle import spmv as osp
    m = k = 1 << 16
    t = ref.make_zipf_inputs(m, k, 1, 5, torch.int32)
    ptr, col, vals = (t[n].cuda() for n in ("row_ptr", "col_idx", "vals"))
    x_static = torch.zeros(k, 1, device="cuda")
    dy_static = torch.zeros(m, 1, device="cuda")

    def step():
        y = op.spmv_forward(ptr, col, vals, x_static)
        dv, dx = op.spmv_backward(ptr, col, vals, x_static, dy_static)
        return y, dv, dx

    g, (y_s, dv_s, dx_s) = _capture(step)
    hp, hc, hv = (t[n].numpy() for n in ("row_ptr", "col_idx", "vals"))
    for seed in range(3):
        gen = torch.Generator().manual_seed(500 + seed)
        x, dy = torch.randn(k, 1, generator=gen), torch.randn(m, 1, generator=gen)
        x_static.copy_(x.cuda())
        dy_static.copy_(dy.cuda())
        g.replay()
        torch.cuda.synchronize()
        ry = osp.forward_f64(hp, hc, hv, x.numpy())
        rdv, rdx = osp.backward_f64(hp, hc, hv, x.numpy(), dy.numpy())
        for name, got, ref_ in (("y", y_s, ry), ("dvals", dv_s, rdv), ("dX", dx_s, rdx)):
            err = np.abs(got.cpu().double().numpy() - ref_)
            print(f"  replay {seed} {name}: max_abs={err.max():.3e}")
            assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref_)), f"replay {seed}: {name}"
        ey, edv, _ = step()
        torch.cuda.synchronize()
        assert torch.equal(ey, y_s) and torch.equal(edv, dv_s), f"replay {seed}"


def test_rbf_graph_replays_with_new_inputs():
    """The headline RBF forward and backward (tile kernels plus the partial
    reduce, workspace from the caching allocator) captured once and replayed
    on new X, Y and dK: every replay equals an eager call bit for bit and
    matches the float64 oracle."""
    announce("rbf forward + backward graph capture (N = M = 1024)")
    from cases.rbf import op
    from oracle import rbf as orbf
    n = m = 1024
    x_s = torch.zeros(n, 64, device="cuda")
    y_s = torch.zeros(m, 64, device="cuda")
    g_s = torch.zeros(n, m, device="cuda")

    def step():
        xd = x_s.detach().requires_grad_(True)
        yd = y_s.detach().requires_grad_(True)
        k = op.candidate({"X": xd, "Y": yd}, {"gamma": 0.5})
        dx, dy = torch.autograd.grad(k, (xd, yd), g_s)
        return k.detach(), dx, dy

    g, (k_s, dx_s, dy_s) = _capture(step)
    for seed in range(3):
        gen = torch.Generator().manual_seed(600 + seed)
        X = torch.randn(n, 64, generator=gen) * 0.125
        Y = torch.randn(m, 64, generator=gen) * 0.125
        G = torch.randn(n, m, generator=gen)
        x_s.copy_(X.cuda())
        y_s.copy_(Y.cuda())
        g_s.copy_(G.cuda())
        g.replay()
        torch.cuda.synchronize()
        Kr = orbf.forward_f64(X.numpy(), Y.numpy(), 0.5)
        dXr, dYr = orbf.backward_f64(X.numpy(), Y.numpy(), G.numpy(), Kr, 0.5)
        for name, got, ref_ in (("K", k_s, Kr), ("dX", dx_s, dXr), ("dY", dy_s, dYr)):
            err = np.abs(got.cpu().double().numpy() - ref_)
            print(f"  replay {seed} {name}: max_abs={err.max():.3e}")
            assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref_)), f"replay {seed}: {name}"
        ek, edx, edy = step()
        torch.cuda.synchronize()
        assert torch.equal(ek, k_s) and torch.equal(edx, dx_s) and torch.equal(edy, dy_s), seed


@pytest.mark.parametrize("b,d", [(512, 4096), (300, 1000)])
def test_layernorm_graph_replays_with_new_inputs(b, d):
    """LayerNorm forward and backward (row kernels and the column sums; the
    generic path at D = 1000) captured once and replayed on new inputs: every
    replay equals an eager call bit for bit and matches the float64 oracle."""
    announce(f"layernorm graph capture [{b},{d}]")
    from cases.layernorm import op
    from oracle import layernorm as oln
    eps = 1e-5
    x_s = torch.zeros(b, d, device="cuda")
    w_s = torch.ones(d, device="cuda")
    bias_s = torch.zeros(d, device="cuda")
    dy_s = torch.zeros(b, d, device="cuda")

    def step():
        xd = x_s.detach().requires_grad_(True)
        wd = w_s.detach().requires_grad_(True)
        bd = bias_s.detach().requires_grad_(True)
        y = op.candidate({"X": xd, "gamma": wd, "beta": bd}, {"eps": eps})
        grads = torch.autograd.grad(y, (xd, wd, bd), dy_s)
        return (y.detach(),) + tuple(grads)

    g, outs = _capture(step)
    for seed in range(3):
        gen = torch.Generator().manual_seed(700 + seed)
        x = torch.randn(b, d, generator=gen)
        w = 1 + 0.1 * torch.randn(d, generator=gen)
        bias = 0.1 * torch.randn(d, generator=gen)
        dy = torch.randn(b, d, generator=gen)
        for dst, src in ((x_s, x), (w_s, w), (bias_s, bias), (dy_s, dy)):
            dst.copy_(src.cuda())
        g.replay()
        torch.cuda.synchronize()
        ry, _, _ = oln.forward_f64(x.numpy(), w.numpy(), bias.numpy(), eps)
        rdx, rdw, rdb = oln.backward_f64(dy.numpy(), x.numpy(), w.numpy(), eps)
        for name, got, ref_ in zip(("y", "dx", "dw", "db"), outs, (ry, rdx, rdw, rdb)):
            err = np.abs(got.cpu().double().numpy() - ref_)
            print(f"  replay {seed} {name}: max_abs={err.max():.3e}")
            assert np.all(err <= 1e-3 + 1e-3 * np.abs(ref_)), f"replay {seed}: {name}"
        eager = step()
        torch.cuda.synchronize()
        assert all(torch.equal(e, o) for e, o in zip(eager, outs)), seed
