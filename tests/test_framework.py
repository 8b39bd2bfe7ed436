"""The parity harness on the CPU (framework/verify.py): the comparison rule
is torch.allclose's at atol = rtol = 1e-3 (the reference's check,
framework/verify.py:35-105), integers compare exactly, and verify_all reports
PASS for the reference itself and FAIL for a forward or a gradient with a
planted mistake."""

import torch

from framework.verify import compare_tensors, verify_all

INF, NAN = float("inf"), float("nan")


def test_compare_follows_allclose():
    ref = torch.tensor([1.0, -2.0, 0.0, INF, -INF])
    ok, a, r = compare_tensors(ref + torch.tensor([9e-4, -2e-3, 9.9e-4, 0.0, 0.0]), ref)
    assert ok  # within atol + rtol |ref| everywhere; equal infinities are close
    assert abs(a - 2e-3) < 1e-6 and r > 0
    assert not compare_tensors(torch.tensor([1.0021]), torch.tensor([1.0]))[0]
    assert not compare_tensors(torch.tensor([INF]), torch.tensor([-INF]))[0]
    assert not compare_tensors(torch.tensor([NAN]), torch.tensor([NAN]))[0]
    assert not compare_tensors(torch.tensor([1.0]), torch.tensor([NAN]))[0]
    for t in (ref, torch.tensor([1.0, 2.0])):
        assert torch.allclose(t, t) == compare_tensors(t, t)[0]


def test_compare_integers_and_shapes():
    x = torch.tensor([1, -5, 7], dtype=torch.int32)
    assert compare_tensors(x, x.to(torch.int64)) == (True, 0.0, 0.0)
    ok, a, _ = compare_tensors(x + torch.tensor([0, 1, 0], dtype=torch.int32), x.to(torch.int64))
    assert not ok and a == 1.0
    assert not compare_tensors(torch.zeros(3), torch.zeros(4))[0]
    assert compare_tensors(torch.zeros(0, 5), torch.zeros(0, 5))[0]


def _scan_case():
    from cases.scan import make_case
    return make_case(4, 300)


def test_verify_all_passes_the_reference():
    case = _scan_case()
    ok, report = verify_all(case, case.reference_forward, device="cpu")
    assert ok, report
    assert "=== overall: PASS ===" in report and report.count("seed=") == 10


def test_verify_all_catches_a_forward_mistake():
    case = _scan_case()

    def off_by_one_column(inputs, params):
        y = case.reference_forward(inputs, params)
        return torch.cat([y[:, :1] * 0, y[:, :-1]], dim=1)  # exclusive scan

    ok, report = verify_all(case, off_by_one_column, device="cpu")
    assert not ok and "[forward] FAIL" in report


class _DoubledGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return x.cumsum(-1)

    @staticmethod
    def backward(ctx, g):
        return 2 * g.flip(-1).cumsum(-1).flip(-1)


def test_verify_all_catches_a_gradient_mistake():
    case = _scan_case()
    ok, report = verify_all(case, lambda inputs, params: _DoubledGrad.apply(inputs["X"]),
                            device="cpu")
    assert not ok
    assert "[forward] PASS" in report and "[backward] FAIL" in report


def test_loader_refuses_a_stale_library(tmp_path, monkeypatch):
    """A library whose recorded fingerprint differs from its current sources
    is refused (the GPU box must never run code other than the committed
    source); NL2K_ALLOW_STALE=1 loads it anyway, with a warning."""
    import pytest
    from framework import loader
    src = tmp_path / "k.hip"
    src.write_text("extern \"C\" int f(void) { return 1; }\n")
    lib = tmp_path / "libk.so"
    lib.write_bytes(b"not a library")
    (tmp_path / "libk.so.stamp").write_text(loader._fingerprint([str(src)], loader._flags(None, None)))
    assert not loader.is_stale("k", ["k.hip"], str(tmp_path))
    src.write_text("extern \"C\" int f(void) { return 2; }\n")  # source changed after the build
    assert loader.is_stale("k", ["k.hip"], str(tmp_path))
    monkeypatch.delenv("NL2K_ALLOW_STALE", raising=False)
    with pytest.raises(RuntimeError, match="other sources or flags"):
        loader.load_library("k", ["k.hip"], str(tmp_path))
    monkeypatch.setenv("NL2K_ALLOW_STALE", "1")
    with pytest.raises(OSError):  # gets as far as dlopen of the (fake) file
        loader.load_library("k", ["k.hip"], str(tmp_path))


def test_loader_builds_and_loads_a_tiny_library(tmp_path, monkeypatch):
    """hipcc cross-compiles for gfx950 without a GPU; the host side of the
    library is callable here, and the build stamp makes it fresh."""
    from framework import loader
    src = tmp_path / "t.hip"
    src.write_text('extern "C" int nl2k_answer(int x) { return 2 * x + 1; }\n')
    path = loader.build_library("t", ["t.hip"], str(tmp_path))
    assert path.endswith("libt.so") and not loader.is_stale("t", ["t.hip"], str(tmp_path))
    monkeypatch.delenv("NL2K_ALLOW_STALE", raising=False)
    lib = loader.load_library("t", ["t.hip"], str(tmp_path))
    assert lib.nl2k_answer(20) == 41


def test_loader_reports_build_failures(tmp_path):
    """A source that does not compile, or a missing one, raises with the
    compiler's message instead of leaving a library behind."""
    import pytest
    from framework import loader
    (tmp_path / "bad.hip").write_text('extern "C" int f(void) { return undefined_name; }\n')
    with pytest.raises(RuntimeError, match="hipcc failed for libbad.so"):
        loader.build_library("bad", ["bad.hip"], str(tmp_path))
    assert not (tmp_path / "libbad.so").exists()
    with pytest.raises(FileNotFoundError, match="source file not found"):
        loader.build_library("gone", ["gone.hip"], str(tmp_path))
