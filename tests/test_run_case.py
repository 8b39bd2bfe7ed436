"""The case runner CLI (framework/run_case.py): the no-GPU refusal on the
CPU; on the GPU the verify-gated bench at a small cosine_sim size with the
eager baseline, which must print the parity report and one VERDICT line in
the reference's grammar (skill/scripts/bench_case.py:33-54), and the
reference's own headline measurement: ``run_case run --case rbf`` at the
reference defaults (RBF_SIZE = 2048, D = 64, gamma = 1/64, X, Y ~ N(0,1)),
parity first, then the candidate against ``torch.compile(reference_forward)``
(the reference's default baseline, framework/bench.py:129-178) with the
VERDICT line the reference publishes against (fwd 1.10x / bwd 1.17x on
A100, cases/rbf/delivery/README.md:56-57)."""

import re

import pytest
import torch

from framework import run_case


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the CPU-only refusal")
def test_refuses_without_gpu(capsys):
    assert run_case.main(["verify", "--case", "rbf"]) == 2
    assert "needs an MI355X GPU" in capsys.readouterr().err


def test_verdict_grammar_from_a_report():
    from framework.bench import parse_verdict
    report = ("  forward : 3.2100x  (target >=1.05x) PASS\n"
              "  backward: 1.0100x  (target >=1.05x) FAIL\n")
    assert parse_verdict(report, False) == "VERDICT=BENCH_FAIL fwd=3.2100x bwd=1.0100x cv_ok=1"
    assert parse_verdict(report + "  CV > 5% present: result invalid, re-measure\n",
                         False).startswith("VERDICT=CV_INVALID")


@pytest.mark.gpu
def test_run_gates_bench_on_verify(capsys, monkeypatch):
    from conftest import announce
    from cases.cosine_sim import make_case
    announce("run_case run --case cosine_sim (512 x 512, eager baseline)")
    monkeypatch.setattr(run_case, "load_case", lambda name: make_case(512, 512, 64))
    rc = run_case.main(["run", "--case", "cosine_sim", "--baseline", "eager"])
    out = capsys.readouterr().out
    print(out)
    assert rc == 0
    assert "=== overall: PASS ===" in out
    assert re.search(r"^VERDICT=(PASS|BENCH_FAIL|CV_INVALID) fwd=[0-9.]+x bwd=[0-9.]+x cv_ok=[01]$",
                     out, re.M)


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_rbf_reference_verdict_against_torch_compile(capsys):
    from conftest import announce
    from cases.rbf import config
    announce(f"run_case run --case rbf --emit-verdict (N=M={config.N}, torch.compile baseline)")
    assert config.N == config.M == 2048 and config.D == 64
    rc = run_case.main(["run", "--case", "rbf", "--emit-verdict"])
    out = capsys.readouterr().out
    print(out)
    assert rc == 0
    assert "=== overall: PASS ===" in out
    assert "[baseline(torch.compile)]" in out
    m = re.search(r"^VERDICT=(PASS|BENCH_FAIL|CV_INVALID) fwd=([0-9.]+)x bwd=([0-9.]+)x "
                  r"cv_ok=([01])$", out, re.M)
    assert m, "no VERDICT line"
    print(f"[verdict] {m.group(0)}", flush=True)
