"""The standalone delivery (cases/rbf/delivery): its self-test binary, built by
__graft_entry__.build() with the Makefile (hipcc, ARCH=gfx950), runs the
host-pointer entry points of librbf.a against its own float64 CPU
evaluation at atol = rtol = 1e-3 and exits 0 only when every check passes."""

import os
import subprocess

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(REPO, "nl2cuda-kernel-agent_amd", "cases", "rbf", "delivery", "rbf_test")


@pytest.mark.parametrize("args", [[], ["300", "257", "64", "0.5"], ["100", "70", "33"],
                                  ["1", "1", "1"], ["512", "640", "64", "0.015625"]])
def test_delivery_self_test(args):
    if not os.path.exists(BINARY):
        pytest.fail("delivery self-test not built (run __graft_entry__.build())")
    announce(f"delivery rbf_test {' '.join(args) or '(defaults)'}")
    r = subprocess.run([BINARY] + args, capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "overall: PASS" in r.stdout
