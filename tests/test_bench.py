"""bench.py's host-side bookkeeping, without a GPU: the step statistics,
the per-config entry (GB/s, roofline fraction, committed traffic), and the
error summary every config reports against the float64 oracle."""

import math

import numpy as np
import pytest

import bench


def test_repeat_stats_is_a_geomean_with_the_cv_of_the_chunk_geomeans():
    samples = [1.0, 1.0, 4.0, 4.0, 16.0, 16.0]
    gm, cv = bench.repeat_stats(samples)
    assert gm == pytest.approx(4.0)
    chunks = [1.0, 4.0, 16.0]  # geomeans of the three chunks
    mean = sum(chunks) / 3
    sd = math.sqrt(sum((c - mean) ** 2 for c in chunks) / 3)
    assert cv == pytest.approx(sd / mean)
    assert bench.repeat_stats([5.0, 5.0, 5.0])[1] == 0.0


def test_entry_prices_hbm_and_mfma_roofs():
    e = bench._entry("x", "call", [10.0] * 3, 80_000_000)
    assert e["gbs"] == pytest.approx(8000.0)  # 80 MB in 10 us
    assert e["roofline"] == {"bound": "hbm", "frac": 1.0}
    e = bench._entry("x", "call", [20.0] * 3, 1, flops=1.573e9, bound="mfma")
    assert e["tflops"] == pytest.approx(78.65)
    assert e["roofline"]["frac"] == pytest.approx(0.5)
    assert "traffic" not in e


def test_entries_with_a_traffic_profile_carry_it():
    """The layernorm forward entry picks up profiles/layernorm_fwd_8192x4096_
    traffic.json (measured HBM bytes per launch over the algorithmic bytes)."""
    algo = 268_533_760
    e = bench._entry("layernorm [8192,4096]", "forward", [47.0] * 3, algo)
    t = e["traffic"]
    assert t["source"] == "profiles/layernorm_fwd_8192x4096_traffic.json"
    assert t["hbm_bytes"] > algo * 0.95
    assert t["over_algorithmic"] == pytest.approx(t["hbm_bytes"] / algo, abs=1e-3)
    # RBF at 4096 has profiles; other sizes and unprofiled calls do not
    assert "traffic" in bench._entry("rbf N=M=4096 D=64", "backward", [50.0], 138_412_032)
    assert "traffic" not in bench._entry("rbf N=M=8192 D=64", "backward", [50.0], 1)
    assert "traffic" not in bench._entry("spmv zipf 2^20", "backward dvals + dX", [50.0], 1)


def test_errors_use_relative_error_only_above_atol():
    ref = np.array([1.0, 1e-6, -2.0])
    got = np.array([1.0005, 5e-4, -2.0])
    e = bench.errors(got, ref)
    assert e["max_abs"] == pytest.approx(5e-4, rel=1e-6)
    assert e["max_rel"] == pytest.approx(5e-4, rel=1e-6)  # the 1e-6 entry is not a relative error
    assert e["allclose"]
    assert not bench.errors(np.array([1.01]), np.array([1.0]))["allclose"]
    acc = {}
    bench.merge_errors(acc, {"K": e})
    bench.merge_errors(acc, {"K": {"max_abs": 1.0, "max_rel": 0.1, "allclose": False}})
    assert acc["K"] == {"max_abs": 1.0, "max_rel": 0.1, "allclose": False}


def test_until_stable_retries_while_the_rounds_spread_and_keeps_the_steadiest():
    from framework.bench import spread, until_stable
    assert spread([2.0, 2.0]) == 0.0
    assert abs(spread([1.0, 3.0]) - 0.5) < 1e-12
    # Two noisy measurements (round geomeans 1, 2, 1 and 1, 1.2, 1), then a
    # steady one: three tries, the steady result kept.
    rounds = iter([[1.0], [2.0], [1.0], [1.0], [1.2], [1.0], [4.0], [4.0], [4.1]])
    t = until_stable("forward", lambda: next(rounds), rounds=3, cv_limit=0.05, retries=4)
    assert t.stable and t.tries == 3
    assert t.rounds_ms == [4.0, 4.0, 4.1]
    assert abs(t.center_ms - (4.0 * 4.0 * 4.1) ** (1 / 3)) < 1e-12


def test_until_stable_gives_up_after_the_retries_with_the_lowest_spread():
    from framework.bench import until_stable
    noisy = [[1.0], [3.0], [1.0], [1.0], [1.5], [1.0], [1.0], [4.0], [1.0]]
    rounds = iter(noisy)
    t = until_stable("backward", lambda: next(rounds), rounds=3, cv_limit=0.05, retries=2)
    assert not t.stable and t.tries == 3
    assert t.rounds_ms == [1.0, 1.5, 1.0]  # the second try spread least
    # one round's per-iteration times enter as their geometric mean
    t = until_stable("forward", lambda: [1.0, 4.0], rounds=2, cv_limit=0.05, retries=0)
    assert t.stable and abs(t.center_ms - 2.0) < 1e-12
