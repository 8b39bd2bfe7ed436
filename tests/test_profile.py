"""The rocprofv3 summary tool on the CPU (framework/profile.py), fed small
hand-written files in rocprofv3's CSV layout: the kernel-statistics table,
per-dispatch PMC sums over the per-instance rows, the copy calibration that
turns FETCH_SIZE / WRITE_SIZE readings into bytes, and the MFMA counters.
(The reference's skill/scripts/profile_case.py:34-83 prints torch.profiler's
table; this tool reads rocprofv3's files instead.)"""

import csv
import os

import pytest

from framework import profile

COUNTER_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id",
                  "Thread_Id", "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size",
                  "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count",
                  "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp",
                  "End_Timestamp"]
STATS_HEADER = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs",
                "StdDev"]
COPY = "__amd_rocclr_copyBuffer"
REDUCE = "void (anonymous namespace)::rbf_bwd_reduce_kernel(float const*, float*, int)"
TILE = "void nl2k::pair_bwd_d64_3r_kernel<RbfBwdOp, 4, true>(float const*, float*)"


def _write_counters(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(COUNTER_HEADER)
        for disp, name, counter, value in rows:
            w.writerow([disp, disp, "Agent 1", 1, 100, 100, 65536, 7, name, 256, 0, 0, 64, 0, 32,
                        counter, float(value), 1000 * disp, 1000 * disp + 500])


def test_stats_table_reads_rocprof_kernel_stats(tmp_path):
    d = tmp_path / "stats"
    d.mkdir()
    with open(d / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(STATS_HEADER)
        w.writerow([TILE, 20, 1088000, 54400.0, 88.7, 53900, 55100, 300.0])
        w.writerow([REDUCE, 20, 138800, 6940.0, 11.3, 6800, 7100, 80.0])
    table = profile.stats_table(str(tmp_path))
    assert [r["calls"] for r in table] == [20, 20]
    assert table[0]["avg_us"] == pytest.approx(54.4)
    assert table[1]["min_us"] == pytest.approx(6.8) and table[1]["max_us"] == pytest.approx(7.1)
    # argument lists and the anonymous namespace are cut from the names
    assert table[1]["kernel"] == "void rbf_bwd_reduce_kernel"
    assert table[0]["kernel"] == "void nl2k::pair_bwd_d64_3r_kernel<RbfBwdOp, 4, true>"


def test_counter_rows_sum_instances_per_dispatch(tmp_path):
    path = tmp_path / "p" / "run_counter_collection.csv"
    _write_counters(str(path), [(1, TILE, "FETCH_SIZE", 1000.0), (1, TILE, "FETCH_SIZE", 500.0),
                                (2, TILE, "FETCH_SIZE", 1400.0), (2, REDUCE, "WRITE_SIZE", 7.0)])
    rows = profile.counter_rows(str(tmp_path / "p"))
    assert len(rows) == 4 and rows[0] == (1, TILE, "FETCH_SIZE", 1000.0)
    vals, names = profile.per_dispatch(rows, "FETCH_SIZE", ["pair_bwd"])
    assert vals == {1: 1500.0, 2: 1400.0} and names[1] == TILE
    assert profile.per_dispatch(rows, "WRITE_SIZE", ["pair_bwd"])[0] == {}


def test_traffic_calibration_against_a_copy_of_known_size():
    """The copy moves 256 MiB per launch: its median per-dispatch reading
    fixes the bytes per counter unit (gfx950: FETCH_SIZE reads about 128 KiB
    per 256 MiB read, i.e. 2048 B per unit; WRITE_SIZE is in KiB), and each
    kernel's median per-dispatch reading times that factor is its bytes per
    launch."""
    copy_rows = []
    for disp, total in ((1, 131084), (2, 131084), (3, 140000)):  # one outlier dispatch
        copy_rows += [(disp, COPY, "FETCH_SIZE", total // 2), (disp, COPY, "FETCH_SIZE",
                                                               total - total // 2)]
    krows = [(10, TILE, "FETCH_SIZE", 70000.0), (11, TILE, "FETCH_SIZE", 70264.0),
             (12, TILE, "FETCH_SIZE", 90000.0), (10, REDUCE, "FETCH_SIZE", 1.0),
             (13, REDUCE, "FETCH_SIZE", 17900.0), (14, REDUCE, "FETCH_SIZE", 17950.0)]
    res = profile.calibrated_counter(krows, copy_rows, "FETCH_SIZE",
                                     ["pair_bwd_d64_3r", "rbf_bwd_reduce"])
    factor = (256 << 20) / 131084
    assert res["copy_counter_median"] == 131084 and res["copy_dispatches"] == 3
    assert res["bytes_per_unit"] == pytest.approx(factor)
    tile = res["kernels"]["pair_bwd_d64_3r"]
    assert tile["dispatches"] == 3 and tile["median_counter"] == 70264.0
    assert tile["bytes_per_launch"] == pytest.approx(70264.0 * factor)
    red = res["kernels"]["rbf_bwd_reduce"]
    assert red["median_counter"] == 17900.0  # median of {1, 17900, 17950}
    # WRITE_SIZE: the copy writes 256 MiB = 262144 KiB
    wres = profile.calibrated_counter([(5, TILE, "WRITE_SIZE", 33000.0)],
                                      [(1, COPY, "WRITE_SIZE", 262144.0)], "WRITE_SIZE",
                                      ["pair_bwd"])
    assert wres["bytes_per_unit"] == pytest.approx(1024.0)
    assert wres["kernels"]["pair_bwd"]["bytes_per_launch"] == pytest.approx(33000.0 * 1024)


def test_traffic_calibration_refuses_missing_readings():
    with pytest.raises(RuntimeError, match="copy"):
        profile.calibrated_counter([(1, TILE, "FETCH_SIZE", 1.0)], [], "FETCH_SIZE", ["pair"])
    with pytest.raises(RuntimeError, match="no FETCH_SIZE readings"):
        profile.calibrated_counter([], [(1, COPY, "FETCH_SIZE", 1.0)], "FETCH_SIZE", ["pair"])


def test_mfma_summary_per_kernel():
    rows = []
    for disp, util, flops in ((1, 46.0, 4294967296.0), (2, 47.5, 4294967296.0),
                              (3, 45.1, 4294967296.0)):
        rows += [(disp, TILE, "MfmaUtil", util), (disp, TILE, "MfmaFlopsF32", flops)]
    rows += [(4, REDUCE, "MfmaUtil", 0.0), (4, REDUCE, "MfmaFlopsF32", 0.0)]
    s = profile.mfma_summary(rows, ["pair_bwd", "rbf_bwd_reduce"])
    u = s["pair_bwd"]["MfmaUtil"]
    assert (u["median"], u["min"], u["max"], u["dispatches"]) == (46.0, 45.1, 47.5, 3)
    assert s["pair_bwd"]["MfmaFlopsF32"]["median"] == 4294967296.0  # 4 N M D at N = M = 4096
    assert s["rbf_bwd_reduce"]["MfmaUtil"]["median"] == 0.0
    with pytest.raises(RuntimeError, match="no MfmaUtil"):
        profile.mfma_summary(rows, ["not_there"])


def test_kernel_list_separators():
    assert profile.kernel_list("rn_bwd_kernel,rn_colsum_kernel") == ["rn_bwd_kernel",
                                                                    "rn_colsum_kernel"]
    assert profile.kernel_list("scan_rows_kernel<float, float, double, false;x") == [
        "scan_rows_kernel<float, float, double, false", "x"]


def test_counter_summary_medians_and_missing_counters():
    rows = [(1, TILE, "TCC_REQ_sum", 10.0), (1, TILE, "TCC_REQ_sum", 5.0),
            (2, TILE, "TCC_REQ_sum", 20.0), (3, TILE, "TCC_REQ_sum", 30.0),
            (1, TILE, "TCC_HIT_sum", 7.0), (4, REDUCE, "TCC_REQ_sum", 2.0)]
    s = profile.counter_summary(rows, ["pair_bwd", "rbf_bwd_reduce"],
                                ["TCC_REQ_sum", "TCC_HIT_sum", "TCC_MISS_sum"])
    assert s["pair_bwd"]["TCC_REQ_sum"] == {"dispatches": 3, "median": 20.0}  # {15, 20, 30}
    assert s["pair_bwd"]["TCC_HIT_sum"]["median"] == 7.0
    assert "TCC_MISS_sum" not in s["pair_bwd"]
    assert s["rbf_bwd_reduce"] == {"TCC_REQ_sum": {"dispatches": 1, "median": 2.0}}


def test_sequence_gaps_pairs_durations_and_gaps():
    from framework.profile import sequence_gaps
    rows = [(0, 100_000, "reduce_kernel<512"), (105_000, 135_000, "pair_fwd_d64"),
            (140_000, 190_000, "pair_bwd_d64_3r"), (190_000, 197_000, "rbf_bwd_reduce"),
            (300_000, 400_000, "reduce_kernel<512"), (406_000, 437_000, "pair_fwd_d64"),
            (443_000, 492_000, "pair_bwd_d64_3r"), (492_500, 499_000, "rbf_bwd_reduce"),
            (600_000, 700_000, "other")]
    g = sequence_gaps(rows, ["reduce_kernel<512", "pair_fwd", "pair_bwd", "rbf_bwd_reduce"])
    assert g["dur pair_fwd"] == [30.0, 31.0]
    assert g["gap reduce_kernel<512 -> pair_fwd"] == [5.0, 6.0]
    assert g["gap pair_fwd -> pair_bwd"] == [5.0, 6.0]
    assert g["gap pair_bwd -> rbf_bwd_reduce"] == [0.0, 0.5]
    assert g["dur rbf_bwd_reduce"] == [7.0, 6.5]
    assert sequence_gaps(rows, ["pair_bwd", "pair_fwd"]) == {}
