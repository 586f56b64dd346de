"""bench.py's parsers of rocprofv3 output (CPU): the counter pass that gives
`roofline.traffic`, `traffic_by_stage` and `clock_GHz`, and the marked
kernel trace that gives the dominant kernels' durations.  Synthetic CSV files
in rocprofv3's column layout."""
import csv

import pytest

import bench

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
G2 = "void moe::(anonymous namespace)::gemm2_tiled_kernel<2, 4, 2, 4, 2>(unsigned short const*, float*)"
G1 = "moe::(anonymous namespace)::gemm1_wide_kernel(unsigned char const*, float const*, int)"
ROUTE = "void moe::(anonymous namespace)::route_kernel<16, false>(float const*)"
PERM = "void moe::(anonymous namespace)::perm_kernel<4>(int const*)"
COPY = "__amd_rocclr_copyBuffer"


def _write(tmp_path, rows):
    f = tmp_path / "pmc_counter_collection.csv"
    with open(f, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(FIELDS, r)))
    return [str(f)]


def test_pmc_scale_means_and_clock(tmp_path):
    us = 1000  # ns
    rows = [
        # an early small copy, then the 1 GiB calibration copy (the last copy counts)
        (1, COPY, "FETCH_SIZE", 4096, 0, 10 * us),
        (9, COPY, "FETCH_SIZE", 524288, 0, 200 * us),
        # GEMM2: two dispatches, FETCH 100 and 300 KiB (mean 200), 200 us at 1.6 GHz
        (3, G2, "FETCH_SIZE", 100, 0, 200 * us),
        (3, G2, "GRBM_GUI_ACTIVE", 8 * 1.6 * 200 * us, 0, 200 * us),
        (6, G2, "FETCH_SIZE", 300, 0, 200 * us),
        (6, G2, "GRBM_GUI_ACTIVE", 8 * 1.6 * 200 * us, 0, 200 * us),
        # GEMM1 at 1.8 GHz
        (2, G1, "FETCH_SIZE", 50, 0, 150 * us),
        (2, G1, "GRBM_GUI_ACTIVE", 8 * 1.8 * 150 * us, 0, 150 * us),
        # route + perm form one stage; short dispatches get no clock
        (0, ROUTE, "FETCH_SIZE", 10, 0, 12 * us),
        (0, ROUTE, "GRBM_GUI_ACTIVE", 8 * 5.0 * 12 * us, 0, 12 * us),
        (1, PERM, "FETCH_SIZE", 2, 0, 6 * us),
    ]
    per_stage, clocks = bench.parse_pmc(_write(tmp_path, rows), "FETCH_SIZE")
    scale = 1024 * 1048576 / 524288  # bytes per KiB, times 2: the copy read 512 MiB worth of counts
    assert per_stage["gemm2"] == pytest.approx(200 * scale)
    assert per_stage["gemm1_swiglu"] == pytest.approx(50 * scale)
    assert per_stage["route"] == pytest.approx((10 + 2) * scale)
    assert clocks == {"gemm2": pytest.approx(1.6), "gemm1_swiglu": pytest.approx(1.8)}


def test_pmc_other_counters_ignored_and_calibration_required(tmp_path):
    rows = [
        (9, COPY, "WRITE_SIZE", 1048576, 0, 100),
        (3, G2, "WRITE_SIZE", 2048, 0, 100),
        (3, G2, "FETCH_SIZE", 999999, 0, 100),  # a row of another counter
    ]
    per_stage, clocks = bench.parse_pmc(_write(tmp_path, rows), "WRITE_SIZE")
    assert per_stage == {"gemm2": pytest.approx(2048 * 1024.0)}
    assert clocks == {}
    no_copy = [(3, G2, "FETCH_SIZE", 100, 0, 100)]
    assert bench.parse_pmc(_write(tmp_path, no_copy), "FETCH_SIZE") is None


def test_split_trace_spans_per_workload():
    rows = [
        (0, "trace_mark_begin()", 1),
        (1, ROUTE, 4000), (2, G1, 100000), (3, G2, 200000),
        (4, ROUTE, 6000), (5, G1, 120000), (6, G2, 220000),
        (7, "trace_mark_end()", 1),
        (8, G2, 999999999),  # between spans: not counted
        (9, "trace_mark_begin()", 1),
        (10, PERM, 3000), (11, ROUTE, 5000),
        (12, PERM, 5000), (13, ROUTE, 7000),
        (14, "trace_mark_end()", 1),
    ]
    out, err = bench.split_trace(rows[::-1], ["skewed_t8192", "small_t64"], 2)  # any row order
    assert err is None
    a, b = out["skewed_t8192"], out["small_t64"]
    assert a["calls"] == 2
    assert a["stage_us"] == {"route": 5.0, "gemm1_swiglu": 110.0, "gemm2": 210.0}
    assert a["kernel_us"]["gemm2_tiled_kernel<2, 4, 2, 4, 2>"] == 210.0
    assert b["stage_us"] == {"route": 10.0}  # route + perm per call
    assert b["kernel_us"] == {"perm_kernel<4>": 4.0, "route_kernel<16, false>": 6.0}


def test_split_trace_needs_one_span_per_workload():
    rows = [(0, "trace_mark_begin()", 1), (1, G2, 10), (2, "trace_mark_end()", 1)]
    out, err = bench.split_trace(rows, ["a", "b"], 1)
    assert out is None and "1 workload spans, expected 2" in err
