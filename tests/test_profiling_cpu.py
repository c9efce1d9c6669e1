"""The rocprofv3 summaries behind the committed profiles: kernel-name shortening, the HBM
traffic calibration and the utilisation report, on small hand-made CSV files."""
import csv
import os

import pytest

from tiktok_techjam_2026_track3_amd import profiling as P

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp",
          "End_Timestamp"]
ATTN = "_ZN12_GLOBAL__N_113attn_fwd_mfmaIDF16_Li64ELi4ELi2ELi2ELi2ELb0ELb0ELb0ELb0EEEvNS_8AttnArgsE"
REDO = "_ZN12_GLOBAL__N_113attn_fwd_mfmaIDF16_Li64ELi4ELi2ELi2ELi2ELb0ELb0ELb0ELb0ELb1EEEvNS_8AttnArgsE"
BOUND = "_ZN12_GLOBAL__N_114attn_key_boundIDF16_Li64EEEvNS_8AttnArgsEPf"
COPY = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda(...)>"


def _write(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(FIELDS, r)))


def test_short_name_reads_mangled_template_arguments():
    assert P.short_name(ATTN) == "attn_fwd_mfma<f16,64,4,2,2,2,0,0,0,0>"
    assert P.short_name(COPY) == "torch vectorized_elementwise_kernel"


def test_counters_sum_dimensions_and_keep_durations(tmp_path):
    # one dispatch whose counter arrives as two dimension instances (e.g. two XCDs)
    _write(tmp_path / "a", [(1, ATTN, "GRBM_GUI_ACTIVE", 100, 1000, 3000),
                            (1, ATTN, "GRBM_GUI_ACTIVE", 140, 1000, 3000)])
    t = P.counters(str(tmp_path / "a"))
    assert t[ATTN]["GRBM_GUI_ACTIVE"] == [240.0]
    assert t[ATTN][P.DURATION] == [2000.0]


def test_utilisation_formulas(tmp_path):
    dur = 100_000.0                       # 100 us
    cyc = 200_000.0                       # 2.0 GHz
    simd_cycles = cyc * 1024
    pass1 = [(7, ATTN, "GRBM_GUI_ACTIVE", cyc * 8, 0, dur),
             (7, ATTN, "SQ_VALU_MFMA_BUSY_CYCLES", 0.5 * simd_cycles, 0, dur),
             (7, ATTN, "SQ_VALU_MFMA_COEXEC_CYCLES", 0.1 * simd_cycles, 0, dur),
             (7, ATTN, "SQ_ACTIVE_INST_VALU", 0.25 * simd_cycles / 4, 0, dur),
             (7, ATTN, "SQ_WAVE_CYCLES", 1000.0, 0, dur)]
    pass2 = [(7, ATTN, "GRBM_GUI_ACTIVE", cyc * 8, 0, dur),
             (7, ATTN, "SQ_INSTS_VALU_MFMA_MOPS_F16", 1e9 / 512, 0, dur),
             (7, ATTN, "SQ_WAIT_INST_ANY", 300.0, 0, dur)]
    _write(tmp_path / "p1", pass1)
    _write(tmp_path / "p2", pass2)
    (r,) = P.utilisation([str(tmp_path / "p1"), str(tmp_path / "p2")])
    assert r["cycles"] == pytest.approx(cyc)
    assert r["clock_ghz"] == pytest.approx(2.0)
    assert r["mfma_busy"] == pytest.approx(0.5)
    assert r["coexec"] == pytest.approx(0.2)
    assert r["valu_active"] == pytest.approx(0.25)
    assert r["mfma_ops"] == pytest.approx(1e9)
    assert r["mfma_tops"] == pytest.approx(1e9 / dur / 1e3)   # 10 TOP/s
    assert r["wait"] == pytest.approx(0.3)
    assert r["dispatches"] == 1


def test_traffic_scales_by_the_copy_calibration(tmp_path):
    n = 1 << 20
    # the copy kernel reads and writes n bytes; its counters read half / all of that (KiB)
    _write(tmp_path / "cf", [(1, COPY, "FETCH_SIZE", n / 2 / 1024, 0, 1)])
    _write(tmp_path / "cw", [(1, COPY, "WRITE_SIZE", n / 1024, 0, 1)])
    _write(tmp_path / "kf", [(2, ATTN, "FETCH_SIZE", 300.0, 0, 1)])
    _write(tmp_path / "kw", [(2, ATTN, "WRITE_SIZE", 100.0, 0, 1)])
    rec = P.traffic("C2", "attn_fwd_mfma", str(tmp_path / "kf"), str(tmp_path / "kw"),
                    str(tmp_path / "cf"), str(tmp_path / "cw"), float(n))
    assert rec["copy_fetch_factor"] == pytest.approx(2.0)
    assert rec["copy_write_factor"] == pytest.approx(1.0)
    assert rec["fetch_bytes"] == pytest.approx(300.0 * 1024 * 2)
    assert rec["write_bytes"] == pytest.approx(100.0 * 1024)
    assert rec["bytes_per_launch"] == pytest.approx(300.0 * 1024 * 2 + 100.0 * 1024)


def test_traffic_sums_the_stage_kernels_per_call(tmp_path):
    """A stage of several launches (sweep, redo, bound pass): each kernel's mean per dispatch,
    summed -- two calls of three launches give the bytes of one call, not the mean of six."""
    n = 1 << 20
    _write(tmp_path / "cf", [(1, COPY, "FETCH_SIZE", n / 1024, 0, 1)])
    _write(tmp_path / "cw", [(1, COPY, "WRITE_SIZE", n / 1024, 0, 1)])
    _write(tmp_path / "kf", [(2, ATTN, "FETCH_SIZE", 1000.0, 0, 1), (3, REDO, "FETCH_SIZE", 2.0, 0, 1),
                             (4, BOUND, "FETCH_SIZE", 50.0, 0, 1), (5, ATTN, "FETCH_SIZE", 1200.0, 0, 1),
                             (6, REDO, "FETCH_SIZE", 4.0, 0, 1), (7, BOUND, "FETCH_SIZE", 50.0, 0, 1)])
    _write(tmp_path / "kw", [(2, ATTN, "WRITE_SIZE", 100.0, 0, 1), (3, REDO, "WRITE_SIZE", 0.0, 0, 1),
                             (4, BOUND, "WRITE_SIZE", 1.0, 0, 1)])
    rec = P.traffic("C5", "attn_fwd_mfma|attn_key_bound", str(tmp_path / "kf"), str(tmp_path / "kw"),
                    str(tmp_path / "cf"), str(tmp_path / "cw"), float(n))
    assert rec["stage"] == "attn"
    assert sorted(rec["kernels"]) == sorted(P.short_name(k) for k in (ATTN, REDO, BOUND))
    assert P.short_name(BOUND) == "attn_key_bound<f16,64>"
    assert rec["fetch_bytes"] == pytest.approx((1100.0 + 3.0 + 50.0) * 1024)
    assert rec["write_bytes"] == pytest.approx((100.0 + 0.0 + 1.0) * 1024)


def test_bench_matches_traffic_records_by_kernel_family(tmp_path, monkeypatch):
    """bench.py attaches a traffic record only when every kernel it summed belongs to the
    stage's kernel family on this build (the matrix-core attention and its bound pass, or the
    vector-ALU kernel), never by a name prefix shared between families."""
    import json
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    f = tmp_path / "traffic.json"
    f.write_text(json.dumps({
        "C2": {"stage": "attn", "bytes_per_launch": 5.0,
               "kernels": {"attn_fwd_mfma<f16,64,4,2,2,2,0,0,0,0,0>": {}, "attn_key_bound<f16,64>": {}}},
        "C1": {"stage": "attn", "bytes_per_launch": 7.0, "kernels": {"attn_fwd_f32<64>": {}}},
        "C3": {"stage": "qkv", "bytes_per_launch": 9.0, "kernels": {"gemm_kernel<bf16>": {}}}}))
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(f))
    mfma = ("attn_fwd_mfma", "attn_key_bound")
    assert bench.measured_traffic("C2", "attn", mfma) == 5.0
    assert bench.measured_traffic("C2", "attn", ("attn_fwd_valu",)) is None
    assert bench.measured_traffic("C1", "attn", mfma) is None        # another family's record
    assert bench.measured_traffic("C3", "attn", mfma) is None        # another stage's record
    assert bench.measured_traffic("C4", "attn", mfma) is None        # no record
