"""flide_amd.rocprof: per-dispatch counter parsing, copy-kernel scaling, and the committed traffic figures
that bench.py reports (CPU only)."""
from __future__ import annotations

import csv

from flide_amd import rocprof

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(FIELDS, r)))
    return str(path)


def test_traffic_scales_by_copy_kernel(tmp_path):
    # kernel: FETCH 3000 units (median of 1000/3000/5000), WRITE 10 units; copy: 1 GiB read as 524288 FETCH
    # units (2048 B each) and 1048576 WRITE units (1024 B each)
    fk = _write(tmp_path / "f.csv", [(1, "gemm_kernel", "FETCH_SIZE", 1000), (2, "gemm_kernel", "FETCH_SIZE", 3000),
                                     (3, "gemm_kernel", "FETCH_SIZE", 5000), (4, "other", "FETCH_SIZE", 9e9)])
    wk = _write(tmp_path / "w.csv", [(1, "gemm_kernel", "WRITE_SIZE", 10)])
    fc = _write(tmp_path / "fc.csv", [(1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 524288)])
    wc = _write(tmp_path / "wc.csv", [(1, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 1048576)])
    md = rocprof.traffic_md("cfgX", "gemm", fk, wk, fc, wc, "cmd")
    assert "traffic_bytes_per_dispatch: %d" % (3000 * 2048 + 10 * 1024) in md
    assert "| dispatches (FETCH / WRITE pass) | 3 / 1 |" in md


def test_per_dispatch_sums_counter_instances(tmp_path):
    p = _write(tmp_path / "x.csv", [(7, "k", "FETCH_SIZE", 1.5), (7, "k", "FETCH_SIZE", 2.5), (8, "k", "FETCH_SIZE", 1)])
    assert sorted(rocprof.per_dispatch(p, "k", "FETCH_SIZE")) == [1.0, 4.0]


def test_committed_traffic_figures_parse():
    # both products at every GPU workload have a committed summary with a positive byte count
    for w in ("cfg1_decode_bf16", "cfg2_prefill_bf16", "cfg3_fp8", "cfg4_skewed_bf16"):
        for kernel in ("gate_up", "down"):
            assert rocprof.traffic_for(w, kernel) > 0, (w, kernel)
    assert rocprof.traffic_for("no_such_workload") is None


def _write_mfma(path, rows):
    fields = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(fields, r)))
    return str(path)


def test_mfma_summary(tmp_path):
    # one dispatch of 1 ms: 8 XCDs x 2e6 cycles (2 GHz), MFMA busy on a quarter of the 1024 SIMDs' cycles,
    # 1e9 bf16 MOPS (5.12e11 FLOP) for 5e11 algorithmic FLOP
    p = _write_mfma(tmp_path / "m.csv", [
        (1, "gemm", "GRBM_GUI_ACTIVE", 8 * 2e6, 0, 1_000_000),
        (1, "gemm", "SQ_VALU_MFMA_BUSY_CYCLES", 0.25 * 2e6 * 1024, 0, 1_000_000),
        (1, "gemm", "SQ_INSTS_VALU_MFMA_MOPS_BF16", 1e9, 0, 1_000_000),
        (1, "other", "GRBM_GUI_ACTIVE", 1, 0, 5)])
    md = rocprof.mfma_md(p, "gemm", 5e11, 2.5e15, "t", "cmd")
    assert "mfma_busy: 0.2500" in md and "sclk_ghz: 2.000" in md
    assert "executed / algorithmic = 1.02" in md and "500.0 TFLOP/s = 20.0% of 2500" in md
