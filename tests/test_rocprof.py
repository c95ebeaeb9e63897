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
    # every committed traffic summary yields a positive byte count for its workload
    files = sorted(rocprof.PROFILES.glob("*_traffic.md"))
    assert files, "no traffic summaries under profiles/"
    for f in files:
        workload = next(w for w in ("cfg1_decode_bf16", "cfg2_prefill_bf16", "cfg3_fp8", "cfg4_skewed_bf16")
                        if f.name.endswith(f"_{w}_traffic.md"))
        assert rocprof.traffic_for(workload) > 0
    assert rocprof.traffic_for("no_such_workload") is None
