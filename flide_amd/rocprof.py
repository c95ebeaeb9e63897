"""rocprofv3 helpers for this package's measurements.

    python -m flide_amd.rocprof copy                       # the calibration kernel (run under rocprofv3 --pmc)
    python -m flide_amd.rocprof stats  <kernel_stats.csv> <title> <command> > summary.md
    python -m flide_amd.rocprof traffic <workload> <kernel-regex> <fetch.csv> <write.csv> \\
                                         <copy_fetch.csv> <copy_write.csv> <command> > traffic.md
    python -m flide_amd.rocprof mfma <counters.csv> <kernel-regex> <flop-per-dispatch> <peak-flop/s> \\
                                      <title> <command> > mfma.md
    python -m flide_amd.rocprof pipe <kernel-regex> <title> <command> <pass1.csv> [<pass2.csv> ...] > pipe.md

`copy` runs a plain device-to-device copy of COPY_BYTES (the HIP runtime's copy kernel) a few times. Under
`rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` its counters give the scale from the counters'
units to bytes on this GPU: the copy reads and writes exactly COPY_BYTES per dispatch.

`traffic` takes the per-dispatch FETCH_SIZE / WRITE_SIZE of the kernels matching a regex (median over
their dispatches), scales each by the copy kernel's factor, and writes a markdown summary that ends in
one machine-readable line `traffic_bytes_per_dispatch: <int>`; bench.py reports that number as the
roofline's `traffic` for the same workload.
"""
from __future__ import annotations

import csv
import re
import statistics
import sys
from pathlib import Path

COPY_BYTES = 1 << 30
PROFILES = Path(__file__).resolve().parent.parent / "profiles"


def copy_probe(reps: int = 5) -> None:
    import torch

    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {COPY_BYTES} bytes x {reps}", flush=True)


def _counter_rows(path: str) -> list[dict]:
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _kernel_name(row: dict) -> str:
    return row.get("Kernel_Name") or row.get("Kernel-Name") or row.get("KernelName") or ""


def per_dispatch(path: str, regex: str, counter: str) -> list[float]:
    """Counter value of every dispatch whose kernel name matches `regex` (summed over the counter's
    instances when a dispatch has several rows)."""
    pat = re.compile(regex)
    by_dispatch: dict[str, float] = {}
    for r in _counter_rows(path):
        if r.get("Counter_Name") != counter or not pat.search(_kernel_name(r)):
            continue
        key = r.get("Dispatch_Id") or r.get("Correlation_Id") or str(len(by_dispatch))
        by_dispatch[key] = by_dispatch.get(key, 0.0) + float(r["Counter_Value"])
    return list(by_dispatch.values())


def traffic_md(workload: str, regex: str, fetch: str, write: str, copy_fetch: str, copy_write: str,
               command: str) -> str:
    f_k = per_dispatch(fetch, regex, "FETCH_SIZE")
    w_k = per_dispatch(write, regex, "WRITE_SIZE")
    f_c = per_dispatch(copy_fetch, "copy", "FETCH_SIZE")
    w_c = per_dispatch(copy_write, "copy", "WRITE_SIZE")
    if not (f_k and w_k and f_c and w_c):
        raise SystemExit(f"no dispatches matched: kernel {len(f_k)}/{len(w_k)}, copy {len(f_c)}/{len(w_c)}")
    fk, wk, fc, wc = (statistics.median(v) for v in (f_k, w_k, f_c, w_c))
    rf, rw = COPY_BYTES / fc, COPY_BYTES / wc
    total = int(round(fk * rf + wk * rw))
    lines = [
        f"# HBM traffic per dispatch: {workload}",
        "",
        f"Kernels matching `{regex}`; counters from two rocprofv3 `--pmc` passes over the same command,",
        "scaled by what the same counters read for a plain 1 GiB device-to-device copy (the runtime's copy kernel).",
        "",
        "```",
        command,
        "```",
        "",
        "| quantity | value |",
        "|---|---|",
        f"| dispatches (FETCH / WRITE pass) | {len(f_k)} / {len(w_k)} |",
        f"| FETCH_SIZE median | {fk:.1f} |",
        f"| WRITE_SIZE median | {wk:.1f} |",
        f"| copy kernel FETCH_SIZE / WRITE_SIZE for {COPY_BYTES} B | {fc:.1f} / {wc:.1f} |",
        f"| scale: bytes per FETCH unit / per WRITE unit | {rf:.2f} / {rw:.2f} |",
        f"| HBM bytes read per dispatch | {fk * rf:.4g} |",
        f"| HBM bytes written per dispatch | {wk * rw:.4g} |",
        "",
        f"traffic_bytes_per_dispatch: {total}",
        "",
    ]
    return "\n".join(lines)


def stats_md(path: str, title: str, command: str, top: int = 12) -> str:
    rows = _counter_rows(path)
    rows.sort(key=lambda r: -float(r.get("TotalDurationNs", 0)))
    total = sum(float(r.get("TotalDurationNs", 0)) for r in rows) or 1.0
    out = [f"# {title}", "", "```", command, "```", "",
           "| kernel | calls | avg us | total ms | % |", "|---|---|---|---|---|"]
    for r in rows[:top]:
        name = re.sub(r"\(anonymous namespace\)::|grouped_detail::", "", r["Name"])
        name = name if len(name) <= 110 else name[:107] + "..."
        tot = float(r["TotalDurationNs"])
        out.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | {tot / 1e6:.3f} | "
                   f"{100 * tot / total:.1f} |")
    out.append("")
    return "\n".join(out)


MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                 "SQ_INSTS_VALU_MFMA_MOPS_F8", "GRBM_GUI_ACTIVE")
SIMDS, XCDS = 1024, 8   # MI355X: 256 CUs x 4 SIMDs, 8 XCDs


def _dispatches(path: str, regex: str) -> dict[str, dict]:
    """dispatch id -> {counter: value summed over the row's instances, "ns": kernel duration}."""
    pat = re.compile(regex)
    out: dict[str, dict] = {}
    for r in _counter_rows(path):
        if not pat.search(_kernel_name(r)):
            continue
        d = out.setdefault(r.get("Dispatch_Id") or r.get("Correlation_Id"), {})
        c = r["Counter_Name"]
        d[c] = d.get(c, 0.0) + float(r["Counter_Value"])
        d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    return out


def mfma_md(path: str, regex: str, flop: float, peak: float, title: str, command: str) -> str:
    """Matrix-core utilisation of the dispatches matching `regex`, medians over dispatches:
      clock        GRBM_GUI_ACTIVE / 8 XCDs / kernel duration (the counter sums the 8 XCDs' cycles)
      MFMA busy    SQ_VALU_MFMA_BUSY_CYCLES / (per-XCD GRBM_GUI_ACTIVE x 1024 SIMDs)
      MFMA FLOP    SQ_INSTS_VALU_MFMA_MOPS_{BF16,F8} x 512 (what the matrix cores executed, padding included)
    next to the launch's algorithmic FLOP (`flop`) over its duration against `peak`."""
    ds = list(_dispatches(path, regex).values())
    if not ds:
        raise SystemExit(f"no dispatches matched {regex}")
    med = lambda key: statistics.median(d.get(key, 0.0) for d in ds)   # noqa: E731
    ns = med("ns")
    gui = med("GRBM_GUI_ACTIVE") / XCDS
    busy = med("SQ_VALU_MFMA_BUSY_CYCLES")
    mops = med("SQ_INSTS_VALU_MFMA_MOPS_BF16") + med("SQ_INSTS_VALU_MFMA_MOPS_F8")
    clock = gui / ns   # GHz
    util = busy / (gui * SIMDS) if gui else 0.0
    lines = [
        f"# MFMA utilisation: {title}",
        "",
        f"Kernels matching `{regex}`; one rocprofv3 `--pmc` pass ({' '.join(MFMA_COUNTERS)}).",
        "",
        "```",
        command,
        "```",
        "",
        "| quantity | value |",
        "|---|---|",
        f"| dispatches | {len(ds)} |",
        f"| duration (median, under counter collection) | {ns / 1e3:.1f} us |",
        f"| GRBM_GUI_ACTIVE per XCD | {gui:.0f} cycles |",
        f"| shader clock during the kernel | {clock:.2f} GHz |",
        f"| SQ_VALU_MFMA_BUSY_CYCLES | {busy:.4g} |",
        f"| SQ_BUSY_CYCLES | {med('SQ_BUSY_CYCLES'):.4g} |",
        f"| **MFMA busy** (of all SIMD cycles) | **{100 * util:.1f}%** |",
        f"| MFMA FLOP executed (MOPS x 512) | {mops * 512:.4g} |",
        f"| algorithmic FLOP per dispatch | {flop:.4g} (executed / algorithmic = {mops * 512 / flop:.2f}) |",
        f"| algorithmic FLOP/s at this duration | {flop / ns / 1e3:.1f} TFLOP/s = {100 * flop / ns * 1e9 / peak:.1f}% "
        f"of {peak / 1e12:.0f} TFLOP/s |",
        f"| peak at the measured clock (x {clock:.2f} / 2.4 GHz) | {peak / 1e12 * clock / 2.4:.0f} TFLOP/s |",
        "",
        f"mfma_busy: {util:.4f}",
        f"sclk_ghz: {clock:.3f}",
        "",
    ]
    return "\n".join(lines)


PIPE_PASSES = (
    "SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_WAIT_INST_LDS SQ_ACTIVE_INST_LDS "
    "SQ_ACTIVE_INST_VALU SQ_INSTS_MFMA GRBM_GUI_ACTIVE",
    "SQ_INSTS_VMEM SQ_INSTS_LDS SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE",
    "TA_TA_BUSY TA_ADDR_STALLED_BY_TC_CYCLES TD_TD_BUSY TD_TC_STALL TCP_TCC_READ_REQ TCP_TCC_READ_REQ_LATENCY "
    "TCP_PENDING_STALL_CYCLES TCP_TOTAL_CACHE_ACCESSES GRBM_GUI_ACTIVE",
)
CUS = 256


def pipe_md(regex: str, title: str, command: str, paths: list[str]) -> str:
    """Where a kernel's time goes along the memory pipe, medians over the dispatches matching `regex`,
    from several --pmc passes of the same command. Unit-cycle counters are divided by the per-XCD
    GRBM_GUI_ACTIVE and the 256 CUs (a fraction of CU cycles); TCP_TCC_READ_REQ_LATENCY, the cycles
    L2 read requests spend outstanding, gives the average requests in flight per CU (Little's law) and,
    over TCP_TCC_READ_REQ, the average L2 read latency."""
    vals: dict[str, float] = {}
    for path in paths:
        ds = list(_dispatches(path, regex).values())
        if not ds:
            raise SystemExit(f"no dispatches matched {regex} in {path}")
        for key in ds[0]:
            vals.setdefault(key, statistics.median(d.get(key, 0.0) for d in ds))
    gui = vals["GRBM_GUI_ACTIVE"] / XCDS
    per_cu = lambda key: vals.get(key, 0.0) / CUS / gui   # noqa: E731
    req, lat = vals.get("TCP_TCC_READ_REQ", 0.0), vals.get("TCP_TCC_READ_REQ_LATENCY", 0.0)
    rows = [
        ("duration (median, under counter collection)", f"{vals['ns'] / 1e3:.1f} us"),
        ("shader clock", f"{gui / vals['ns']:.2f} GHz"),
        ("MFMA busy (of SIMD cycles)", f"{vals.get('SQ_VALU_MFMA_BUSY_CYCLES', 0.0) / (gui * SIMDS):.1%}"),
        ("TA busy (address unit, of CU cycles)", f"{per_cu('TA_TA_BUSY'):.1%}"),
        ("TD busy (data return to VGPRs / LDS)", f"{per_cu('TD_TD_BUSY'):.1%}"),
        ("TD stalled waiting on the L1/L2", f"{per_cu('TD_TC_STALL'):.1%}"),
        ("L1 stalled on pending misses", f"{per_cu('TCP_PENDING_STALL_CYCLES'):.1%}"),
        ("L1 -> L2 read requests per CU per cycle", f"{per_cu('TCP_TCC_READ_REQ'):.3f}"),
        ("L2 read requests in flight per CU (average)", f"{per_cu('TCP_TCC_READ_REQ_LATENCY'):.1f}"),
        ("average L2 read latency", f"{lat / req:.0f} cycles" if req else "-"),
        ("L1 accesses per CU per cycle", f"{per_cu('TCP_TOTAL_CACHE_ACCESSES'):.3f}"),
        ("LDS instructions / MFMA instructions", f"{vals.get('SQ_INSTS_LDS', 0.0) / max(vals.get('SQ_INSTS_MFMA', 1.0), 1.0):.2f}"),
        ("LDS bank conflict cycles per CU per cycle", f"{per_cu('SQ_LDS_BANK_CONFLICT'):.3f}"),
        ("global load instructions per CU per cycle", f"{per_cu('SQ_INSTS_VMEM'):.4f}"),
    ]
    lines = [f"# Memory pipe: {title}", "", f"Kernels matching `{regex}`; {len(paths)} rocprofv3 `--pmc` passes:", ""]
    lines += ["```", command, "```", "", "| quantity | value |", "|---|---|"]
    lines += [f"| {a} | {b} |" for a, b in rows]
    lines.append("")
    return "\n".join(lines)


def traffic_for(workload: str, kernel: str = "gate_up") -> int | None:
    """The committed traffic figure of one product (`gate_up` or `down`) at a bench workload
    (profiles/<kernel>_<workload>_traffic.md), if any."""
    p = PROFILES / f"{kernel}_{workload}_traffic.md"
    if p.exists():
        m = re.search(r"^traffic_bytes_per_dispatch: (\d+)$", p.read_text(), re.M)
        if m:
            return int(m.group(1))
    return None


def main(argv: list[str]) -> int:
    if not argv:
        print(__doc__)
        return 2
    if argv[0] == "copy":
        copy_probe()
        return 0
    if argv[0] == "stats" and len(argv) == 4:
        print(stats_md(argv[1], argv[2], argv[3]))
        return 0
    if argv[0] == "traffic" and len(argv) == 8:
        print(traffic_md(*argv[1:]))
        return 0
    if argv[0] == "pipe" and len(argv) >= 5:
        print(pipe_md(argv[1], argv[2], argv[3], argv[4:]))
        return 0
    if argv[0] == "mfma" and len(argv) == 7:
        print(mfma_md(argv[1], argv[2], float(argv[3]), float(argv[4]), argv[5], argv[6]))
        return 0
    print(__doc__)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
