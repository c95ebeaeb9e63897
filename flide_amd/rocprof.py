"""rocprofv3 helpers for this package's measurements.

    python -m flide_amd.rocprof copy                       # the calibration kernel (run under rocprofv3 --pmc)
    python -m flide_amd.rocprof stats  <kernel_stats.csv> <title> <command> > summary.md
    python -m flide_amd.rocprof traffic <workload> <kernel-regex> <fetch.csv> <write.csv> \\
                                         <copy_fetch.csv> <copy_write.csv> <command> > traffic.md

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


def traffic_for(workload: str) -> int | None:
    """The committed traffic figure for a bench workload (profiles/*_<workload>_traffic.md), if any."""
    for p in sorted(PROFILES.glob(f"*_{workload}_traffic.md")):
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
    print(__doc__)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
