"""Summaries of rocprofv3 CSV output for this library's kernels.

    python -m turborag_amd.rocprof_summary kernels <dir>/<prefix> "<command>"
        Markdown table of a ``--kernel-trace --stats --output-format csv`` run:
        calls / average / min / median / max duration per kernel.

    python -m turborag_amd.rocprof_summary traffic <fetch-prefix> <write-prefix> \
        <copy-bytes> "<fetch command>" "<write command>" [json-out]
        HBM traffic per dispatch of each library kernel from two ``--pmc``
        runs (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by
        the factor that maps the same counter of a plain device copy of
        <copy-bytes> read and written onto those bytes.

    python -m turborag_amd.rocprof_summary counters <prefix> "<command>"
        Mean of every counter of a ``--pmc`` run (derived metrics included,
        e.g. MfmaUtil, VALUBusy, OccupancyPercent) per library kernel.

<prefix> is the path rocprofv3 wrote to minus the ``_kernel_trace.csv`` /
``_counter_collection.csv`` suffix.
"""
from __future__ import annotations

import csv
import json
import re
import statistics
import sys
from collections import defaultdict
from pathlib import Path


def short_name(name: str) -> str:
    n = name.replace("(anonymous namespace)::", "").replace("void ", "")
    n = re.sub(r"\(.*", "", n)
    return n[:90]


def is_copy(name: str) -> bool:
    """The runtime's device-to-device copy kernel (torch's same-dtype copy_)."""
    return "copyBuffer" in name


def kernel_durations(prefix: str) -> dict[str, list[float]]:
    """Per-kernel dispatch durations in µs from <prefix>_kernel_trace.csv."""
    d: dict[str, list[float]] = defaultdict(list)
    with open(f"{prefix}_kernel_trace.csv", newline="") as f:
        for r in csv.DictReader(f):
            dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
            d[short_name(r["Kernel_Name"])].append(dur)
    return d


def kernels_md(prefix: str, command: str) -> str:
    d = kernel_durations(prefix)
    out = [f"Command (repo root, MI355X):\n\n```\n{command}\n```\n",
           "| kernel | calls | avg µs | min µs | median µs | max µs |",
           "|---|---:|---:|---:|---:|---:|"]
    order = sorted(d.items(), key=lambda kv: -sum(kv[1]))
    # every kernel of this library, then the busiest others (torch, copies)
    ours = [kv for kv in order if kv[0].startswith("tq::")]
    others = [kv for kv in order if not kv[0].startswith("tq::")][:8]
    for n, v in ours + others:
        out.append(f"| `{n}` | {len(v)} | {statistics.mean(v):.3f} | {min(v):.3f} | "
                   f"{statistics.median(v):.3f} | {max(v):.3f} |")
    return "\n".join(out) + "\n"


def counter_values(prefix: str, counter: str) -> dict[str, list[float]]:
    d: dict[str, list[float]] = defaultdict(list)
    with open(f"{prefix}_counter_collection.csv", newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                d[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return d


def traffic(fetch_prefix: str, write_prefix: str, copy_bytes: int) -> dict:
    """{kernel: {fetch_B, write_B, bytes}} plus the two calibration factors."""
    fetch = counter_values(fetch_prefix, "FETCH_SIZE")
    write = counter_values(write_prefix, "WRITE_SIZE")

    def copy_kib(d):
        # The calibration copy is the largest copy of the run; smaller copies
        # (host uploads, small device copies) are ignored.
        v = [x for n, xs in d.items() if is_copy(n) for x in xs]
        if not v:
            raise SystemExit("no copy kernel dispatches in the counter run")
        big = max(v)
        return statistics.median([x for x in v if x >= 0.5 * big])

    f_fac = copy_bytes / (copy_kib(fetch) * 1024.0)
    w_fac = copy_bytes / (copy_kib(write) * 1024.0)
    res = {"calibration": {"copy_bytes_each_way": copy_bytes, "fetch_factor": round(f_fac, 4),
                           "write_factor": round(w_fac, 4)}, "kernels": {}}
    for n in fetch:
        if "tq::" not in n:
            continue
        fb = statistics.median(fetch[n]) * 1024.0 * f_fac
        wb = statistics.median(write.get(n, [0.0])) * 1024.0 * w_fac
        res["kernels"][short_name(n)] = {"dispatches": len(fetch[n]), "fetch_B": round(fb),
                                         "write_B": round(wb), "bytes": round(fb + wb)}
    return res


def counters_md(prefix: str, command: str) -> str:
    """Kernel x counter table of per-dispatch means (library kernels)."""
    d: dict[str, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    with open(f"{prefix}_counter_collection.csv", newline="") as f:
        for r in csv.DictReader(f):
            if "tq::" in r["Kernel_Name"]:
                d[short_name(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    names = sorted({c for v in d.values() for c in v})
    out = [f"Command (repo root, MI355X):\n\n```\n{command}\n```\n",
           "| kernel | dispatches | " + " | ".join(names) + " |",
           "|---|---:|" + "---:|" * len(names)]
    for k, v in d.items():
        n = max(len(x) for x in v.values())
        cells = [f"{statistics.mean(v[c]):.2f}" if c in v else "" for c in names]
        out.append(f"| `{k}` | {n} | " + " | ".join(cells) + " |")
    return "\n".join(out) + "\n"


def main(argv: list[str]) -> int:
    if len(argv) >= 3 and argv[0] == "kernels":
        print(kernels_md(argv[1], argv[2]))
        return 0
    if len(argv) >= 3 and argv[0] == "counters":
        print(counters_md(argv[1], argv[2]))
        return 0
    if len(argv) >= 6 and argv[0] == "traffic":
        res = traffic(argv[1], argv[2], int(argv[3]))
        out = [f"FETCH_SIZE run:\n\n```\n{argv[4]}\n```\n", f"WRITE_SIZE run:\n\n```\n{argv[5]}\n```\n",
               f"Calibration: a plain device copy of {res['calibration']['copy_bytes_each_way']} B "
               f"read and written; factor bytes/counter = {res['calibration']['fetch_factor']} "
               f"(FETCH_SIZE), {res['calibration']['write_factor']} (WRITE_SIZE).\n",
               "| kernel | dispatches | fetch B | write B | total B |", "|---|---:|---:|---:|---:|"]
        for n, k in res["kernels"].items():
            out.append(f"| `{n}` | {k['dispatches']} | {k['fetch_B']} | {k['write_B']} | "
                       f"{k['bytes']} |")
        print("\n".join(out))
        if len(argv) >= 7:
            Path(argv[6]).write_text(json.dumps(res, indent=1) + "\n")
        return 0
    print(__doc__)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
