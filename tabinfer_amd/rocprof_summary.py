"""Summaries of rocprofv3 CSV output, as committed under profiles/.

    python -m tabinfer_amd.rocprof_summary stats  <dir-with-run_kernel_stats.csv>
    python -m tabinfer_amd.rocprof_summary pmc    <fetch-dir> <write-dir> [--calib KERNEL BYTES]
    python -m tabinfer_amd.rocprof_summary counters <dir> COUNTER [COUNTER ...]

`stats` prints the per-kernel table of a `rocprofv3 --kernel-trace --stats`
run (calls, average and total duration).

`counters` prints, per kernel, the average of each named counter per dispatch
of one `rocprofv3 --pmc` run (e.g. the MFMA counters).

`pmc` prints, per kernel, the average FETCH_SIZE and WRITE_SIZE (KiB per
dispatch) of two `rocprofv3 --pmc` runs. With --calib, the counters of the
named calibration kernel, which is known to read and write BYTES each, give
the factor that turns a counter into bytes (on the MI355X box FETCH_SIZE of a
plain copy reads half of the bytes the copy fetches; WRITE_SIZE reads them
exactly), and scaled HBM bytes per dispatch are printed beside the raw values.
"""
import collections
import csv
import os
import sys


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def short(name, width=70):
    name = name.replace("(anonymous namespace)::", "")
    if "(" in name:
        head, _, _ = name.partition("(")
        name = head
    return name[:width]


def stats(d):
    rows = _rows(os.path.join(d, "run_kernel_stats.csv"))
    out = ["| kernel | calls | avg us | min us | max us | total ms | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        out.append("| %s | %s | %.3f | %.3f | %.3f | %.3f | %.2f |" % (
            short(r["Name"]), r["Calls"], float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3,
            float(r["MaxNs"]) / 1e3, float(r["TotalDurationNs"]) / 1e6, float(r["Percentage"])))
    return "\n".join(out)


def pmc_avg(d, counter):
    acc = collections.defaultdict(list)
    for r in _rows(os.path.join(d, "run_counter_collection.csv")):
        if r["Counter_Name"] == counter:
            acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}, {k: len(v) for k, v in acc.items()}


def pmc(fetch_dir, write_dir, calib=None):
    fa, fn = pmc_avg(fetch_dir, "FETCH_SIZE")
    wa, _ = pmc_avg(write_dir, "WRITE_SIZE")
    kf = kw = None
    lines = []
    if calib:
        name, nbytes = calib
        hit = [k for k in fa if name in k]
        if hit:
            kib = nbytes / 1024.0
            kf = kib / fa[hit[0]]
            kw = kib / wa[hit[0]] if hit[0] in wa and wa[hit[0]] else None
            lines.append("calibration kernel %s (%d bytes read, %d written): FETCH_SIZE factor %.4f, WRITE_SIZE factor %s"
                         % (short(hit[0]), nbytes, nbytes, kf, "%.4f" % kw if kw else "n/a"))
    lines.append("")
    lines.append("| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read bytes | HBM write bytes |")
    lines.append("|---|---:|---:|---:|---:|---:|")
    for k in sorted(fa, key=lambda k: -fa[k] * fn[k]):
        rd = "%.0f" % (fa[k] * kf * 1024) if kf else "-"
        wr = "%.0f" % (wa.get(k, 0.0) * kw * 1024) if kw else "-"
        lines.append("| %s | %d | %.1f | %.1f | %s | %s |" % (short(k), fn[k], fa[k], wa.get(k, float("nan")), rd, wr))
    return "\n".join(lines)


def counters(d, names):
    avgs = [pmc_avg(d, n) for n in names]
    kernels = sorted(set().union(*[a[0].keys() for a in avgs]))
    lines = ["| kernel | dispatches | " + " | ".join(names) + " |", "|---|---:|" + "---:|" * len(names)]
    for k in kernels:
        n = max(a[1].get(k, 0) for a in avgs)
        lines.append("| %s | %d | %s |" % (short(k), n, " | ".join("%.0f" % a[0][k] if k in a[0] else "-" for a in avgs)))
    return "\n".join(lines)


def main(argv):
    if len(argv) >= 2 and argv[0] == "stats":
        print(stats(argv[1]))
    elif len(argv) >= 3 and argv[0] == "counters":
        print(counters(argv[1], argv[2:]))
    elif len(argv) >= 3 and argv[0] == "pmc":
        calib = None
        if "--calib" in argv:
            i = argv.index("--calib")
            calib = (argv[i + 1], int(argv[i + 2]))
        print(pmc(argv[1], argv[2], calib))
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
