"""Summaries of rocprofv3 CSV output, as committed under profiles/.

    python -m tabinfer_amd.rocprof_summary stats  <dir-with-run_kernel_stats.csv>
    python -m tabinfer_amd.rocprof_summary pmc    <fetch-dir> <write-dir> [--calib KERNEL BYTES]
    python -m tabinfer_amd.rocprof_summary counters <dir> COUNTER [COUNTER ...]
    python -m tabinfer_amd.rocprof_summary traffic <fetch-dir> <write-dir> --calib KERNEL BYTES
        --commit HASH --sources FILE [FILE ...] --map NAME=KERNEL [NAME=KERNEL ...] -o OUT.json
        [--note WORD ...]

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

`traffic` writes the scaled HBM bytes (read + written) per dispatch of the kernels
named by --map (NAME=substring of the kernel's name) as JSON, stamped with the commit
the runs measured and the sha256 of each kernel source file given, so that a reader
can tell a figure measured on other sources (bench.py marks such a figure stale).
"""
import hashlib
import json
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


def pmc_vals(d, counter):
    acc = collections.defaultdict(list)
    for r in _rows(os.path.join(d, "run_counter_collection.csv")):
        if r["Counter_Name"] == counter:
            acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return acc


def pmc_avg(d, counter):
    acc = pmc_vals(d, counter)
    return {k: sum(v) / len(v) for k, v in acc.items()}, {k: len(v) for k, v in acc.items()}


def calib_factors(fetch_dir, write_dir, calib):
    """KiB-to-bytes factors of FETCH_SIZE and WRITE_SIZE from the calibration kernel's
    largest dispatches (those within half of its largest reading: a run may also use the
    same copy kernel for small copies), each of which reads and writes `BYTES`."""
    name, nbytes = calib
    out = []
    for d, counter in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        vals = pmc_vals(d, counter)
        hit = [k for k in vals if name in k]
        if len(hit) != 1:
            raise SystemExit("calibration kernel %s: %d matches in %s" % (name, len(hit), d))
        big = [v for v in vals[hit[0]] if v >= 0.5 * max(vals[hit[0]])]
        out.append(nbytes / 1024.0 / (sum(big) / len(big)))
    return out[0], out[1], short(hit[0])


def pmc(fetch_dir, write_dir, calib=None):
    fa, fn = pmc_avg(fetch_dir, "FETCH_SIZE")
    wa, _ = pmc_avg(write_dir, "WRITE_SIZE")
    kf = kw = None
    lines = []
    if calib:
        kf, kw, cname = calib_factors(fetch_dir, write_dir, calib)
        lines.append("calibration kernel %s (its dispatches reading and writing %d bytes): FETCH_SIZE factor %.4f, "
                     "WRITE_SIZE factor %.4f" % (cname, calib[1], kf, kw))
    lines.append("")
    lines.append("| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read bytes | HBM write bytes |")
    lines.append("|---|---:|---:|---:|---:|---:|")
    for k in sorted(fa, key=lambda k: -fa[k] * fn[k]):
        rd = "%.0f" % (fa[k] * kf * 1024) if kf else "-"
        wr = "%.0f" % (wa.get(k, 0.0) * kw * 1024) if kw else "-"
        lines.append("| %s | %d | %.1f | %.1f | %s | %s |" % (short(k), fn[k], fa[k], wa.get(k, float("nan")), rd, wr))
    return "\n".join(lines)


def traffic(fetch_dir, write_dir, calib, commit, sources, mapping, note=""):
    fa, fn = pmc_avg(fetch_dir, "FETCH_SIZE")
    wa, _ = pmc_avg(write_dir, "WRITE_SIZE")
    kf, kw, _ = calib_factors(fetch_dir, write_dir, calib)
    fams = {}
    for name, sub in mapping:
        hit = sorted(k for k in fa if sub in k)
        if len(hit) != 1:
            raise SystemExit("--map %s=%s matches %d kernels: %s" % (name, sub, len(hit), [short(k) for k in hit]))
        k = hit[0]
        fams[name] = int(round(fa[k] * kf * 1024 + wa.get(k, 0.0) * kw * 1024))
    stamp = {"commit": commit, "sources": {}}
    for path in sources:
        with open(path, "rb") as f:
            stamp["sources"][os.path.relpath(path)] = hashlib.sha256(f.read()).hexdigest()
    return {"families": fams, "kernels": {n: short(s, 200) for n, s in mapping},
            "_source": ("%s: " % note if note else "") +
                       "rocprofv3 --pmc FETCH_SIZE x %.4f + WRITE_SIZE x %.4f (%s %d-byte calibration), HBM bytes per "
                       "dispatch" % (kf, kw, calib[0], calib[1]),
            "_stamp": stamp}


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
    elif len(argv) >= 3 and argv[0] == "traffic":
        opts, cur = {}, None
        for a in argv[3:]:
            if a.startswith("--") or a == "-o":
                cur = a
                opts[cur] = []
            elif cur:
                opts[cur].append(a)
        calib = (opts["--calib"][0], int(opts["--calib"][1]))
        mapping = [tuple(m.split("=", 1)) for m in opts["--map"]]
        res = traffic(argv[1], argv[2], calib, opts["--commit"][0], opts.get("--sources", []), mapping,
                      " ".join(opts.get("--note", [])))
        with open(opts["-o"][0], "w") as f:
            json.dump(res, f, indent=1)
            f.write("\n")
        print(json.dumps(res, indent=1))
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
