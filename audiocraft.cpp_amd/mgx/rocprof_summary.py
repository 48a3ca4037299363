"""Summaries of rocprofv3 CSV output for the decode-step kernels.

    python3 -m mgx.rocprof_summary stats <kernel_stats.csv>
        per-kernel calls / total / average / min / max duration, GEMV instances also summed
        into one "k_gemv (all instances)" line;
    python3 -m mgx.rocprof_summary traffic <fetch counter_collection.csv> <write counter_collection.csv> <copy MiB>
        average FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the GEMV dispatches, each scaled
        by the same counter on the device-to-device copy of <copy MiB> that ran in the same
        process, and the resulting HBM bytes per GEMV launch.

Used to write the text summaries under profiles/; needs only the CSV files.
"""
import collections
import csv
import sys


def _rows(path):
    with open(path, newline="") as f:
        yield from csv.DictReader(f)


def _short(name):
    name = name.replace(".kd", "")
    return name if len(name) <= 96 else name[:93] + "..."


def stats(path):
    agg = collections.OrderedDict()
    for r in _rows(path):
        agg[r["Name"]] = (int(r["Calls"]), float(r["TotalDurationNs"]), float(r["AverageNs"]), float(r["MinNs"]),
                          float(r["MaxNs"]), float(r["Percentage"]))
    out = [f"{'kernel':96s} {'calls':>8s} {'total_ms':>10s} {'avg_us':>8s} {'min_us':>8s} {'max_us':>8s} {'pct':>6s}"]
    g_calls, g_total = 0, 0.0
    for name, (calls, total, avg, mn, mx, pct) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"{_short(name):96s} {calls:8d} {total / 1e6:10.3f} {avg / 1e3:8.2f} {mn / 1e3:8.2f} {mx / 1e3:8.2f} {pct:6.2f}")
        if "k_gemv" in name:
            g_calls += calls
            g_total += total
    if g_calls:
        out.append(f"{'k_gemv (all instances)':96s} {g_calls:8d} {g_total / 1e6:10.3f} {g_total / g_calls / 1e3:8.2f}")
    return "\n".join(out)


def _counter(path, counter):
    """Mean counter value (KiB) per dispatch for the GEMV kernels and for the copy kernel."""
    gemv, copy = [], []
    for r in _rows(path):
        if r.get("Counter_Name") != counter:
            continue
        v = float(r["Counter_Value"])
        if "k_gemv" in r["Kernel_Name"]:
            gemv.append(v)
        elif "copyBuffer" in r["Kernel_Name"]:
            copy.append(v)
    return (sum(gemv) / len(gemv) if gemv else 0.0), len(gemv), (max(copy) if copy else 0.0)


def traffic(fetch_csv, write_csv, copy_mib):
    f_gemv, n_f, f_copy = _counter(fetch_csv, "FETCH_SIZE")
    w_gemv, n_w, w_copy = _counter(write_csv, "WRITE_SIZE")
    copy_kib = float(copy_mib) * 1024.0
    f_scale = copy_kib / f_copy if f_copy else float("nan")
    w_scale = copy_kib / w_copy if w_copy else float("nan")
    per_launch = (f_gemv * f_scale + w_gemv * w_scale) * 1024.0
    return "\n".join([
        f"gemv dispatches: {n_f} (FETCH_SIZE run), {n_w} (WRITE_SIZE run)",
        f"FETCH_SIZE per GEMV dispatch: {f_gemv:.1f} KiB raw; copy of {copy_mib} MiB read {f_copy:.1f} KiB -> scale {f_scale:.4f}",
        f"WRITE_SIZE per GEMV dispatch: {w_gemv:.1f} KiB raw; copy of {copy_mib} MiB wrote {w_copy:.1f} KiB -> scale {w_scale:.4f}",
        f"traffic_bytes_per_launch: {per_launch:.0f}",
    ])


def main(argv):
    if len(argv) >= 2 and argv[0] == "stats":
        print(stats(argv[1]))
    elif len(argv) >= 4 and argv[0] == "traffic":
        print(traffic(argv[1], argv[2], argv[3]))
    else:
        print(__doc__, file=sys.stderr)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
