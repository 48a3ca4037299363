"""Summaries of rocprofv3 CSV output for the decode-step kernels.

    python3 -m mgx.rocprof_summary stats <kernel_stats.csv>
        per-kernel calls / total / average / min / max duration, the GEMV and attention-combine
        instances also summed into one "(all instances)" line each;
    python3 -m mgx.rocprof_summary traffic <fetch counter_collection.csv> <write counter_collection.csv> <copy MiB>
                                           [<name>=<regex>[+<regex>...] [last=<n>]]
        average FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the GEMV dispatches -- or, with a
        unit spec, of each listed kernel's last n dispatches, summed over the kernels (one
        "launch" of a unit such as the attention is one dispatch of each) -- each scaled by the
        same counter on the device-to-device copy of <copy MiB> that ran in the same process,
        and the resulting HBM bytes per launch;
    python3 -m mgx.rocprof_summary window <kernel_trace.csv> <first regex> <end regex> [skip=<n>]
        the dispatches from the first one whose kernel matches <first regex> (the (n+1)-th with
        skip) up to (not including) the next one matching <end regex> ("$" for the trace's end)
        -- e.g. a prompt's prefill, from its first wide matrix-core GEMV to the first sampler
        launch, or the decode steps after the first n: the window's wall time, its busy time and
        per-kernel calls / total / average duration.

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
    families = {"k_gemv": [0, 0.0], "k_attn_combine": [0, 0.0]}
    for name, (calls, total, avg, mn, mx, pct) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"{_short(name):96s} {calls:8d} {total / 1e6:10.3f} {avg / 1e3:8.2f} {mn / 1e3:8.2f} {mx / 1e3:8.2f} {pct:6.2f}")
        for fam, acc in families.items():
            if fam in name:
                acc[0] += calls
                acc[1] += total
    for fam, (calls, total) in families.items():
        if calls:
            out.append(f"{fam + ' (all instances)':96s} {calls:8d} {total / 1e6:10.3f} {total / calls / 1e3:8.2f}")
    return "\n".join(out)


def _counter(path, counter, pattern=None, last=0):
    """Mean counter value (KiB) per dispatch of the kernels matching `pattern` (default: every
    GEMV), over their last `last` dispatches when given, and the copy kernel's value."""
    import re
    vals, copy = [], []
    rx = re.compile(pattern) if pattern else None
    for r in _rows(path):
        if r.get("Counter_Name") != counter:
            continue
        v = float(r["Counter_Value"])
        name = r["Kernel_Name"]
        if "copyBuffer" in name:
            copy.append(v)
        elif (rx.search(name) if rx else "k_gemv" in name):
            vals.append((int(r.get("Dispatch_Id", 0) or 0), v))
    vals.sort()
    if last:
        vals = vals[-last:]
    v = [x for _, x in vals]
    return (sum(v) / len(v) if v else 0.0), len(v), (max(copy) if copy else 0.0)


def traffic(fetch_csv, write_csv, copy_mib, unit=None, last=0):
    copy_kib = float(copy_mib) * 1024.0
    name, patterns = ("gemv", [None]) if unit is None else (unit.split("=", 1)[0], unit.split("=", 1)[1].split("+"))
    lines, total = [], 0.0
    for pat in patterns:
        f_avg, n_f, f_copy = _counter(fetch_csv, "FETCH_SIZE", pat, last)
        w_avg, n_w, w_copy = _counter(write_csv, "WRITE_SIZE", pat, last)
        f_scale = copy_kib / f_copy if f_copy else float("nan")
        w_scale = copy_kib / w_copy if w_copy else float("nan")
        total += (f_avg * f_scale + w_avg * w_scale) * 1024.0
        label = pat or "k_gemv"
        lines += [f"{label}: {n_f} dispatches (FETCH_SIZE run), {n_w} (WRITE_SIZE run)",
                  f"  FETCH_SIZE per dispatch {f_avg:.1f} KiB raw; copy of {copy_mib} MiB read {f_copy:.1f} KiB -> scale {f_scale:.4f}",
                  f"  WRITE_SIZE per dispatch {w_avg:.1f} KiB raw; copy of {copy_mib} MiB wrote {w_copy:.1f} KiB -> scale {w_scale:.4f}"]
    lines.append(f"traffic_bytes_per_launch {name}: {total:.0f}" if unit else f"traffic_bytes_per_launch: {total:.0f}")
    return "\n".join(lines)


def window(path, first, end, skip=0):
    import re
    rows = sorted(_rows(path), key=lambda r: int(r["Start_Timestamp"]))
    rf = re.compile(first)
    hits = [i for i, r in enumerate(rows) if rf.search(r["Kernel_Name"])]
    if len(hits) <= skip:
        return f"{len(hits)} dispatches match {first!r}, fewer than skip + 1 = {skip + 1}"
    i0 = hits[skip]
    if end == "$":
        i1 = len(rows)
    else:
        re_end = re.compile(end)
        i1 = next((i for i in range(i0 + 1, len(rows)) if re_end.search(rows[i]["Kernel_Name"])), len(rows))
    w = rows[i0:i1]
    agg = collections.defaultdict(lambda: [0, 0.0])
    for r in w:
        name = r["Kernel_Name"].split("(")[0]
        if "k_attn_combine" in name:
            name = "k_attn_combine<*>"
        agg[name][0] += 1
        agg[name][1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    wall = (int(w[-1]["End_Timestamp"]) - int(w[0]["Start_Timestamp"])) / 1e6
    busy = sum(v[1] for v in agg.values()) / 1e3
    out = [f"window: {len(w)} dispatches, {wall:.2f} ms wall, {busy:.2f} ms busy",
           f"{'kernel':72s} {'calls':>7s} {'total_ms':>9s} {'avg_us':>8s} {'share':>6s}"]
    for name, (calls, us) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"{_short(name):72s} {calls:7d} {us / 1e3:9.2f} {us / calls:8.2f} {us / 1e3 / busy:6.1%}")
    return "\n".join(out)


def main(argv):
    if len(argv) >= 2 and argv[0] == "stats":
        print(stats(argv[1]))
    elif len(argv) >= 4 and argv[0] == "window":
        skip = int(argv[4].split("=", 1)[1]) if len(argv) >= 5 else 0
        print(window(argv[1], argv[2], argv[3], skip))
    elif len(argv) >= 4 and argv[0] == "traffic":
        unit = argv[4] if len(argv) >= 5 else None
        last = int(argv[5].split("=", 1)[1]) if len(argv) >= 6 else 0
        print(traffic(argv[1], argv[2], argv[3], unit, last))
    else:
        print(__doc__, file=sys.stderr)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
