"""The rocprofv3 CSV summaries behind the committed profiles: per-kernel stats with the GEMV and
attention-combine families summed, and the counter traffic per launch scaled by the copy of
known size (FETCH_SIZE reads half of a copy's bytes on this GPU, WRITE_SIZE all of them)."""
import csv

import pytest

from mgx import rocprof_summary as S


def write(path, rows, fields):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(r)


def counters(path, counter, per_kernel, copy_kib):
    rows, d = [], 0
    for name, vals in per_kernel:
        for v in vals:
            d += 1
            rows.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": v})
    rows.append({"Dispatch_Id": 0, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": counter,
                 "Counter_Value": copy_kib})
    write(path, rows, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])


def test_traffic_scales_by_the_copy_and_takes_the_last_dispatches(tmp_path):
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    qkv = "void mgx::k_gemv<8, 2, 16, 3, 0, 2, 8>(mgx::GemvArgs)"
    ff0 = "void mgx::k_gemv<8, 2, 16, 3, 0, 3, 8>(mgx::GemvArgs)"
    # early dispatches (prefill) read more; the unit takes the last two of its kernel
    counters(f, "FETCH_SIZE", [(qkv, [9000.0, 3000.0, 3000.0]), (ff0, [5000.0])], 512.0 * 1024)
    counters(w, "WRITE_SIZE", [(qkv, [90.0, 30.0, 30.0]), (ff0, [20.0])], 1024.0 * 1024)
    out = S.traffic(str(f), str(w), 1024, "qkv=k_gemv<8, 2, 16, 3, 0, 2, 8>", last=2)
    line = [l for l in out.splitlines() if l.startswith("traffic_bytes_per_launch qkv:")][0]
    assert float(line.split(":")[1]) == pytest.approx((3000.0 * 2.0 + 30.0 * 1.0) * 1024)
    # a unit of two kernels adds one dispatch of each
    out = S.traffic(str(f), str(w), 1024, "both=k_gemv<8, 2, 16, 3, 0, 2+k_gemv<8, 2, 16, 3, 0, 3", last=1)
    line = [l for l in out.splitlines() if l.startswith("traffic_bytes_per_launch both:")][0]
    assert float(line.split(":")[1]) == pytest.approx(((3000.0 + 5000.0) * 2.0 + (30.0 + 20.0)) * 1024)


def test_stats_sums_the_instance_families(tmp_path):
    p = tmp_path / "stats.csv"
    rows = [("void mgx::k_gemv<8, 2, 16, 3, 0, 2, 8>(mgx::GemvArgs)", 10, 60000.0),
            ("void mgx::k_gemv<8, 1, 16, 3, 0, 0, 4>(mgx::GemvArgs)", 10, 40000.0),
            ("void mgx::k_attn_combine<20>(mgx::AttnArgs)", 4, 12000.0),
            ("void mgx::k_attn_combine<21>(mgx::AttnArgs)", 4, 14000.0),
            ("mgx::k_attn_chunk(mgx::AttnArgs)", 8, 64000.0)]
    write(p, [{"Name": n, "Calls": c, "TotalDurationNs": t, "AverageNs": t / c, "MinNs": t / c, "MaxNs": t / c,
               "Percentage": 0.0} for n, c, t in rows],
          ["Name", "Calls", "TotalDurationNs", "AverageNs", "MinNs", "MaxNs", "Percentage"])
    out = S.stats(str(p)).splitlines()
    assert out[1].startswith("mgx::k_attn_chunk")                 # largest total first
    gemv = [l for l in out if l.startswith("k_gemv (all instances)")][0].split()
    assert gemv[3:6] == ["20", "0.100", "5.00"]
    comb = [l for l in out if l.startswith("k_attn_combine (all instances)")][0].split()
    assert comb[3:6] == ["8", "0.026", "3.25"]


def test_window_takes_the_dispatches_between_the_markers(tmp_path):
    p = tmp_path / "trace.csv"
    # (kernel, start ns, end ns): a decode launch, the window (two wide GEMVs, an attention,
    # two combines), the sampler that ends it, and a later wide GEMV outside it
    rows = [("void mgx::k_gemv<8, 2, 16, 3, 0, 2, 8>(mgx::GemvArgs)", 0, 5000),
            ("void mgx::k_gemv_mf<8, 48, 16, 1, 1, true>(mgx::GemvArgs)", 10000, 16000),
            ("mgx::k_attn_prefill(mgx::AttnArgs)", 17000, 29000),
            ("void mgx::k_attn_combine<3>(mgx::AttnArgs)", 30000, 34000),
            ("void mgx::k_attn_combine<4>(mgx::AttnArgs)", 35000, 37000),
            ("void mgx::k_gemv_mf<8, 48, 16, 1, 1, true>(mgx::GemvArgs)", 38000, 42000),
            ("mgx::k_sample(mgx::SampleArgs)", 43000, 60000),
            ("void mgx::k_gemv_mf<8, 48, 16, 1, 1, true>(mgx::GemvArgs)", 61000, 70000)]
    # rows out of start order: the window sorts them
    write(p, [{"Kernel_Name": n, "Start_Timestamp": s, "End_Timestamp": e} for n, s, e in reversed(rows)],
          ["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
    out = S.window(str(p), "k_gemv_mf", "k_sample").splitlines()
    assert out[0] == "window: 5 dispatches, 0.03 ms wall, 0.03 ms busy"
    gemv = [l for l in out if l.startswith("void mgx::k_gemv_mf")][0].split()
    assert gemv[-4:] == ["2", "0.01", "5.00", "35.7%"]
    comb = [l for l in out if l.startswith("k_attn_combine<*>")][0].split()
    assert comb[1:4] == ["2", "0.01", "3.00"]
    assert out[2].startswith("mgx::k_attn_prefill")              # largest total first


def test_window_skips_to_the_nth_match_and_runs_to_the_end(tmp_path):
    p = tmp_path / "trace.csv"
    rows = [("mgx::k_sample(mgx::SampleArgs)", 0, 1000), ("mgx::k_attn_chunk(mgx::AttnArgs)", 2000, 3000),
            ("mgx::k_sample(mgx::SampleArgs)", 4000, 5000), ("mgx::k_attn_chunk(mgx::AttnArgs)", 6000, 9000),
            ("mgx::k_sample(mgx::SampleArgs)", 10000, 11000)]
    write(p, [{"Kernel_Name": n, "Start_Timestamp": s, "End_Timestamp": e} for n, s, e in rows],
          ["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
    out = S.window(str(p), "k_sample", "$", skip=1).splitlines()
    assert out[0].startswith("window: 3 dispatches")
    chunk = [l for l in out if l.startswith("mgx::k_attn_chunk")][0].split()
    assert chunk[1:4] == ["1", "0.00", "3.00"]
    assert "fewer than" in S.window(str(p), "k_sample", "$", skip=3)
