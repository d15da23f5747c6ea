"""mockbird_amd.profile_frames on a hand-made kernel trace (CPU only): runs
split at idle gaps, frames cut at the delimiting kernel, warm-up frames
dropped, per-kernel counts and times per frame."""
import csv
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from mockbird_amd import profile_frames as pf  # noqa: E402


def _trace(path):
    rows, t = [], 0
    def add(name, dur_us, grid=64, gap_us=1):
        nonlocal t
        t += int(gap_us * 1000)
        rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(dur_us * 1000),
                     "Grid_Size_X": grid})
        t += int(dur_us * 1000)
    for run, grid in ((0, 64), (1, 256)):
        if run:
            t += 20_000_000  # 20 ms idle: a new run
        for f in range(5):
            add("void mb::k_gemm<2, 2, 0>(float const*, long)", 10 + run, grid)
            add("void mb::k_gemm<2, 2, 0>(float const*, long)", 10 + run, grid)
            add("mb::k_attn(int)", 30 if f == 0 else 20, grid)
            add("mb::(anonymous namespace)::k_add_i32(int*, int, int)", 1, grid)
            add("mb::k_frame_emit(int*)", 2, grid)
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_runs_frames_and_breakdown(tmp_path):
    p = str(tmp_path / "t.csv")
    _trace(p)
    runs = pf.split_runs(pf.load(p), 5e6)
    assert len(runs) == 2 and all(len(r) == 25 for r in runs)
    fr = pf.frames_of(runs[0], "k_frame_emit", skip=1, last=None)
    assert len(fr) == 3  # 5 delimiters -> 4 frames after the first, one skipped
    b = pf.breakdown(runs[0], fr)
    k = {name: (c, avg, per) for name, c, avg, per in b["kernels"]}
    assert k["mb::k_gemm<2, 2, 0>"] == (2, 10.0, 20.0)
    assert k["mb::k_attn"] == (1, 20.0, 20.0)
    assert k["mb::k_add_i32"] == (1, 1.0, 1.0)
    assert b["launches"] == 5 and b["kernel_us"] == 43.0
    assert abs(b["span_us"] - 48.0) < 1e-9  # 43 us of kernels + 5 gaps of 1 us
    last = pf.breakdown(runs[1], pf.frames_of(runs[1], "k_frame_emit", 0, 2))
    assert last["frames"] == 2 and dict((n, c) for n, c, _, _ in last["kernels"])["mb::k_gemm<2, 2, 0>"] == 2
    assert pf.grid_of(runs[1], "k_frame_emit") == "256"


def test_cli_prints_a_table_per_run(tmp_path, capsys):
    p = str(tmp_path / "t.csv")
    _trace(p)
    assert pf.main([p, "--delimiter", "k_frame_emit", "--skip", "1", "--grid-of", "k_frame_emit"]) == 0
    out = capsys.readouterr().out
    assert out.count("| kernel |") == 2 and "grid 256" in out and "`mb::k_attn` | 1 | 20.00" in out


def test_grids_lists_one_launch_shape_per_line(tmp_path, capsys):
    p = str(tmp_path / "t.csv")
    _trace(p)
    g = pf.by_grid(pf.load(p), "k_gemm")
    assert [(k, grid, n, avg) for k, grid, _, n, avg, _, _ in g] == [
        ("mb::k_gemm<2, 2, 0>", 64, 10, 10.0), ("mb::k_gemm<2, 2, 0>", 256, 10, 11.0)]
    assert pf.main([p, "--grids", "k_attn"]) == 0
    out = capsys.readouterr().out
    assert "| `mb::k_attn` | 64 | 0 | 5 | 22.00 | 20.00 | 30.00 |" in out


def test_grids_on_a_counter_collection(tmp_path, capsys):
    p = str(tmp_path / "c.csv")
    rows = []
    for d, (grid, val) in enumerate([(64, 10.0), (64, 30.0), (64, 20.0), (256, 5.0), (256, 7.0)]):
        for c, scale in (("FETCH_SIZE", 1.0), ("WRITE_SIZE", 0.5)):
            rows.append({"Dispatch_Id": d, "Kernel_Name": "mb::k_ring_write<true>(int)",
                         "Grid_Size": grid, "Counter_Name": c, "Counter_Value": val * scale})
    rows.append({"Dispatch_Id": 9, "Kernel_Name": "other", "Grid_Size": 64,
                 "Counter_Name": "FETCH_SIZE", "Counter_Value": 1.0})
    with open(p, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    got = pf.counters_by_grid(p, "k_ring_write")
    assert got == [("mb::k_ring_write<true>", 64, "FETCH_SIZE", 3, 20.0),
                   ("mb::k_ring_write<true>", 64, "WRITE_SIZE", 3, 10.0),
                   ("mb::k_ring_write<true>", 256, "FETCH_SIZE", 2, 6.0),
                   ("mb::k_ring_write<true>", 256, "WRITE_SIZE", 2, 3.0)]
    assert pf.main([p, "--grids", "k_ring_write"]) == 0
    assert "| `mb::k_ring_write<true>` | 256 | FETCH_SIZE | 2 | 6.0 |" in capsys.readouterr().out


def test_nth_launch_means(tmp_path, capsys):
    p = str(tmp_path / "t.csv")
    _trace(p)
    run = pf.split_runs(pf.load(p), 5e6)[0]
    fr = pf.frames_of(run, "k_frame_emit", skip=0, last=None)
    got = pf.nth_launches(run, fr, "k_gemm")
    assert got == {"mb::k_gemm<2, 2, 0>": [10.0, 10.0]}
    assert pf.main([p, "--delimiter", "k_frame_emit", "--nth", "k_attn"]) == 0
    assert "`mb::k_attn` by launch order in the frame (us): 20.00" in capsys.readouterr().out


def test_grids_by_run_splits_shapes_sharing_a_grid(tmp_path):
    p = str(tmp_path / "r.csv")
    rows, t = [], 0
    for name, dur, n in (("mb::k_gemm<1>(int)", 5, 3), ("mb::k_other(int)", 1, 1),
                         ("mb::k_gemm<1>(int)", 9, 2), ("mb::k_gemm<2>(int)", 4, 2),
                         ("mb::k_gemm<1>(int)", 7, 1)):
        for _ in range(n):
            rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur * 1000,
                         "Grid_Size_X": 64, "Workgroup_Size_X": 256})
            t += dur * 1000 + 100
    with open(p, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    runs = pf.by_grid(pf.load(p), "k_gemm", by_run=True)
    # the k_other dispatch between the two k_gemm<1> runs does not match the
    # filter, so those two runs join; k_gemm<2> splits them from the last
    assert [(k, n, avg) for k, _, _, n, avg, _, _ in runs] == [
        ("mb::k_gemm<1>", 5, 6.6), ("mb::k_gemm<2>", 2, 4.0), ("mb::k_gemm<1>", 1, 7.0)]
    assert [(k, n) for k, _, _, n, _, _, _ in pf.by_grid(pf.load(p), "k_gemm")] == [
        ("mb::k_gemm<1>", 6), ("mb::k_gemm<2>", 2)]


def test_counters_by_run(tmp_path):
    p = str(tmp_path / "c.csv")
    rows = []
    for d, (name, val) in enumerate([("mb::k_g<1>(int)", 10.0), ("mb::k_g<1>(int)", 12.0),
                                     ("mb::k_g<2>(int)", 5.0), ("mb::k_g<1>(int)", 30.0)]):
        rows.append({"Dispatch_Id": d, "Kernel_Name": name, "Grid_Size": 64,
                     "Counter_Name": "MfmaUtil", "Counter_Value": val})
    with open(p, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    assert pf.counters_by_grid(p, "k_g", by_run=True) == [
        ("mb::k_g<1>", 64, "MfmaUtil", 2, 11.0), ("mb::k_g<2>", 64, "MfmaUtil", 1, 5.0),
        ("mb::k_g<1>", 64, "MfmaUtil", 1, 30.0)]
    assert pf.counters_by_grid(p, "k_g")[0] == ("mb::k_g<1>", 64, "MfmaUtil", 3, 12.0)
