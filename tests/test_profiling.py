"""The profiling tool's arithmetic on small synthetic rocprofv3 outputs (CPU only): marker
segmentation, the copy-calibrated HBM traffic per launch unit, the matrix-pipe busy share,
and the kernel labels of the trace summary.  These are the figures `profiles/` and the
benchmark's roofline entries are made from."""
import argparse
import csv
import json
import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "yolo11.cu_amd"))
import profiling  # noqa: E402

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _counters(d, counter_rows):
    """counter_collection.csv from (kernel, {counter: value}) per dispatch, in order."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (kernel, vals) in enumerate(counter_rows):
            for c, v in vals.items():
                w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": kernel, "Counter_Name": c, "Counter_Value": v})
    with open(os.path.join(d, "run_agent_info.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Simd_Count", "Num_Xcc"])
        w.writeheader()
        w.writerow({"Name": "AMD EPYC", "Simd_Count": 0, "Num_Xcc": 0})
        w.writerow({"Name": "gfx950", "Simd_Count": 1024, "Num_Xcc": 8})
    return d


M = "yolo::k_marker()"


def test_segments_split_by_markers(tmp_path):
    d = _counters(str(tmp_path / "c"), [
        ("warmup()", {"X": 5}), (M, {"X": 0}), ("a()", {"X": 1}), ("b()", {"X": 2}), (M, {"X": 0}),
        ("between()", {"X": 7}), (M, {"X": 0}), ("c()", {"X": 3}), (M, {"X": 0})])
    segs = profiling._segments(d, "X", unit=10.0)
    # dispatches outside a marker pair (the warmup, `between`) belong to no segment
    assert segs == [[("a()", 10.0), ("b()", 20.0)], [("c()", 30.0)]]


def _plan(path, units, passes, copy_bytes):
    plan = {"model": "yolo11x", "batch": 16, "passes": passes, "num_units": len(units), "units": units,
            "copy_bytes": copy_bytes, "op_configs": {}}
    json.dump(plan, open(path, "w"))
    return path


def test_traffic_scaled_by_the_copy(tmp_path):
    """Bytes = KiB x 1024 x (known copy bytes / what the counter read for the copy), median over
    passes, fetch + write per unit."""
    units = [{"unit": 0, "first": 3, "ops": [3], "kernel": "k_conv_gemm cfg 2", "class": "1x1", "flops": 1.0,
              "bytes": 4096.0},
             {"unit": 1, "first": 5, "ops": [5, 6], "kernel": "k_dwconv", "class": "depthwise 3x3", "flops": 0.0,
              "bytes": 1000.0}]
    plan = _plan(str(tmp_path / "plan.json"), units, 3, 2 * 1024.0 * 8)   # the copy moves 16 KiB

    def run(counter, per_pass, copy_kib):
        rows = []
        for p in range(3):
            for u in range(2):
                rows += [(M, {counter: 0})] + [(f"k{u}_{j}()", {counter: v}) for j, v in enumerate(per_pass[p][u])]
                rows += [(M, {counter: 0})]
        rows += [(M, {counter: 0}), ("yolo::k_copyc()", {counter: copy_kib}), (M, {counter: 0})]
        return _counters(str(tmp_path / counter), rows)

    # FETCH reads twice the copy's bytes (scale 2 x 16 / 16), WRITE exactly them (scale 1)
    fdir = run("FETCH_SIZE", [[[1, 1], [2]], [[3, 1], [2]], [[2, 2], [5]]], 8)
    wdir = run("WRITE_SIZE", [[[1], [1]], [[1], [1]], [[1], [1]]], 16)
    out_json = str(tmp_path / "t.json")
    args = argparse.Namespace(plan=plan, write_plan=None, fetch=fdir, write=wdir, json=out_json, md=None)
    profiling.summarize(args)
    got = json.load(open(out_json))
    assert got["scale"]["FETCH_SIZE"] == pytest.approx(2.0) and got["scale"]["WRITE_SIZE"] == pytest.approx(1.0)
    cols = got["columns"]
    u3 = dict(zip(cols, got["per_unit_first_op"]["3"]))
    # unit 0 fetch per pass (KiB): 2, 4, 4 -> median 4 KiB x 1024 x 2; write 1 KiB
    assert u3["fetch_bytes"] == 4 * 1024 * 2 and u3["write_bytes"] == 1024
    assert u3["traffic_bytes"] == 4 * 1024 * 2 + 1024 and u3["algorithmic_bytes"] == 4096
    u5 = dict(zip(cols, got["per_unit_first_op"]["5"]))
    assert u5["fetch_bytes"] == 2 * 1024 * 2      # passes 2, 2, 5 -> median 2
    assert got["total_traffic_bytes"] == u3["traffic_bytes"] + u5["traffic_bytes"]


def test_mfma_busy_share(tmp_path):
    """Executed FLOPs = busy cycles x 1,024; busy share = busy / (GUI_ACTIVE / XCDs x SIMDs)."""
    flops = 2.0 * 1024 * 1000          # the unit's algorithmic FLOPs
    units = [{"unit": 0, "first": 0, "ops": [0], "kernel": "k_conv_first", "class": "stem 3x3 s2", "flops": flops,
              "bytes": 1.0},
             {"unit": 1, "first": 1, "ops": [1], "kernel": "k_copyc", "class": "", "flops": 0.0, "bytes": 1.0}]
    plan = _plan(str(tmp_path / "plan.json"), units, 1, 1.0)
    busy, gui = 2500.0, 8 * 10.0       # 10 cycles on each of 8 XCDs = 10,240 SIMD-cycles
    rows = [(M, {}), ("k_conv_first()", {"SQ_VALU_MFMA_BUSY_CYCLES": busy, "GRBM_GUI_ACTIVE": gui}), (M, {}),
            (M, {}), ("k_copyc()", {"SQ_VALU_MFMA_BUSY_CYCLES": 0, "GRBM_GUI_ACTIVE": gui}), (M, {}),
            (M, {}), ("k_copyc()", {"SQ_VALU_MFMA_BUSY_CYCLES": 0, "GRBM_GUI_ACTIVE": gui}), (M, {})]
    rows = [(k, v or {"SQ_VALU_MFMA_BUSY_CYCLES": 0, "GRBM_GUI_ACTIVE": 0}) for k, v in rows]
    d = _counters(str(tmp_path / "pmc"), rows)
    md = str(tmp_path / "m.md")
    profiling.mfma(argparse.Namespace(plan=plan, pmc=d, md=md, top=5))
    text = open(md).read()
    # 2,500 x 1,024 executed against 2,048,000 algorithmic = 1.25x; busy 2,500 / 10,240
    row = next(ln for ln in text.splitlines() if ln.startswith("| stem 3x3 s2 |"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[4] == "1.250" and cells[5] == f"{2500 / 10240:.3f}" and cells[6] == f"{2000 / 10240:.3f}"
    assert "k_copyc" not in text.split("Units holding")[1]   # units without FLOPs are left out


def test_trace_labels_follow_the_tile_tables(tmp_path, capsys):
    """Trace rows name GEMM instantiations by tile config and streaming convs by op config, read
    from conv.hip's tables; mangled template names are demangled."""
    d = tmp_path / "tr"
    d.mkdir()
    rows = [("yolo::k_letterbox()", 0, 1000),
            ("void yolo::k_conv_gemm<256, 256, 4, 4, 64, 2, 1>(yolo::GemmLaunch)", 1000, 3000),
            ("_ZN4yolo10k_conv_tapILi1ELi1ELi256ELi192ELi4ELi2ELi1ELi3EEEvNS_4ViewES1_S1_PKDF16_PKfiiiiiiii", 3000, 4000),
            ("void yolo::k_conv_gemm<64, 64, 2, 2, 64, 3, 0>(yolo::GemmLaunch)", 4000, 4500)]
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for k, a, b in rows:
            w.writerow({"Kernel_Name": k, "Start_Timestamp": a, "End_Timestamp": b})
    profiling.trace(argparse.Namespace(csv=str(d), letterboxes_per_frame=1, top=10))
    out = capsys.readouterr().out
    assert "k_conv_gemm<256, 256, 4, 4, 64, 2, 1> [cfg 31 uni]" in out
    assert "k_conv_gemm<64, 64, 2, 2, 64, 3, 0> [cfg 12 1x1]" in out
    assert "yolo::k_conv_tap<1, 1, 256, 192, 4, 2, 1, 3> [op config 1109]" in out
    assert "4.500 ms" not in out and "1 frames: 0.0045 ms and 4 dispatches per frame" in out


def test_conv_roofline_ceiling():
    """The per-layer roofline tool on yolo11x b16 and yolo11n b1 (generator graph, CPU): the
    conv count and FLOPs equal what the engine's op descriptions give (173 convs, 3.118 TFLOP:
    the matrix-pipe profile's algorithmic total), and the summed per-layer times sit between
    the larger of the two whole-frame bounds and their sum."""
    x = profiling.conv_roofline("x", 16)
    assert x["convs"] == 173 and abs(x["tflop"] - 3.118) < 5e-4
    t_mfma, t_hbm = x["tflop"] * 1e12 / 2.5e15, x["gbytes"] * 1e9 / 6.3e12
    assert max(t_mfma, t_hbm) * 1e3 <= x["roofline_ms"] <= (t_mfma + t_hbm) * 1e3
    # slower MFMA-bound layers lower the reachable utilisation, by at most the factor f (no
    # layer's time grows more than 1/f)
    u = [x["at_frac"]["0.44"]["util"], x["at_frac"]["0.6"]["util"], x["util"]]
    assert u[0] < u[1] < u[2] < 1.0
    assert u[0] >= 0.44 * u[2] and u[1] >= 0.6 * u[2]
    # batch 1 of yolo11n: every conv is bound by its bytes, so the peak fraction plays no part
    n = profiling.conv_roofline("n", 1)
    assert n["mfma_bound"] == 0
    assert abs(n["roofline_ms"] - n["gbytes"] * 1e9 / 6.3e12 * 1e3) < 1e-9
    # (at 0.44 of the peak, layers just below the ridge become MFMA-bound, never faster)
    assert n["roofline_ms"] <= n["at_frac"]["0.44"]["ms"] <= n["roofline_ms"] / 0.44
