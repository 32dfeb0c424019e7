"""Profiling tools: HBM traffic per launch unit (or per tile config of one conv shape) and
matrix-pipe occupancy per launch unit from rocprofv3 PMC passes, and the steady-state kernel
time of a frame from a rocprofv3 kernel trace.

HBM traffic per launch unit:

    OUT=out/traffic_x
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/fetch -o run -- \\
        python3 yolo11.cu_amd/profiling.py collect --scale x --batch 16 --plan $OUT/plan.json
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/write -o run -- \\
        python3 yolo11.cu_amd/profiling.py collect --scale x --batch 16 --plan $OUT/wplan.json \\
        --replay $OUT/plan.json
    python3 yolo11.cu_amd/profiling.py summarize --plan $OUT/plan.json --write-plan $OUT/wplan.json \\
        --fetch $OUT/fetch --write $OUT/write --json profiles/yolo11x_b16_traffic.json \\
        --md profiles/yolo11x_b16_traffic.md

`collect` builds the engine as the benchmark does (seeded model, autotuned tiles), stages the
benchmark's frames, and runs every launch unit of the frame between two marker kernels
(yolo_marker), `--passes` times, so each dispatch in the trace belongs to the unit between its
markers; then a plain copy of known size, the scale reference: FETCH_SIZE and WRITE_SIZE are
scaled by the known bytes of that copy over what the counters read for it.  `summarize` maps
the dispatches to units, takes the median over the passes, pairs the two runs' units with
the same ops and kernel, and writes the per-unit traffic beside each unit's algorithmic bytes
(unitwork.py) as JSON and as a markdown table.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

COPY_HWC = (160, 160, 384)   # the scale reference: a copy of B x 160 x 160 x 384 fp16


def collect(args):
    import modelgen
    import unitwork
    import yolort
    B = args.batch
    work = tempfile.mkdtemp(prefix="yolo_traffic_")
    d = os.path.join(work, "model")
    modelgen.write_model(d, "yolo11", args.scale, cls_bias=-8.0)
    eng = yolort.Engine(d, B, yolort.YOLO_NOGRAPH)
    frames = [modelgen.synth_frame(640, 640, 50, 100 + i) for i in range(B)]
    devs = []
    for s, f in enumerate(frames):
        b = yolort.DeviceBuffer(f.nbytes)
        eng.upload(b, f)
        eng.preprocess(b.ptr, 640, 640, s)
        devs.append(b)
    # a second counter's run (--replay: the first run's plan) takes the first run's kernel
    # choices, since the autotuner times candidates and could pick differently; launch units
    # are planned with timing too, so each run records its own and summarize pairs them
    if args.replay:
        prev = json.load(open(args.replay))
        for k, (cfg, tail, split) in prev["op_configs"].items():
            k = int(k)
            if cfg < 0:                      # stem and depthwise convs: no choice to replay
                continue
            if eng.op_config(k) != cfg:
                eng.set_op_config(k, cfg)
            if cfg >= 1000:                  # special kernels: no split, no tail
                continue
            if split != eng.op_split(k):
                eng.set_op_split(k, split)
            if tail != eng.op_tail(k):
                eng.set_op_tail(k, tail)
    plan = {"model": f"yolo11{args.scale}", "batch": B, "passes": args.passes,
            "units": unitwork.units(eng, B), "copy_bytes": 2.0 * B * COPY_HWC[0] * COPY_HWC[1] * COPY_HWC[2],
            "op_configs": {str(k): (eng.op_config(k), eng.op_tail(k), eng.op_split(k))
                           for k in range(eng.num_ops) if eng.op_info(k)["kind"] == "CONV"}}
    plan["num_units"] = eng.num_units()
    for _ in range(args.passes):
        for u in range(plan["num_units"]):
            eng.marker()
            eng.run_unit(u, B)
            eng.marker()
    eng.sync()
    dc = os.path.join(work, "copy")
    modelgen.write_copy(dc, *COPY_HWC)
    ec = yolort.Engine(dc, B, yolort.YOLO_NOGRAPH | yolort.YOLO_NOTUNE)
    ec.marker()
    ec.run_unit(0, B)
    ec.marker()
    ec.sync()
    json.dump(plan, open(args.plan, "w"))
    for b in devs:
        b.free()
    ec.close()
    eng.close()
    print(f"collected {args.passes} passes of {plan['num_units']} units", flush=True)


def tiles(args):
    """One conv shape under each of the given op configs (`--passes` launches of each, every
    launch between two markers), then the scale-reference copy."""
    import modelgen
    import numpy as np
    import yolort
    k, st, H, cin, cout = args.shape
    B = args.batch
    work = tempfile.mkdtemp(prefix="yolo_tiles_")
    d = os.path.join(work, "conv")
    modelgen.write_single_conv(d, H, H, cin, cout, k, st, seed=1)
    eng = yolort.Engine(d, B, yolort.YOLO_NOGRAPH | yolort.YOLO_NOTUNE)
    eng.write(0, np.random.default_rng(1).standard_normal((B, H, H, cin), dtype=np.float32).astype(np.float16))
    done = []
    for cfg in args.cfgs:
        try:
            eng.set_op_config(0, cfg)
        except ValueError:
            continue
        eng.run_op(0, B)
        for _ in range(args.passes):
            eng.marker()
            eng.run_op(0, B)
            eng.marker()
        done.append(cfg)
    eng.sync()
    eng.close()
    dc = os.path.join(work, "copy")
    modelgen.write_copy(dc, *COPY_HWC)
    ec = yolort.Engine(dc, B, yolort.YOLO_NOGRAPH | yolort.YOLO_NOTUNE)
    ec.marker()
    ec.run_unit(0, B)
    ec.marker()
    ec.sync()
    ec.close()
    ho = (H + 2 * (k // 2) - k) // st + 1
    plan = {"shape": [k, st, H, cin, cout], "batch": B, "passes": args.passes, "cfgs": done,
            "copy_bytes": 2.0 * B * COPY_HWC[0] * COPY_HWC[1] * COPY_HWC[2],
            "input_bytes": 2.0 * B * H * H * cin, "weight_bytes": 2.0 * cout * k * k * cin,
            "output_bytes": 2.0 * B * ho * ho * cout, "bias_bytes": 4.0 * cout}
    json.dump(plan, open(args.plan, "w"))
    print(f"collected {args.passes} launches of {len(done)} configs", flush=True)


def tiles_summary(args):
    """Markdown rows of `tiles` runs: per config, the median scaled FETCH and WRITE bytes of a
    launch against the algorithmic bytes."""
    import re
    src = open(os.path.join(HERE, "csrc", "conv.hip")).read()
    body = src[src.index("#define YOLO_TILES("):]
    body = body[:body.index("\n\n")]
    shapes = {int(m.group(1).split(", ")[0]): m.group(1).split(", ")[1:] for m in re.finditer(r"X\(([\d, ]+)\)", body)}
    print("| shape | cfg | tile (BM, BN, WM, WN, BK, NS) | N tiles | fetch MB | write MB | traffic / algorithmic | "
          "fetch / (input + weights) |")
    print("|---|---|---|---|---|---|---|---|")
    for pf, fdir, wdir in zip(args.plans[0::3], args.plans[1::3], args.plans[2::3]):
        plan = json.load(open(pf))
        n, cfgs = plan["passes"], plan["cfgs"]
        res = {}
        for counter, path in (("FETCH_SIZE", fdir), ("WRITE_SIZE", wdir)):
            segs = _segments(path, counter)
            if len(segs) != len(cfgs) * n + 1:
                raise SystemExit(f"{path}: {len(segs)} marker segments, expected {len(cfgs) * n + 1}")
            scale = plan["copy_bytes"] / sum(v for _, v in segs[-1])
            res[counter] = [statistics.median(sum(v for _, v in segs[i * n + p]) for p in range(n)) * scale
                            for i in range(len(cfgs))]
        k, st, H, cin, cout = plan["shape"]
        alg = plan["input_bytes"] + plan["weight_bytes"] + plan["output_bytes"] + plan["bias_bytes"]
        for i, c in enumerate(cfgs):
            t = shapes.get(c, ["?"] * 6)
            ntn = -(-cout // int(t[1])) if t[1] != "?" else "?"
            f, w = res["FETCH_SIZE"][i], res["WRITE_SIZE"][i]
            print(f"| {k}x{k} s{st} {cin}->{cout} @{H}, b{plan['batch']} | {c} | ({', '.join(t)}) | {ntn} | "
                  f"{f / 1e6:.1f} | {w / 1e6:.1f} | {(f + w) / alg:.2f}x | "
                  f"{f / (plan['input_bytes'] + plan['weight_bytes']):.2f}x |")


def _segments(path: str, counter: str, unit: float = 1024.0) -> list[list[tuple[str, float]]]:
    """Dispatches between marker pairs, in dispatch order: [[(kernel, value), ...], ...]; values
    times `unit` (the byte counters read KiB)."""
    f = path if path.endswith(".csv") else glob.glob(os.path.join(path, "*counter_collection.csv"))[0]
    per = {}
    for r in csv.DictReader(open(f)):
        if r["Counter_Name"] != counter:
            continue
        k = int(r["Dispatch_Id"])
        name, v = per.get(k, (r["Kernel_Name"], 0.0))
        per[k] = (name, v + float(r["Counter_Value"]))
    segs, cur = [], None
    for k in sorted(per):
        name, v = per[k]
        if "k_marker" in name:
            if cur is None:
                cur = []
            else:
                segs.append(cur)
                cur = None
        elif cur is not None:
            cur.append((name, v * unit))
    return segs


def _per_unit(plan: dict, path: str, counter: str) -> tuple[float, dict]:
    """(scale, {op tuple: (bytes per pass (median, scaled), kernel, unit record)}) of one run."""
    nu, passes = plan["num_units"], plan["passes"]
    segs = _segments(path, counter)
    if len(segs) != nu * passes + 1:
        raise SystemExit(f"{counter}: {len(segs)} marker segments, expected {nu * passes + 1}")
    scale = plan["copy_bytes"] / sum(v for _, v in segs[-1])   # the copy reads and writes copy_bytes
    out = {}
    for info in plan["units"]:
        u = info["unit"]
        vals = [sum(v for _, v in segs[p * nu + u]) for p in range(passes)]
        kernels = sorted({n.split("(")[0] for p in range(passes) for n, _ in segs[p * nu + u]})
        out[tuple(info["ops"])] = (statistics.median(vals) * scale, kernels, info)
    return scale, out


def summarize(args):
    fplan, wplan = json.load(open(args.plan)), json.load(open(args.write_plan or args.plan))
    fscale, fet = _per_unit(fplan, args.fetch, "FETCH_SIZE")
    wscale, wri = _per_unit(wplan, args.write, "WRITE_SIZE")
    rows, total_t, total_a, unpaired = [], 0.0, 0.0, []
    for ops, (fb, kern, info) in fet.items():
        if ops not in wri or wri[ops][2]["kernel"] != info["kernel"]:
            unpaired.append(info["first"])
            continue
        wb = wri[ops][0]
        t = fb + wb
        total_t += t
        total_a += info["bytes"]
        rows.append({"unit": info["unit"], "first_op": info["first"], "ops": info["ops"], "kernel": info["kernel"],
                     "class": info["class"], "dispatched": kern, "fetch_bytes": int(fb), "write_bytes": int(wb),
                     "traffic_bytes": int(t), "algorithmic_bytes": int(info["bytes"]),
                     "ratio": round(t / info["bytes"], 3) if info["bytes"] else None})
    out = {"model": fplan["model"], "batch": fplan["batch"], "passes": fplan["passes"],
           "scale": {"FETCH_SIZE": round(fscale, 4), "WRITE_SIZE": round(wscale, 4),
                     "reference": f"copy of {int(fplan['copy_bytes'])} bytes read + written"},
           "total_traffic_bytes": int(total_t), "total_algorithmic_bytes": int(total_a),
           "unpaired_first_ops": unpaired, "per_unit": rows}
    if args.md:
        _markdown(out, args)
    # the committed figures: one compact row per unit, keyed by its first op
    slim = {k: out[k] for k in ("model", "batch", "passes", "scale", "total_traffic_bytes",
                                "total_algorithmic_bytes", "unpaired_first_ops")}
    slim["columns"] = ["kernel", "class", "fetch_bytes", "write_bytes", "traffic_bytes", "algorithmic_bytes"]
    slim["per_unit_first_op"] = {str(r["first_op"]): [r[c] for c in slim["columns"]] for r in rows}
    with open(args.json, "w") as f:
        json.dump(slim, f, separators=(",", ":"))


def _markdown(out, args):
    classes = {}
    for r in out["per_unit"]:
        c = classes.setdefault(r["class"] or r["kernel"], [0, 0, 0])
        c[0] += 1
        c[1] += r["traffic_bytes"]
        c[2] += r["algorithmic_bytes"]
    lines = [f"# HBM traffic per launch unit: {out['model']} detect, batch {out['batch']}", "",
             "Two `rocprofv3 --pmc` passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch) over every launch",
             "unit of the frame, each unit between two marker kernels; median over "
             f"{out['passes']} passes.  Each counter is scaled by what it reads for a plain copy of known size",
             f"in the same run (FETCH_SIZE x {out['scale']['FETCH_SIZE']}, WRITE_SIZE x {out['scale']['WRITE_SIZE']}).",
             "Algorithmic bytes: input + weights + output (+ residual) per conv, inputs + outputs",
             "elsewhere (yolo11.cu_amd/unitwork.py).", "", "```",
             "OUT=out/traffic_x",
             "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/fetch -o run -- python3 yolo11.cu_amd/profiling.py "
             f"collect --scale {out['model'][-1]} --batch {out['batch']} --passes {out['passes']} --plan $OUT/plan.json",
             "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/write -o run -- python3 yolo11.cu_amd/profiling.py "
             f"collect --scale {out['model'][-1]} --batch {out['batch']} --passes {out['passes']} --plan $OUT/wplan.json "
             "--replay $OUT/plan.json",
             "python3 yolo11.cu_amd/profiling.py summarize --plan $OUT/plan.json --write-plan $OUT/wplan.json "
             f"--fetch $OUT/fetch --write $OUT/write --json {args.json} --md {args.md}", "```", "",
             f"Whole frame: {out['total_traffic_bytes'] / 1e9:.2f} GB moved against "
             f"{out['total_algorithmic_bytes'] / 1e9:.2f} GB algorithmic "
             f"({out['total_traffic_bytes'] / out['total_algorithmic_bytes']:.2f}x), over the units both passes ran "
             "with the same ops and kernel (left out, by first op: "
             f"{', '.join(map(str, out['unpaired_first_ops'])) or 'none'}).", "",
             "| class | units | traffic GB | algorithmic GB | ratio |", "|---|---|---|---|---|"]
    for name, (n, t, a) in sorted(classes.items(), key=lambda kv: -kv[1][1]):
        lines.append(f"| {name} | {n} | {t / 1e9:.3f} | {a / 1e9:.3f} | {t / a:.2f} |" if a else
                     f"| {name} | {n} | {t / 1e9:.3f} | - | - |")
    lines += ["", "Units moving the most bytes:", "",
              "| unit | first op | kernel | class | traffic MB | algorithmic MB | ratio |", "|---|---|---|---|---|---|---|"]
    for r in sorted(out["per_unit"], key=lambda r: -r["traffic_bytes"])[:30]:
        lines.append(f"| {r['unit']} | {r['first_op']} | {r['kernel']} | {r['class']} | {r['traffic_bytes'] / 1e6:.1f} | "
                     f"{r['algorithmic_bytes'] / 1e6:.1f} | {r['ratio']} |")
    open(args.md, "w").write("\n".join(lines) + "\n")


def mfma(args):
    """Matrix-pipe occupancy per launch unit, from a `collect` run under
    `rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE`.  SQ_VALU_MFMA_BUSY_CYCLES adds each
    MFMA's pipe cycles on its SIMD: 16 for a v_mfma_f32_16x16x32_f16 (16,384 FLOPs), so busy x
    1,024 is the FLOP count the MFMAs executed, padded rows and channels included.
    GRBM_GUI_ACTIVE adds the dispatch's cycles over the XCDs, so GUI_ACTIVE / XCDs x SIMDs is
    the SIMD-cycles the dispatch held; busy over that is the matrix pipe's share of them, the
    MFMA utilisation at the clock the dispatch ran at (dispatches run one at a time under the
    counters)."""
    plan = json.load(open(args.plan))
    nu, passes = plan["num_units"], plan["passes"]
    agent = glob.glob(os.path.join(args.pmc, "*agent_info.csv"))
    gpu = next(r for r in csv.DictReader(open(agent[0])) if r.get("Name", "").startswith("gfx"))
    simds, xcds = int(gpu["Simd_Count"]), int(gpu["Num_Xcc"])
    busy = _segments(args.pmc, "SQ_VALU_MFMA_BUSY_CYCLES", 1.0)
    act = _segments(args.pmc, "GRBM_GUI_ACTIVE", 1.0)
    for segs in (busy, act):
        if len(segs) != nu * passes + 1:
            raise SystemExit(f"{len(segs)} marker segments, expected {nu * passes + 1}")
    classes, rows = {}, []
    for info in plan["units"]:
        if not info["flops"]:
            continue
        u = info["unit"]
        b = statistics.median(sum(v for _, v in busy[p * nu + u]) for p in range(passes))
        a = statistics.median(sum(v for _, v in act[p * nu + u]) for p in range(passes))
        cyc = a / xcds * simds
        name = "attention" if info["kernel"].startswith("k_attention") else info["class"]
        c = classes.setdefault(name, [0, 0.0, 0.0, 0.0])
        c[0] += 1
        c[1] += info["flops"]
        c[2] += b * 1024.0
        c[3] += cyc
        rows.append((info["first"], info["kernel"], info["class"], info["flops"], b * 1024.0, cyc))
    conv = [v for k, v in classes.items() if k != "attention"]
    tf, te, tc = (sum(v[i] for v in conv) for i in (1, 2, 3))
    lines = [f"# Matrix-pipe occupancy per launch unit: {plan['model']} detect, batch {plan['batch']}", "",
             "One `rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE` pass over every launch unit of",
             f"the frame (each unit between two marker kernels, median over {passes} passes; dispatches run",
             "one at a time under the counters).  Executed = busy cycles x 1,024 FLOPs (a",
             "v_mfma_f32_16x16x32_f16 holds its SIMD's matrix pipe 16 cycles for 16,384 FLOPs), padding",
             "included; algorithmic = `2*B*Ho*Wo*Cout*k^2*Cin/g` (yolo11.cu_amd/unitwork.py).  Busy share =",
             f"busy / (GRBM_GUI_ACTIVE / {xcds} XCDs x {simds} SIMDs), the MFMA utilisation at the clock the",
             "dispatch ran at (algorithmic share: the same with algorithmic FLOPs).", "", "```",
             f"OUT=out/mfma_{plan['model'][-1]}",
             "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE --output-format csv -d $OUT/pmc -o run -- "
             f"python3 yolo11.cu_amd/profiling.py collect --scale {plan['model'][-1]} --batch {plan['batch']} "
             f"--passes {passes} --plan $OUT/plan.json",
             f"python3 yolo11.cu_amd/profiling.py mfma --plan $OUT/plan.json --pmc $OUT/pmc --md {args.md}", "```", "",
             f"Conv units: {tf / 1e12:.3f} TFLOP algorithmic, {te / 1e12:.3f} TFLOP executed "
             f"({te / tf:.3f}x); matrix pipe busy {te / 1024 / tc:.3f} of the SIMD-cycles "
             f"(algorithmic {tf / 1024 / tc:.3f}).", "",
             "| class | units | algorithmic GFLOP | executed GFLOP | executed / algorithmic | busy share | "
             "algorithmic share |", "|---|---|---|---|---|---|---|"]
    for name, (n, f, e, c) in sorted(classes.items(), key=lambda kv: -kv[1][3]):
        lines.append(f"| {name} | {n} | {f / 1e9:.1f} | {e / 1e9:.1f} | {e / f:.3f} | {e / 1024 / c:.3f} | "
                     f"{f / 1024 / c:.3f} |")
    lines += ["", "Units holding the most SIMD-cycles:", "",
              "| first op | kernel | class | algorithmic GFLOP | executed / algorithmic | busy share |",
              "|---|---|---|---|---|---|"]
    for first, kern, cls, f, e, c in sorted(rows, key=lambda r: -r[5])[:args.top]:
        lines.append(f"| {first} | {kern} | {cls} | {f / 1e9:.2f} | {e / f:.3f} | {e / 1024 / c:.3f} |")
    text = "\n".join(lines) + "\n"
    if args.md:
        open(args.md, "w").write(text)
    print(text)


def trace(args):
    """Steady-state kernel time per frame from a `rocprofv3 --kernel-trace` CSV of
    `bench.py --only <n|x> --no-graph` (stream-ordered launches of the frame's kernels): every
    dispatch from the first letterbox on (after load and autotune), grouped by kernel; GEMM
    and streaming-conv instantiations labelled with their op config numbers."""
    import re
    f = args.csv if args.csv.endswith(".csv") else glob.glob(os.path.join(args.csv, "*kernel_trace.csv"))[0]
    rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Start_Timestamp"]))
    src = open(os.path.join(HERE, "csrc", "conv.hip")).read()
    def table(macro):   # the X(...) rows of one tile table: index -> the template arguments
        body = src[src.index(f"#define {macro}("):]
        body = body[:body.index("\n\n")]
        return {tuple(map(int, m.group(1).split(", ")[1:])): int(m.group(1).split(", ")[0])
                for m in re.finditer(r"X\(([\d, ]+)\)", body)}
    tiles, taps, wstaps = table("YOLO_TILES"), table("YOLO_TAP_TILES"), table("YOLO_TAPWS_TILES")
    km = {0: "1x1", 1: "uni", 2: "gen"}

    def demangle(name):
        # kernels whose trace name stays mangled: yolo::<kernel><integer/bool template args>
        m = re.match(r"_ZN4yolo(\d+)", name)
        if not m:
            return name
        n0 = m.end()
        ident = name[n0:n0 + int(m.group(1))]
        targs = re.match(r"I((?:L[ib]-?\d+E)+)E", name[n0 + len(ident):])
        if not targs:
            return f"yolo::{ident}"
        vals = re.findall(r"L([ib])(-?\d+)E", targs.group(1))
        return f"yolo::{ident}<{', '.join(v if t == 'i' else ('true' if v == '1' else 'false') for t, v in vals)}>"

    def label(name):
        name = demangle(name.split("(")[0])
        m = re.search(r"k_conv_gemm<(\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d)>", name)
        if m:
            v = tuple(map(int, m.groups()))
            return f"{name} [cfg {tiles.get(v[:6], '?')} {km[v[6]]}]"
        m = re.search(r"k_conv_tapws<(\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+)>", name)
        if m:
            return f"{name} [op config {1200 + wstaps.get(tuple(map(int, m.groups())), -1200)}]"
        m = re.search(r"k_conv_tap<(\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+)>", name)
        if m:
            return f"{name} [op config {1100 + taps.get(tuple(map(int, m.groups())), -1100)}]"
        return name
    start = next(i for i, r in enumerate(rows) if "letterbox" in r["Kernel_Name"])
    rows = rows[start:]
    agg: dict = {}
    for r in rows:
        agg.setdefault(label(r["Kernel_Name"]), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    tot = sum(sum(v) for v in agg.values())
    frames = sum(1 for r in rows if "letterbox" in r["Kernel_Name"]) // args.letterboxes_per_frame
    print(" calls   total_us    avg_us   min_us   max_us    pct  kernel")
    for name, v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:args.top]:
        print(f"{len(v):6d} {sum(v):10.1f} {sum(v) / len(v):9.2f} {min(v):8.2f} {max(v):8.2f} "
              f"{100 * sum(v) / tot:6.2f}  {name[:110]}")
    print(f"steady-state kernel time {tot / 1e3:.3f} ms over {len(rows)} dispatches, {frames} frames: "
          f"{tot / 1e3 / max(frames, 1):.4f} ms and {len(rows) / max(frames, 1):.0f} dispatches per frame")


def conv_roofline(scale: str = "x", batch: int = 16, peak: float = 2.5e15, bw: float = 6.3e12,
                  fracs=(0.44, 0.6)) -> dict:
    """Per-layer roofline of a model's convs at a batch size, from the generator's op graph
    (CPU only).  Each conv takes max(FLOPs / peak, bytes / bw), its bytes counted as unitwork
    counts them (input, weights, output, the residual a following ADD fuses in, fp32 bias);
    bw defaults to the copy rate measured on MI355X (6.3 TB/s, read + write).  The ratio of all
    conv FLOPs to the summed per-layer times, over the peak, is the conv MFMA utilisation a
    frame could reach with every conv at its own roofline.  For each f in `fracs` the same
    with MFMA-bound layers at f of the peak (0.44: the best GEMM tile's main loop streaming
    from HBM, measured in isolation)."""
    import modelgen
    g = modelgen.build_model("yolo11", scale, calibrate=False).graph
    ops = g.ops
    flops = nbytes = t_roof = 0.0
    t_frac = {f: 0.0 for f in fracs}
    mfma_bound = 0
    for i, op in enumerate(ops):
        if op[0] != "CONV":
            continue
        _, x, out, k, _s, _p, grp, _act, cin, cout = op[:10]
        H, W, _ = g.shape(x)
        Ho, Wo, _ = g.shape(out)
        f = 2.0 * batch * Ho * Wo * cout * k * k * cin / grp
        out_px = batch * Ho * Wo * cout
        b = 2.0 * (batch * H * W * cin + cout * k * k * cin / grp + out_px) + 4.0 * cout
        nx = ops[i + 1] if i + 1 < len(ops) else None
        if nx is not None and nx[0] == "ADD" and out in (nx[1], nx[2]):
            b += 2.0 * out_px   # the residual read of the fused add
        flops += f
        nbytes += b
        t_roof += max(f / peak, b / bw)
        mfma_bound += f / peak >= b / bw
        for fr in fracs:
            t_frac[fr] += max(f / (peak * fr), b / bw)
    return {"scale": scale, "batch": batch, "convs": sum(op[0] == "CONV" for op in ops),
            "mfma_bound": mfma_bound, "tflop": flops / 1e12, "gbytes": nbytes / 1e9,
            "roofline_ms": t_roof * 1e3, "util": flops / t_roof / peak,
            "at_frac": {str(fr): {"ms": t * 1e3, "util": flops / t / peak} for fr, t in t_frac.items()}}


def ceiling(args):
    r = conv_roofline(args.scale, args.batch)
    print(f"yolo11{r['scale']} b{r['batch']}: {r['convs']} convs ({r['mfma_bound']} MFMA-bound), "
          f"{r['tflop']:.3f} TFLOP, {r['gbytes']:.2f} GB; every conv at its roofline: {r['roofline_ms']:.3f} ms, "
          f"conv MFMA util {r['util']:.3f}")
    for fr, v in r["at_frac"].items():
        print(f"  MFMA-bound convs at {fr} of the peak: {v['ms']:.3f} ms, util {v['util']:.3f}")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("collect")
    c.add_argument("--scale", default="x")
    c.add_argument("--batch", type=int, default=16)
    c.add_argument("--passes", type=int, default=3)
    c.add_argument("--plan", required=True, help="where this run writes its plan")
    c.add_argument("--replay", help="a first run's plan whose kernel choices this run takes")
    s = sub.add_parser("summarize")
    s.add_argument("--plan", required=True, help="the FETCH_SIZE run's plan")
    s.add_argument("--write-plan", help="the WRITE_SIZE run's plan (default: --plan)")
    s.add_argument("--fetch", required=True)
    s.add_argument("--write", required=True)
    s.add_argument("--json", required=True)
    s.add_argument("--md")
    ti = sub.add_parser("tiles")
    ti.add_argument("--shape", type=int, nargs=5, required=True, metavar=("K", "S", "H", "CIN", "COUT"))
    ti.add_argument("--batch", type=int, default=16)
    ti.add_argument("--cfgs", type=int, nargs="+", required=True)
    ti.add_argument("--passes", type=int, default=3)
    ti.add_argument("--plan", required=True)
    ts = sub.add_parser("tiles-summary")
    ts.add_argument("plans", nargs="+", help="triples: plan.json, FETCH_SIZE dir, WRITE_SIZE dir")
    mf = sub.add_parser("mfma")
    mf.add_argument("--plan", required=True, help="the collect run's plan")
    mf.add_argument("--pmc", required=True, help="its rocprofv3 output directory")
    mf.add_argument("--md")
    mf.add_argument("--top", type=int, default=20)
    ce = sub.add_parser("ceiling", help="per-layer roofline of the convs (CPU only)")
    ce.add_argument("--scale", default="x")
    ce.add_argument("--batch", type=int, default=16)
    t = sub.add_parser("trace")
    t.add_argument("csv", help="a rocprofv3 kernel_trace.csv, or the directory holding it")
    t.add_argument("--letterboxes-per-frame", type=int, default=1)
    t.add_argument("--top", type=int, default=32)
    args = ap.parse_args()
    {"collect": collect, "summarize": summarize, "trace": trace, "tiles": tiles,
     "tiles-summary": tiles_summary, "mfma": mfma, "ceiling": ceiling}[args.cmd](args)


if __name__ == "__main__":
    main()
