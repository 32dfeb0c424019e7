#!/usr/bin/env python3
"""Benchmark of the YOLO frame path on one MI355X -> one JSON line on stdout.

Workloads (BASELINE.json metric "e2e ms/frame & FPS @640 fp16 (yolo11n b1, yolo11x b16);
conv MFMA util %"):
  * primary (value): yolo11n detect, batch 1, 810x1080 synthetic BGR frame in pinned host
    memory; one step = one launch of the whole-frame graph (H2D of the raw frame +
    letterbox + net + DFL decode + NMS + D2H of the results into pinned memory) + wait +
    host fetch of the detections: the loop of the reference's `pipeline` mode
    (engine/engine.cu:1992-2031).  The same loop with the frame already in HBM is a side
    figure.
  * yolo11x detect, batch 16, sixteen 640x640 frames in HBM: whole-frame graph
    throughput, and conv MFMA utilisation = sum(conv FLOPs) / (sum(conv kernel time) * peak),
    the kernel time of each launch unit (one conv or a grouped launch, as the graph runs
    them) from hipEvents around 5 back-to-back launches; the same ratio with stream-ordered
    per-op events (launch gaps included) is reported beside it.
  * roofline: the implicit-GEMM conv kernel on the isolated-conv-sweep shape
    3x3 s1 256->256 @80x80, batch 32, as the autotuner configures it
    (tile, and the tail retile's second dispatch where it picked one), timed with hipEvents
    on the engine stream around 5 back-to-back launches; `traffic` = HBM bytes per launch of
    that configuration, from the committed PMC passes (profiles/conv_gemm_c1_traffic.json).
  * prepost_roofline: letterbox, decode and mask assembly against the HBM roofline, NMS time.
  * yolo11n-obb at 1024 (15 classes, 1024x1024 frame) and yolo11n-seg at 640, batch 1:
    whole-frame graph, frame in HBM (side figures; the reference quotes 1.6 ms and 1.21 ms
    on an RTX 3060 Ti, README.md:80-81).
  * yolo11m detect b1 with a 1080x1920 frame at IoU 0.7 (H2D included),
    the five isolated conv shapes at batch 1 and 32 (config 1), and yolo11n-cls at 224
    (whole-frame graph with the classify preprocess): side figures.
  * cpu_baseline: the reference's CPU path, a torch fp32 per-op interpreter of the graph
    plus CPU letterbox/decode/NMS (oracle/torchref.py), for yolo11n batch 1 on this host's
    cores, in a separate process, bounded to ~15 s.

Weights are seeded random-init (no checkpoints offline); data are synthetic frames.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "yolo11.cu_amd"))
sys.path.insert(0, ROOT)

from unitwork import conv_kernel_name, unit_table, units as unit_list  # noqa: E402  (the package dir is on sys.path)

PEAK_FP16 = 2.5e15        # MI355X dense fp16 MFMA, FLOP/s
PEAK_HBM = 8.0e12         # MI355X HBM3E, B/s


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic(cfg, tail=-1):
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 PMC passes
    (FETCH_SIZE and WRITE_SIZE per tile config, or per tile + tail-retile pair summed over
    its two dispatches, each scaled by a plain copy of known size) for the configuration this
    run's autotuner picked; None if it has no measurement."""
    path = os.path.join(ROOT, "profiles", "conv_gemm_c1_traffic.json")
    try:
        rec = json.load(open(path))
        if tail >= 0:
            return int(rec["per_retile"][f"{cfg}+{tail}"]["traffic_bytes"])
        return int(rec["per_cfg"][str(cfg)]["traffic_bytes"])
    except (OSError, ValueError, KeyError):
        return None


def measured_x_traffic(firsts, kernel):
    """(HBM bytes per batch, same kernels) of the yolo11x b16 launch units whose first ops are
    `firsts`: FETCH_SIZE + WRITE_SIZE of their dispatches in the committed PMC passes of
    profiling.py, each scaled by a plain copy of known size; `same kernels` says whether that
    run's autotuner chose this run's kernel for every one of them (it times candidates, so
    two runs can differ).  None where the passes have no figure for one of them."""
    path = os.path.join(ROOT, "profiles", "yolo11x_b16_traffic.json")
    try:
        tab = json.load(open(path))
        col = {c: i for i, c in enumerate(tab["columns"])}
        rec = tab["per_unit_first_op"]
        same = all(rec[str(k)][col["kernel"]] == kernel for k in firsts)
        return int(sum(rec[str(k)][col["traffic_bytes"]] for k in firsts)), same
    except (OSError, ValueError, KeyError):
        return None


def conv_flops(eng, k):
    info = eng.op_info(k)
    H, W, _ = eng.tensor_shape(info["out"])
    return 2.0 * H * W * info["Cout"] * info["k"] * info["k"] * info["Cin"] / max(info["g"], 1)


def group_roofline(g, traffic=None):
    """Roofline entry of a kernel group: MFMA-bound when its arithmetic intensity is above
    the chip's ratio (2.5 PFLOP/s / 8 TB/s = 312.5 FLOP/B), HBM-bound below."""
    ai = g["flops"] / g["bytes"] if g["bytes"] else 0.0
    sec = g["ms"] * 1e-3
    if ai >= PEAK_FP16 / PEAK_HBM:
        ach = g["flops"] / sec
        r = {"bound": "mfma", "achieved": round(ach / 1e12, 2), "peak": 2500.0, "unit": "TFLOP/s",
             "frac": round(ach / PEAK_FP16, 4)}
    else:
        ach = g["bytes"] / sec
        r = {"bound": "hbm", "achieved": round(ach / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
             "frac": round(ach / PEAK_HBM, 4), "tflops": round(g["flops"] / sec / 1e12, 1)}
    r.update({"traffic": traffic, "kernel": g["kernel"], "class": g["class"], "launches": g["launches"],
              "ms": round(g["ms"], 4), "flops": g["flops"], "bytes": g["bytes"], "ai": round(ai, 1)})
    return r


def attn_flops(eng, k):
    """QK^T and PV of one image: 2 * heads * N^2 * (kd + hd), kd = 32 (the loader's rule);
    heads and hd follow from the qkv width heads * (2 kd + hd) and the output width heads * hd."""
    info = eng.op_info(k)
    H, W, cout = eng.tensor_shape(info["out"])
    cin = eng.tensor_shape(info["a"])[2]
    heads = (cin - cout) // 64
    hd = cout // heads
    n = H * W
    return 2.0 * heads * n * n * (32 + hd)


def bench_n(workdir, steps, warmup, graph=True):
    """yolo11n b1.  The headline step is the reference's `pipeline` loop
    (engine/engine.cu:1992-2031): one whole-frame graph holding the H2D of the raw 810x1080
    frame from pinned host memory, letterbox, network, decode, NMS and the result copy, then
    a wait and the host fetch of the detections.  The same loop with the frame already in
    HBM, the graph alone (hipEvents), and the pre/post stages are side figures."""
    import modelgen
    import yolort
    d = os.path.join(workdir, "yolo11n")
    modelgen.write_model(d, "yolo11", "n", cls_bias=-8.0)
    img = modelgen.synth_frame(810, 1080, 20, 1)
    eng = yolort.Engine(d, 1, 0 if graph else yolort.YOLO_NOGRAPH)
    dev = yolort.DeviceBuffer(img.nbytes)
    eng.upload(dev, img)
    if not graph:   # stream-ordered launches of the same kernels (for profilers)
        for _ in range(warmup + steps):
            eng.preprocess(dev.ptr, 810, 1080, 0)
            eng.run(1)
            eng.get(0)
        dev.free()
        eng.close()
        return None

    def loop():
        for _ in range(warmup):
            eng.frame_run()
            eng.get(0)
        t0 = time.perf_counter()
        for _ in range(steps):
            eng.frame_run()
            dets = eng.get(0)
        return (time.perf_counter() - t0) * 1e3 / steps, dets

    # frame already in HBM
    eng.frame_graph([dev.ptr], [810], [1080])
    ms_hbm, _ = loop()
    graph_ms_hbm = eng.time_graph(1, 1, max(steps, 50))
    stages = eng.profile_stages(50)
    # headline: the raw frame is uploaded from pinned memory inside the graph
    pin = yolort.PinnedBuffer(img.shape)
    pin.array[...] = img
    eng.frame_graph([dev.ptr], [810], [1080], [pin.ptr])
    ms, dets = loop()
    graph_ms = eng.time_graph(1, 1, max(steps, 50))
    kept, raw = len(dets), eng.raw_count(0)
    per_op = eng.profile_ops(1, 20)
    # attribution of the graph's time: every launch unit timed with hipEvents around 5
    # back-to-back launches (no host gap), grouped by kernel
    per_unit = eng.profile_units(1, 20, 5)
    units = unit_table(eng, 1, per_unit)
    pin.free()
    dev.free()
    eng.close()
    return dict(ms=ms, graph_ms=graph_ms, ms_hbm=ms_hbm, graph_ms_hbm=graph_ms_hbm, kept=kept, raw=raw,
                stream_ops_ms=float(per_op.sum()), stages=stages, frame=(810, 1080), A=8400, ncpad=80,
                units=units, units_ms=float(sum(g["ms"] for g in units)),
                launches=int(sum(g["launches"] for g in units)))


def bench_task(workdir, task, imgsz, nc, cls_bias, frame, steps, warmup, graph=True):
    """yolo11n of another task head at batch 1: the whole-frame graph (letterbox + net +
    decode + NMS [+ masks] + result copy) with the raw frame in HBM, like bench_n."""
    import modelgen
    import yolort
    d = os.path.join(workdir, f"yolo11n-{task}")
    modelgen.write_model(d, "yolo11", "n", task, nc, imgsz, 0, cls_bias)
    eng = yolort.Engine(d, 1, 0 if graph else yolort.YOLO_NOGRAPH)
    dev = yolort.DeviceBuffer(frame.nbytes)
    eng.upload(dev, frame)
    h, w = frame.shape[:2]
    get = eng.get_obb if task == "obb" else eng.get
    if not graph:
        for _ in range(warmup + steps):
            eng.preprocess(dev.ptr, h, w, 0)
            eng.run(1)
            get(0)
        dev.free()
        eng.close()
        return None
    eng.frame_graph([dev.ptr], [h], [w])
    for _ in range(warmup):
        eng.frame_run()
        get(0)
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.frame_run()
        dets = get(0)
    ms = (time.perf_counter() - t0) * 1e3 / steps
    graph_ms = eng.time_graph(1, 1, max(steps, 50))
    kept, raw = len(dets), eng.raw_count(0)
    stages = eng.profile_stages(50)
    dev.free()
    eng.close()
    return dict(ms=ms, graph_ms=graph_ms, kept=kept, raw=raw, stages=stages)


def bench_m(workdir, steps, warmup, graph=True):
    """yolo11m detect b1, a 1080x1920 synthetic frame in HBM, whole-frame
    graph (letterbox + net + DFL decode + NMS at conf 0.25 / IoU 0.7 / max 300)."""
    import modelgen
    import yolort
    d = os.path.join(workdir, "yolo11m")
    modelgen.write_model(d, "yolo11", "m", cls_bias=-8.0)
    img = modelgen.synth_frame(1080, 1920, 20, 2)
    eng = yolort.Engine(d, 1, 0 if graph else yolort.YOLO_NOGRAPH)
    eng.set_thresholds(0.25, 0.7, 300)
    dev = yolort.DeviceBuffer(img.nbytes)
    eng.upload(dev, img)
    if not graph:
        for _ in range(warmup + steps):
            eng.preprocess(dev.ptr, 1080, 1920, 0)
            eng.run(1)
            eng.get(0)
        dev.free()
        eng.close()
        return None
    def loop():
        for _ in range(warmup):
            eng.frame_run()
            eng.get(0)
        t0 = time.perf_counter()
        for _ in range(steps):
            eng.frame_run()
            dets = eng.get(0)
        return (time.perf_counter() - t0) * 1e3 / steps, dets

    eng.frame_graph([dev.ptr], [1080], [1920])
    ms_hbm, _ = loop()
    pin = yolort.PinnedBuffer(img.shape)
    pin.array[...] = img
    eng.frame_graph([dev.ptr], [1080], [1920], [pin.ptr])
    ms, dets = loop()
    graph_ms = eng.time_graph(1, 1, max(steps, 50))
    kept, raw = len(dets), eng.raw_count(0)
    pin.free()
    dev.free()
    eng.close()
    return dict(ms=ms, graph_ms=graph_ms, ms_hbm=ms_hbm, kept=kept, raw=raw)


def bench_cls(workdir, steps, warmup, graph=True):
    """yolo11n-cls (1000 classes) at 224, batch 1: whole-frame graph (antialiased resize +
    centre crop of an 810x1080 frame in HBM, network, probabilities copy) + top-5 fetch."""
    import modelgen
    import yolort
    d = os.path.join(workdir, "yolo11n-cls")
    modelgen.write_model(d, "yolo11", "n", "classify", 1000, 224, 0)
    img = modelgen.synth_frame(810, 1080, 20, 1)
    eng = yolort.Engine(d, 1, 0 if graph else yolort.YOLO_NOGRAPH)
    dev = yolort.DeviceBuffer(img.nbytes)
    eng.upload(dev, img)
    if not graph:
        for _ in range(warmup + steps):
            eng.preprocess_cls(dev.ptr, 810, 1080, 0)
            eng.run(1)
            eng.get_cls(0, 5)
        dev.free()
        eng.close()
        return None
    eng.frame_graph([dev.ptr], [810], [1080])
    for _ in range(warmup):
        eng.frame_run()
        eng.get_cls(0, 5)
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.frame_run()
        ids, _ = eng.get_cls(0, 5)
    ms = (time.perf_counter() - t0) * 1e3 / steps
    graph_ms = eng.time_graph(1, 1, max(steps, 50))
    dev.free()
    eng.close()
    return dict(ms=ms, graph_ms=graph_ms, top1=int(ids[0]))


def bench_sweep(workdir, iters):
    """the five isolated conv shapes at batch 1 and 32 (autotuned tile and
    split), TFLOP/s per shape from hipEvent timing on the engine stream."""
    import numpy as np
    import modelgen
    import yolort
    shapes = [(80, 80, 256, 256, 3, 1), (80, 80, 256, 512, 3, 2), (40, 40, 512, 256, 1, 1),
              (20, 20, 512, 512, 3, 1), (20, 20, 1024, 512, 1, 1)]
    out = {}
    for (H, W, cin, cout, k, s) in shapes:
        d = os.path.join(workdir, f"sweep_{H}_{cin}_{cout}_{k}_{s}")
        modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=7)
        Ho, Wo = (H + 2 * (k // 2) - k) // s + 1, (W + 2 * (k // 2) - k) // s + 1
        for B in (1, 32):
            eng = yolort.Engine(d, B, yolort.YOLO_NOGRAPH)
            x = np.random.default_rng(11).standard_normal((B, H, W, cin), dtype=np.float32).astype(np.float16)
            eng.write(0, x)
            ms = float(eng.profile_ops(B, iters)[0])
            fl = 2.0 * B * Ho * Wo * cout * k * k * cin
            out[f"{k}x{k}s{s} {cin}->{cout} @{H}x{W} b{B}"] = {
                "us": round(ms * 1e3, 2), "tflops": round(fl / ms / 1e9, 1),
                "tile": eng.op_config(0), "split": eng.op_split(0), "tail": eng.op_tail(0)}
            eng.close()
    return out


def bench_x(workdir, iters, graph=True):
    import modelgen
    import yolort
    d = os.path.join(workdir, "yolo11x")
    t0 = time.perf_counter()
    modelgen.write_model(d, "yolo11", "x", cls_bias=-8.0)
    log(f"yolo11x generated in {time.perf_counter() - t0:.1f}s")
    B = 16
    t0 = time.perf_counter()
    eng = yolort.Engine(d, B, yolort.YOLO_NOGRAPH)
    log(f"yolo11x engine (autotune) ready in {time.perf_counter() - t0:.1f}s")
    frames = [modelgen.synth_frame(640, 640, 50, 100 + i) for i in range(B)]
    devs = [yolort.DeviceBuffer(f.nbytes) for f in frames]
    for b, f in zip(devs, frames):
        eng.upload(b, f)
    if not graph:
        for _ in range(iters):
            for s, b in enumerate(devs):
                eng.preprocess(b.ptr, 640, 640, s)
            eng.run(B)
        for b in devs:
            b.free()
        eng.close()
        return None
    eng.frame_graph([b.ptr for b in devs], [640] * B, [640] * B)
    for _ in range(3):
        eng.frame_run()
    ms = eng.time_graph(1, B, iters)
    kept = [len(eng.get(s)) for s in range(B)]
    per_op = eng.profile_ops(B, max(3, iters // 4))
    # kernel time per launch unit (grouped launches as the graph runs them), each unit run
    # 5 times back to back so the per-launch gaps of a stream-ordered pass are excluded
    per_unit = eng.profile_units(B, 2, 5)
    conv_f, conv_t, conv_t_ev, attn_t, attn_f = 0.0, 0.0, 0.0, 0.0, 0.0
    for k in range(eng.num_ops):
        info = eng.op_info(k)
        if info["kind"] == "CONV":
            conv_f += B * conv_flops(eng, k)
            conv_t += per_unit[k] * 1e-3
            conv_t_ev += per_op[k] * 1e-3
        elif info["kind"] == "ATTN":
            attn_f += B * attn_flops(eng, k)
    # an attention launch may carry its block's V-gather copies: the unit's time (reported
    # on its first op, a copy then) counts as attention time
    for u in unit_list(eng, B):
        if any(eng.op_info(k)["kind"] == "ATTN" for k in u["ops"]):
            attn_t += per_unit[u["first"]] * 1e-3
    units = unit_table(eng, B, per_unit)
    top = next(g for g in units if g["class"])          # the conv kernel group with the most time
    mt = measured_x_traffic(top["firsts"], top["kernel"])
    for b in devs:
        b.free()
    eng.close()
    dominant = group_roofline(top, mt[0] if mt else None)
    dominant["traffic_same_kernels"] = mt[1] if mt else None
    return dict(dominant=dominant, units=units[:12],
                ms_per_batch=ms, img_per_s=B * 1e3 / ms, conv_tflops=conv_f / conv_t / 1e12,
                conv_mfma_util=conv_f / conv_t / PEAK_FP16, conv_ms=conv_t * 1e3,
                conv_mfma_util_stream_events=conv_f / conv_t_ev / PEAK_FP16, conv_ms_stream_events=conv_t_ev * 1e3,
                attn_ms=attn_t * 1e3, attn_tflops=attn_f / attn_t / 1e12, attn_mfma_util=attn_f / attn_t / PEAK_FP16,
                stream_ops_ms=float(per_op.sum()), kept_min=min(kept),
                kept_max=max(kept))


def bench_conv(workdir, iters):
    import numpy as np
    import modelgen
    import yolort
    d = os.path.join(workdir, "conv_c1")
    H, W, cin, cout, k, s, B = 80, 80, 256, 256, 3, 1, 32
    modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=7)
    eng = yolort.Engine(d, B, yolort.YOLO_NOGRAPH)
    x = np.random.default_rng(11).standard_normal((B, H, W, cin), dtype=np.float32).astype(np.float16)
    eng.write(0, x)
    # kernel time per launch (both dispatches of a tail retile): 5 back-to-back launches timed
    # with HIP events on the engine stream, averaged over `iters` rounds
    ms = float(eng.profile_units(B, iters, 5)[0])
    flops = 2.0 * B * H * W * cout * k * k * cin
    # algorithmic HBM bytes: input + weights + output (fp16) + bias (fp32)
    nbytes = 2.0 * (B * H * W * cin + cout * k * k * cin + B * H * W * cout) + 4 * cout
    cfg = eng.op_config(0)
    tail = eng.op_tail(0)
    eng.close()
    # a plain copy of known size on the same shape (scale reference for HBM counters)
    dc = os.path.join(workdir, "copy_c1")
    modelgen.write_copy(dc, H, W, cin)
    ec = yolort.Engine(dc, B, yolort.YOLO_NOGRAPH)
    copy_ms = float(ec.profile_units(B, iters, 5)[0])
    ec.close()
    copy_bytes = 2.0 * 2 * B * H * W * cin
    return dict(ms=ms, flops=flops, bytes=nbytes, tflops=flops / ms / 1e9, cfg=cfg, tail=tail,
                shape=f"3x3 s1 {cin}->{cout} @{H}x{W} b{B}", copy_ms=copy_ms,
                copy_gbs=copy_bytes / copy_ms / 1e6)


def bench_serve(workdir, seconds=4.0, procs=4, callers=16, frontends=4):
    """The gRPC server (yoloserve) with yolo11n, max batch 16, target 50 ms (the reference
    server's defaults, server/serve.cpp:344-346), JPEG decoded on the engine (entropy decoding
    on the library's decoder threads, the rest on the GPU), the gRPC service in `frontends`
    processes sharing the port (0: in this process), under a closed loop of
    `procs` client processes x `callers` threads sending 640x640 JPEG frames over 127.0.0.1.
    Throughput is the sum over the client processes; p50 is the median of their medians,
    p99 the worst of their p99s."""
    import io
    import subprocess
    import modelgen
    import yolort
    import yoloserve
    from PIL import Image
    d = os.path.join(workdir, "yolo11n_serve")
    modelgen.write_model(d, "yolo11", "n", cls_bias=-8.0)
    paths = []
    for i in range(16):
        p = os.path.join(workdir, f"serve_{i}.jpg")
        Image.fromarray(modelgen.synth_frame(640, 640, 50, 500 + i)[..., ::-1].copy()).save(p, "JPEG", quality=90)
        paths.append(p)
    models = [yoloserve.Model("yolo11n", yolort.Engine(d, 16), 16)]
    srv = yoloserve.Server(models, target_ms=50.0, log=lambda *a: None)
    gs, port = yoloserve.grpc_server(srv, "127.0.0.1:0", frontends=frontends)
    script = os.path.join(ROOT, "yolo11.cu_amd", "yoloserve.py")
    imgs = sum([["--image", p] for p in paths], [])

    def load(secs):
        cmd = [sys.executable, script, "bench", "--addr", f"127.0.0.1:{port}", "--concurrency", str(callers),
               "--seconds", str(secs)] + imgs
        ps = [subprocess.Popen(cmd, stdout=subprocess.PIPE, text=True) for _ in range(procs)]
        res = []
        for p in ps:
            out, _ = p.communicate(timeout=secs + 120)
            if p.returncode != 0:
                raise RuntimeError(f"client process failed ({p.returncode})")
            res.append(json.loads(out.strip().splitlines()[-1]))
        return res

    try:
        load(1.0)                                        # warm-up (connections, graphs)
        res = load(seconds)
    finally:
        gs.stop(0)
        srv.stop()
        models[0].eng.close()
    import numpy as np
    return dict(clients=procs * callers, client_procs=procs, img_per_s=sum(r["img_per_s"] for r in res),
                p50_ms=float(np.median([r["p50_ms"] for r in res])), p99_ms=max(r["p99_ms"] for r in res),
                mean_batch=float(np.mean([r["mean_batch"] for r in res])), requests=sum(r["requests"] for r in res),
                exec_ms_b16=round(models[0].exec_ms, 4), frames="640x640 JPEG q90, decoded on the engine",
                decoder_threads=yolort.decoder_threads(), frontend_processes=frontends)


def bench_feeder(workdir, seconds=4.0, feeders=48, native=True):
    """The server's engine side alone: `feeders` threads submit 640x640 JPEG frames straight
    to yoloserve.Server (no gRPC) in a closed loop, yolo11n with max batch 16 and target
    50 ms; throughput and mean batch.  native=True is the library's batch worker
    (yolo_batcher_*), False the same loop in Python."""
    import io
    import threading
    import modelgen
    import yolort
    import yoloserve
    from PIL import Image
    d = os.path.join(workdir, "yolo11n_feed")
    if not os.path.exists(os.path.join(d, "model.graph")):
        modelgen.write_model(d, "yolo11", "n", cls_bias=-8.0)
    streams = []
    for i in range(16):
        b = io.BytesIO()
        Image.fromarray(modelgen.synth_frame(640, 640, 50, 500 + i)[..., ::-1].copy()).save(b, "JPEG", quality=90)
        streams.append(b.getvalue())
    eng = yolort.Engine(d, 16)
    srv = yoloserve.Server([yoloserve.Model("yolo11n", eng, 16)], target_ms=50.0, log=lambda *a: None,
                           native=native)
    stop_at = [0.0]
    counts = [0] * feeders
    batches = [0.0] * feeders
    errors = [0]

    def feed(i):
        k = i
        while time.perf_counter() < stop_at[0]:
            r = srv.submit_jpeg(streams[k % 16])
            k += 1
            r.done.wait()
            if r.error:
                errors[0] += 1
                continue
            counts[i] += 1
            batches[i] += r.resp.batch

    try:
        for secs, measure in ((1.0, False), (seconds, True)):
            counts[:] = [0] * feeders
            batches[:] = [0.0] * feeders
            stop_at[0] = time.perf_counter() + secs
            t0 = time.perf_counter()
            ts = [threading.Thread(target=feed, args=(i,)) for i in range(feeders)]
            for t in ts:
                t.start()
            for t in ts:
                t.join()
            el = time.perf_counter() - t0
    finally:
        srv.stop()
        eng.close()
    n = sum(counts)
    return dict(img_per_s=round(n / el, 1), feeders=feeders, mean_batch=round(sum(batches) / max(n, 1), 2),
                errors=errors[0], worker="native (yolo_batcher)" if native else "python")


def bench_jpeg(workdir, batches=60, graphs=True):
    """JPEG decode on the engine for a batch of 16 640x640 q90 frames (the server bench's
    frames): yolo_stage_jpeg wall time per batch with the GPU drained (entropy decoding on the
    library's decoder threads, then H2D of the coefficients, IDCT, colour and the letterbox),
    the single-thread entropy decode of one frame, and PIL's full decode of one frame for
    comparison (the server's decoder for everything the engine does not decode)."""
    import io
    import modelgen
    import yolort
    from PIL import Image
    d = os.path.join(workdir, "yolo11n_jpeg")
    modelgen.write_model(d, "yolo11", "n", cls_bias=-8.0)
    streams = []
    for i in range(16):
        b = io.BytesIO()
        Image.fromarray(modelgen.synth_frame(640, 640, 50, 500 + i)[..., ::-1].copy()).save(b, "JPEG", quality=90)
        streams.append(b.getvalue())
    eng = yolort.Engine(d, 16, yolort.YOLO_NOTUNE | (0 if graphs else yolort.YOLO_NOGRAPH))
    try:
        for _ in range(5):
            eng.stage_jpeg(streams)
        eng.sync()
        t0 = time.perf_counter()
        for _ in range(batches):
            eng.stage_jpeg(streams)
            eng.sync()
        ms = (time.perf_counter() - t0) / batches * 1e3
    finally:
        eng.close()
    one = streams[0]
    yolort.jpeg_coefficients(one)
    t0 = time.perf_counter()
    for _ in range(50):
        yolort.jpeg_coefficients(one)
    entropy_ms = (time.perf_counter() - t0) / 50 * 1e3
    t0 = time.perf_counter()
    for _ in range(20):
        with Image.open(io.BytesIO(one)) as im:
            im.load()
    pil_ms = (time.perf_counter() - t0) / 20 * 1e3
    return dict(ms_per_batch16=round(ms, 4), img_per_s=round(16e3 / ms, 1), decoder_threads=yolort.decoder_threads(),
                entropy_ms_one_frame_one_thread=round(entropy_ms, 4), pil_decode_ms_one_frame=round(pil_ms, 4),
                frames="640x640 JPEG q90 4:2:0, ~69 KB")


def cpu_baseline(budget_s=15.0):
    """The reference's CPU path -- a torch fp32 per-op interpreter of the graph
    (export/export.py:446-526, restated in oracle/torchref.py) plus the CPU letterbox,
    decode and NMS -- timed on the yolo11n batch-1 frame of config 0, in a separate
    process that never loads the GPU library, with every core this process may use."""
    import subprocess
    script = os.path.join(ROOT, "oracle", "torchref.py")
    r = subprocess.run([sys.executable, script, "--seconds", str(budget_s)], capture_output=True,
                       text=True, timeout=budget_s + 300)
    if r.returncode != 0:
        raise RuntimeError(f"cpu baseline failed ({r.returncode}): {r.stderr[-2000:]}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    return dict(value=round(1e3 / res["ms"], 3), unit="frames/s", cores=int(res["threads"]), kind="port",
                impl="torch fp32 per-op interpreter (export/export.py:446-526) + numpy letterbox/decode/NMS",
                host_cpu_count=res["cpu_count"], affinity_cpus=res["affinity"],
                sample=f"yolo11n b1 810x1080 frame, letterbox + 112 ops + decode + NMS on the CPU; median of "
                       f"{res['frames']} frames = {res['ms']:.1f} ms/frame ({res['threads']} torch threads)")


def _finite(o):
    """The JSON line in standard JSON: a figure that came out non-finite (a zero time) is null."""
    if isinstance(o, dict):
        return {k: _finite(v) for k, v in o.items()}
    if isinstance(o, (list, tuple)):
        return [_finite(v) for v in o]
    if isinstance(o, float) and not math.isfinite(o):
        return None
    return o


def prepost_roofline(n, seg):
    """Achieved HBM bandwidth of the pre/post kernels against the 8 TB/s roofline, from the
    stage times (hipEvents, stream-ordered) and their algorithmic bytes:
      letterbox  sh*sw*3 (u8 frame) + S*S*3*2 (fp16 input tensor)
      decode     A*(64 + ncpad)*2 (box bins + class logits, fp16) + 24 per candidate
      masks      Ph*Pw*nm*2 (proto, fp16) + survivors*Ph*Pw (u8 masks)
    NMS is latency-bound: its time is reported, not a bandwidth."""
    out = {}
    if n:
        st = n["stages"]
        sh, sw = n["frame"]
        lb = sh * sw * 3 + 640 * 640 * 3 * 2
        dec = n["A"] * (64 + n["ncpad"]) * 2 + 24 * n["raw"]
        for name, nbytes in (("letterbox", lb), ("decode", dec)):
            us = st[name] * 1e3
            gbs = nbytes / (us * 1e-6) / 1e9
            out[name] = {"workload": "yolo11n b1 810x1080", "us": round(us, 2), "bytes": int(nbytes),
                         "GB/s": round(gbs, 1), "frac": round(gbs * 1e9 / PEAK_HBM, 4)}
        out["nms"] = {"workload": f"yolo11n b1, {n['raw']} candidates", "us": round(st["nms"] * 1e3, 2),
                      "bound": "latency"}
    if seg:
        st = seg["stages"]
        nbytes = 160 * 160 * 32 * 2 + seg["kept"] * 160 * 160
        us = st["masks"] * 1e3
        gbs = nbytes / (us * 1e-6) / 1e9
        out["masks"] = {"workload": f"yolo11n-seg b1, {seg['kept']} survivors", "us": round(us, 2),
                        "bytes": int(nbytes), "GB/s": round(gbs, 1), "frac": round(gbs * 1e9 / PEAK_HBM, 4)}
        out["nms_seg"] = {"workload": f"yolo11n-seg b1, {seg['raw']} candidates", "us": round(st["nms"] * 1e3, 2),
                          "bound": "latency"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", choices=["all", "n", "x", "conv", "obb", "seg", "m", "sweep", "cls", "serve", "feed",
                                       "jpeg"],
                    default="all")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the same kernels stream-ordered (rocprofv3's kernel tracer "
                         "crashes inside hipGraphLaunch on this image); prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (frames are independent: the path shards as one engine "
              f"per GPU with no exchange); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    workdir = tempfile.mkdtemp(prefix="yolo_bench_")
    out = {}
    if args.only in ("all", "conv"):
        log("conv sweep roofline shape ...")
        out["conv"] = bench_conv(workdir, 20)
        log(out["conv"])
    if args.only in ("all", "n"):
        log("yolo11n b1 e2e ...")
        out["n"] = bench_n(workdir, args.steps, args.warmup, not args.no_graph)
        log(out["n"])
    if args.only in ("all", "x"):
        log("yolo11x b16 ...")
        out["x"] = bench_x(workdir, 20, not args.no_graph)
        log(out["x"])
    if args.only in ("all", "m"):
        log("yolo11m b1 1920x1080 e2e (IoU 0.7) ...")
        out["m"] = bench_m(workdir, args.steps, args.warmup, not args.no_graph)
        log(out["m"])
    if args.only in ("all", "cls"):
        log("yolo11n-cls b1 @224 e2e ...")
        out["cls"] = bench_cls(workdir, args.steps, args.warmup, not args.no_graph)
        log(out["cls"])
    if args.only in ("all", "sweep") and not args.no_graph:
        log("conv sweep (config 1) ...")
        out["sweep"] = bench_sweep(workdir, 10)
        log(out["sweep"])
    if args.only in ("all", "obb", "seg"):
        import modelgen
        if args.only in ("all", "obb"):
            log("yolo11n-obb b1 @1024 e2e ...")
            out["obb"] = bench_task(workdir, "obb", 1024, 15, -6.25, modelgen.synth_frame(1024, 1024, 50, 7),
                                    args.steps, args.warmup, not args.no_graph)
            log(out["obb"])
        if args.only in ("all", "seg"):
            log("yolo11n-seg b1 e2e ...")
            out["seg"] = bench_task(workdir, "segment", 640, 80, -8.0, modelgen.synth_polygons(640, 640, 30, 4),
                                    args.steps, args.warmup, not args.no_graph)
            log(out["seg"])
    if args.only in ("all", "jpeg"):
        log("JPEG decode on the engine, batch 16 ...")
        out["jpeg"] = bench_jpeg(workdir, graphs=not args.no_graph)
        log(out["jpeg"])
    if args.only in ("all", "serve", "feed") and not args.no_graph:
        log("server engine side, 48 feeder threads, native batch worker ...")
        out["feed"] = bench_feeder(workdir, native=True)
        log(out["feed"])
        if args.only == "feed":
            log("the same with the Python batch loop ...")
            out["feed_py"] = bench_feeder(workdir, native=False)
            log(out["feed_py"])
    if args.only in ("all", "serve") and not args.no_graph:
        log("gRPC server, yolo11n, 4 client processes x 16 callers ...")
        out["serve"] = bench_serve(workdir)
        log(out["serve"])
    if args.no_graph:
        log("stream-ordered profiling pass done")
        return
    cpu = None
    if args.only == "all" and not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline()
        log(cpu)
    n = out.get("n")
    x = out.get("x")
    conv = out.get("conv")
    line = {
        "metric": "e2e ms/frame & FPS @640 fp16 (yolo11n b1, yolo11x b16); conv MFMA util %",
        "value": round(1e3 / n["ms"], 2) if n else None,
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(n["ms"], 4) if n else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic frames, seeded random-init weights",
        "config": {"workload": "yolo11n detect b1 e2e: H2D of the raw frame from pinned memory + letterbox + "
                               "net + DFL decode + NMS + result copy in one hipGraph, wait, host fetch",
                   "imgsz": 640, "frame": "810x1080 u8 BGR", "batch": 1},
    }
    if n:
        line["yolo11n_b1"] = {"ms_per_frame": round(n["ms"], 4), "graph_ms": round(n["graph_ms"], 4),
                              "ms_per_frame_frame_in_hbm": round(n["ms_hbm"], 4),
                              "graph_ms_frame_in_hbm": round(n["graph_ms_hbm"], 4), "kept": n["kept"],
                              "raw_candidates": n["raw"], "stream_ops_ms": round(n["stream_ops_ms"], 4),
                              "units_ms": round(n["units_ms"], 4), "launch_units": n["launches"],
                              "units": [{"kernel": g["kernel"], "class": g["class"], "launches": g["launches"],
                                         "us": round(g["ms"] * 1e3, 1)} for g in n["units"][:10]]}
    if x:
        line["yolo11x_b16"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in x.items()
                               if k not in ("dominant", "units")}
        line["yolo11x_b16"]["units"] = [{"kernel": g["kernel"], "class": g["class"], "launches": g["launches"],
                                         "us": round(g["ms"] * 1e3, 1),
                                         "tflops": round(g["flops"] / (g["ms"] * 1e-3) / 1e12, 1) if g["flops"] else 0.0}
                                        for g in x["units"]]
        line["roofline_yolo11x_b16"] = x["dominant"]
    for key, name in (("m", "yolo11m_b1_1080p_iou07"), ("obb", "yolo11n_obb_b1_1024"), ("seg", "yolo11n_seg_b1")):
        r = out.get(key)
        if r:
            line[name] = {"ms_per_frame": round(r["ms"], 4), "graph_ms": round(r["graph_ms"], 4),
                          "kept": r["kept"], "raw_candidates": r["raw"]}
            if "ms_hbm" in r:
                line[name]["ms_per_frame_frame_in_hbm"] = round(r["ms_hbm"], 4)
            else:
                line[name]["frame"] = "in HBM"
    if out.get("cls"):
        r = out["cls"]
        line["yolo11n_cls_b1_224"] = {"ms_per_frame": round(r["ms"], 4), "graph_ms": round(r["graph_ms"], 4),
                                      "top1": r["top1"]}
    if out.get("sweep"):
        line["conv_sweep"] = out["sweep"]
    if out.get("jpeg"):
        line["jpeg_decode_b16"] = out["jpeg"]
    if out.get("serve"):
        line["grpc_server_yolo11n"] = {k: (round(v, 3) if isinstance(v, float) else v)
                                       for k, v in out["serve"].items()}
    if out.get("feed"):
        line["server_engine_side_yolo11n"] = out["feed"]
        if out.get("feed_py"):
            line["server_engine_side_yolo11n_python_loop"] = out["feed_py"]
    pp = prepost_roofline(n, out.get("seg"))
    if pp:
        line["prepost_roofline"] = pp
    if conv:
        achieved = conv["flops"] / (conv["ms"] * 1e-3)
        line["roofline"] = {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": 2500.0,
                            "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16, 4),
                            "traffic": measured_traffic(conv["cfg"], conv["tail"]),
                            "kernel": conv_kernel_name(conv["cfg"], conv["tail"]), "shape": conv["shape"],
                            "ms": round(conv["ms"], 4)}
    if cpu:
        line["cpu_baseline"] = cpu
    print(json.dumps(_finite(line)), flush=True)


if __name__ == "__main__":
    main()
