"""Whole-frame parity of the BASELINE configurations on the GPU, through the C ABI.

* Trajectory check of the frame as it is benchmarked (CONV+ADD fused, autotuned tiles,
  letterbox on the GPU): every op of the run is compared with the oracle applied to the
  op's own GPU inputs of that same run (max|gpu - ref| / max|ref| <= 1.5 %, the per-op bar
  of test/compare.py:21-25), then decode + NMS (+ masks) must equal the oracle's exactly on
  the run's head tensors, and the whole-frame graph (letterbox + net + decode + NMS in one
  hipGraph) must return exactly the trajectory's detections.  The composed frame is thereby
  held to the per-op bar at every op boundary and to the exact bar at its output.
* yolo11x batch 16 (config 3): per-op resync of the unfused graph with the oracle on images
  0 and 15, decode + NMS exact on all 16 slots of the batch-16 frame graph, and slot i of
  that graph equal to a batch-1 run of frame i (engine/engine.cu:1843-1888,1914-1936).
* yolo11m, a 1080x1920 frame at IoU 0.7 (config 2), through the frame graph.
"""
import numpy as np
import pytest

import modelgen
import yolort
from oracle import graphfile, interp, post

from _frame_gate import TOL, assert_dets_equal, gate, letterbox_slots, trajectory
import _frame_gate as fg

pytestmark = pytest.mark.gpu

FRAMES = {
    "C0": lambda: modelgen.synth_frame(810, 1080, 20, 1),
    "C2": lambda: modelgen.synth_frame(1080, 1920, 20, 2),
    "C4": lambda: modelgen.synth_polygons(640, 640, 30, 4),
    "v8": lambda: modelgen.synth_frame(810, 1080, 20, 5),
}


@pytest.mark.parametrize("case,arch,scale,task,iou", [
    ("C0", "yolo11", "n", "detect", 0.45),
    ("C4", "yolo11", "n", "segment", 0.45),
    ("C2", "yolo11", "m", "detect", 0.7),
    ("v8", "yolov8", "n", "detect", 0.45)])
def test_frame_trajectory_and_graph(models, case, arch, scale, task, iou):
    d = models(arch, scale, task)
    g = graphfile.load(d)
    img = FRAMES[case]()
    print(f"{case}: {arch}{scale}-{task} frame {img.shape[:2]} iou {iou}", flush=True)
    eng = yolort.Engine(d, 1)          # fused, autotuned, graphs captured (the bench setup)
    eng.set_thresholds(0.25, iou, 300)
    bufs = letterbox_slots(eng, [img])
    np.testing.assert_array_equal(eng.read(0, 1)[0], post.letterbox(img, 640, 640))
    rels, wants = trajectory(eng, g, 1, [0], 0.25, iou)
    gate(rels, case)
    traj = eng.get(0)
    assert_dets_equal(eng, 0, traj, wants[0])
    assert eng.raw_count(0) == wants[0]["n_raw"]
    print(f"{case}: kept {len(traj)} raw {eng.raw_count(0)} (exact vs oracle on the run's heads)", flush=True)
    if task == "segment":
        proto_t = [op.a for op in g.ops if op.kind == "MASKS"][0]
        proto = eng.read(proto_t)[0].astype(np.float32)
        wm = post.masks(proto, wants[0]["coef"], wants[0]["box"], 640, 640)
        ious = []
        for i in range(len(traj)):
            gm = eng.get_mask(0, i).astype(bool)
            union = np.logical_or(gm, wm[i]).sum()
            ious.append(1.0 if union == 0 else np.logical_and(gm, wm[i]).sum() / union)
        print(f"{case}: mask IoU min {min(ious):.4f} over {len(ious)} survivors", flush=True)
        assert min(ious) >= 0.99
    # the whole-frame graph (letterbox + net + decode + NMS + result copy) on the same frame
    eng.frame_graph([bufs[0].ptr], [img.shape[0]], [img.shape[1]])
    for _ in range(2):
        eng.frame_run()
        np.testing.assert_array_equal(eng.get(0), traj)
        assert eng.raw_count(0) == wants[0]["n_raw"]
    # end to end (test/compare_seg.py:61-100): the frame's detections (= the trajectory's, in
    # letterbox space) against the round-fp16 oracle run on the same letterboxed input, held
    # to twice the oracle's own disagreement under fp32 rounding changes plus a small slack
    x = post.letterbox(img, 640, 640)[None].astype(np.float32)
    ref = fg.oracle_frame(g, x, task, iou)
    got = dict(wants[0])
    if task == "segment":
        got["masks"] = np.stack([eng.get_mask(0, i) for i in range(len(traj))]) if len(traj) else None
    d_gpu = fg.disagreement(ref, got)
    floor = fg.noise_floor(g, x, task, iou, ref)
    bound = fg.e2e_bound(floor)
    print(f"{case}: end to end vs the round-fp16 oracle {d_gpu}; oracle floor {floor}; bound {bound}", flush=True)
    assert fg.within(d_gpu, bound), (d_gpu, bound)
    bufs[0].free()
    eng.close()


# ------------------------------------------------------------------ config 3: yolo11x b16
X_B = 16


def _x_frames():
    return [modelgen.synth_frame(640, 640, 50, 100 + i) for i in range(X_B)]


def test_yolo11x_b16_ops_resync(models):
    """Unfused yolo11x at batch 16 with autotuned tiles: every op's output on images 0 and 15
    against the round-fp16 oracle fed the oracle's own previous outputs (resync of those two
    images after each op), then decode + NMS on the resynced heads exact."""
    d = models("yolo11", "x")
    g = graphfile.load(d)
    frames = _x_frames()
    pick = [0, X_B - 1]
    eng = yolort.Engine(d, X_B, yolort.YOLO_NOFUSE | yolort.YOLO_NOGRAPH)
    bufs = letterbox_slots(eng, frames)
    ref = interp.Interp(g, len(pick), round_fp16=True)
    ref.set_input(np.stack([post.letterbox(frames[s], 640, 640) for s in pick]).astype(np.float32))
    for j, s in enumerate(pick):
        np.testing.assert_array_equal(eng.read_slots(0, s)[0], ref.view(0)[j].astype(np.float16))
    assert eng.num_ops == len(g.ops)
    rels = []
    for k, op in enumerate(g.ops):
        t = ref.run_op(op)
        eng.run_op(k, X_B)
        if t is None:
            continue
        want = ref.view(t)
        got = np.concatenate([eng.read_slots(t, s) for s in pick]).astype(np.float32)
        rels.append((k, op.kind, post.rel_err(got, want)))
        if k % 25 == 0:
            print(f"  op {k}/{len(g.ops)} {op.kind} rel {rels[-1][2]:.2e}", flush=True)
        for j, s in enumerate(pick):
            eng.write_slots(t, s, want[j:j + 1])
    gate(rels, "yolo11x b16 resync")
    assert len(rels) == sum(1 for op in g.ops if op.kind not in ("DECODE",))
    eng.run_post(X_B)
    for j, s in enumerate(pick):
        heads = [(b[j], c[j], None, st) for b, c, _, st in ref.heads_in]
        want = post.detect(heads, 80)
        got = eng.get(s)
        print(f"slot {s}: kept {len(got)} raw {eng.raw_count(s)}", flush=True)
        assert eng.raw_count(s) == want["n_raw"]
        assert_dets_equal(eng, s, got, want)
    for b in bufs:
        b.free()
    eng.close()


@pytest.fixture(scope="module")
def x_fused(models):
    """The bench configuration of config 3, built once for the module: fused + autotuned
    yolo11x at batch 16 with its graphs, and the sixteen frames uploaded to the device."""
    d = models("yolo11", "x")
    g = graphfile.load(d)
    frames = _x_frames()
    eng = yolort.Engine(d, X_B)
    devs = []
    for f in frames:
        b = yolort.DeviceBuffer(f.nbytes)
        eng.upload(b, f)
        devs.append(b)
    yield g, frames, eng, devs
    for b in devs:
        b.free()
    eng.close()


def test_yolo11x_b16_frame_graph(x_fused):
    """Sixteen frames in one frame graph: decode + NMS exact on the GPU's own heads for every
    slot; slot i equal to a batch-1 run of frame i on the same handle (the reference's batch
    self-consistency check)."""
    g, frames, eng, devs = x_fused
    eng.frame_graph([b.ptr for b in devs], [640] * X_B, [640] * X_B)
    eng.frame_run()
    batch = [eng.get(s) for s in range(X_B)]
    dec = [op for op in g.ops if op.kind == "DECODE"]
    for s in range(X_B):
        heads = [(eng.read_slots(op.a, s)[0].astype(np.float32), eng.read_slots(op.b, s)[0].astype(np.float32),
                  None, op.stride) for op in dec]
        want = post.detect(heads, 80)
        assert eng.raw_count(s) == want["n_raw"]
        assert_dets_equal(eng, s, batch[s], want)
    print("kept per slot:", [len(b) for b in batch], flush=True)
    assert sum(len(b) for b in batch) > 0
    for i in range(X_B):
        eng.preprocess(devs[i].ptr, 640, 640, 0)
        eng.run(1)
        one = eng.get(0)
        assert len(one) == len(batch[i]), (i, len(one), len(batch[i]))
        np.testing.assert_array_equal(one, batch[i])


def test_yolo11x_b16_trajectory(x_fused):
    """The same fused, autotuned engine run op by op at batch 16: images 0 and 15 of every
    op's output against the oracle applied to that op's GPU inputs; decode + NMS exact."""
    g, frames, eng, devs = x_fused
    for s in range(X_B):
        eng.preprocess(devs[s].ptr, 640, 640, s)
    eng.sync()
    pick = [0, X_B - 1]
    rels, wants = trajectory(eng, g, X_B, pick)
    gate(rels, "yolo11x b16 trajectory")
    for j, s in enumerate(pick):
        assert_dets_equal(eng, s, eng.get(s), wants[j])


def test_branches_eager_equals_serial(models):
    """YOLO_BRANCHES (eager forward with independent branches on side streams) gives tensors
    and detections bit-identical to the single-stream order, over repeated runs."""
    d = models("yolo11", "n")
    g = graphfile.load(d)
    img = modelgen.synth_frame(810, 1080, 20, 3)
    res = {}
    for name, flags in (("branches", yolort.YOLO_BRANCHES), ("serial", 0)):
        eng = yolort.Engine(d, 2, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH | flags)
        bufs = letterbox_slots(eng, [img, modelgen.synth_frame(640, 640, 50, 4)])
        outs = []
        for _ in range(3):
            eng.run(2)
            outs.append([eng.get(s) for s in range(2)])
        outs.append([eng.read(t, 2) for t in range(len(g.tens))])
        res[name] = outs
        for b in bufs:
            b.free()
        eng.close()
    for a, b in zip(res["branches"], res["serial"]):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    assert len(res["serial"][0][0]) > 0
