"""GPU parity of the OBB path (yolo11n-obb at 1024, 15 classes) through the C ABI.

  * every op of the unfused graph in isolation against the oracle (resync), then decode +
    rotated fast-NMS on identical head tensors: same raw count, survivors, order, classes;
    scores, boxes and angles to fp32 transcendental accuracy.  Also with more candidates
    than NMS_CAP (radix select) and with every anchor a candidate (conf 0)
  * the fused/tuned/graph frame under the trajectory gate (each op against the oracle on its
    own GPU inputs, decode + fast-NMS exact on the run's heads, the frame graph equal to it)
  * batch self-consistency and graph replays
"""
import numpy as np
import pytest

import modelgen
import yolort
from oracle import graphfile, interp, post

import _frame_gate as fg

pytestmark = pytest.mark.gpu

TOL = 0.015
OBB_BIAS = -6.25     # ~1,300 candidates at conf 0.25 on the C3-style frame (the reference's
                     # boats.jpg case has 1,346, docs/specs/obb.md:483-484)


def _model(models):
    return models("yolo11", "n", "obb", OBB_BIAS, 1024, 0, 15)


def _all_scores(heads, nc):
    return np.concatenate([1 / (1 + np.exp(-c[..., :nc].astype(np.float64).max(-1))).ravel()
                           for _, c, _, _ in heads])


def _safe_thresholds(heads, nc, conf, iou):
    """Nudges conf / iou away from any score or same-class probiou within 1e-5 of them, so
    the last-ulp differences between the device's and numpy's exp/log/cos/sin cannot flip a
    decision (the margins found are printed)."""
    s = _all_scores(heads, nc)
    while conf > 0 and np.abs(s - conf).min() < 1e-5:
        conf += 1e-3
    c = post.decode_obb_all(heads, nc, conf)
    order = post.rank_order(c["score"], c["anchor"])[:2048]
    rb, th, cl = c["rbox"][order], c["theta"][order], c["cls"][order]
    A, B, C = post.covariance(rb[:, 2], rb[:, 3], th)
    ious = []
    for k in np.unique(cl):
        m = np.nonzero(cl == k)[0]
        i, j = m[:, None], m[None, :]
        v = post.probiou(rb[i, 0], rb[i, 1], A[i], B[i], C[i], rb[j, 0], rb[j, 1], A[j], B[j], C[j])
        ious.append(v[np.triu_indices(len(m), 1)])
    ious = np.concatenate(ious) if ious else np.zeros(0, np.float32)
    while len(ious) and np.abs(ious - iou).min() < 1e-5:
        iou += 1e-3
    print(f"conf {conf:.4f} iou {iou:.4f}: {len(c['score'])} candidates, {len(ious)} same-class pairs",
          flush=True)
    return conf, iou


def _check_post(eng, heads, nc, conf, iou):
    want = post.detect_obb(heads, nc, conf, iou)
    got = eng.get_obb(0)
    print(f"  raw {eng.raw_count(0)} / {want['n_raw']}, kept {len(got)} / {len(want['score'])}", flush=True)
    assert eng.raw_count(0) == want["n_raw"]
    assert len(got) == len(want["score"])
    np.testing.assert_array_equal(got[:, 6].astype(int), want["cls"])
    np.testing.assert_allclose(got[:, 5], want["score"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(got[:, :4], want["rbox"], rtol=0, atol=2e-3)
    np.testing.assert_allclose(got[:, 4], want["theta"], rtol=0, atol=2e-6)


@pytest.mark.parametrize("nmsflag", [0, yolort.YOLO_NMS_BLOCK], ids=["multi", "block"])
def test_obb_ops_resync_and_post(models, nmsflag):
    d = _model(models)
    g = graphfile.load(d)
    img = modelgen.synth_frame(1024, 1024, 50, 7)
    x = post.letterbox(img, 1024, 1024)[None]
    ref = interp.Interp(g, 1, round_fp16=True)
    ref.set_input(x)
    eng = yolort.Engine(d, 1, yolort.YOLO_NOFUSE | yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH | nmsflag)
    assert eng.task() == 1
    eng.write(0, ref.view(0))
    rels, last_decode = [], -1
    for k, op in enumerate(g.ops):
        t = ref.run_op(op)
        eng.run_op(k, 1)
        if op.kind == "DECODEOBB":
            last_decode = k
        if t is None:
            continue
        want = ref.view(t)
        rels.append((k, op.kind, post.rel_err(eng.read(t, 1).astype(np.float32), want)))
        eng.write(t, want)
    worst = sorted(rels, key=lambda r: -r[2])[:5]
    print("worst ops:", ", ".join(f"op{k:03d} {kind} {rel:.2e}" for k, kind, rel in worst), flush=True)
    assert len(rels) == 118      # yolo11n's 109 dumped ops + the 9 angle-branch convs
    assert not [r for r in rels if not r[2] <= TOL]
    heads = [(b[0], c[0], a[0], s) for b, c, a, s in ref.heads_in]
    for conf0 in (0.25, 0.02, 0.0):
        conf, iou = _safe_thresholds(heads, 15, conf0, 0.45)
        eng.set_thresholds(conf, iou, 300)
        eng.run_op(last_decode, 1)
        eng.run_post(1)
        _check_post(eng, heads, 15, conf, iou)
    assert len(eng.get(0)) == 0          # detect getter refuses OBB records
    eng.close()


def _letterbox_gpu(eng, img, slot=0):
    buf = yolort.DeviceBuffer(img.nbytes)
    eng.upload(buf, img)
    eng.preprocess(buf.ptr, img.shape[0], img.shape[1], slot)
    eng.sync()
    return buf


def test_obb_frame_trajectory_and_graph(models):
    """The frame as benchmarked (fused, autotuned, graphs; an 810x1080 frame letterboxed on
    the GPU to 1024) under the trajectory gate of the detect and segment configurations:
    every op's output against the oracle applied to that op's own GPU inputs (1.5 % bar),
    then decode + rotated fast-NMS exact on the run's head tensors (thresholds nudged off
    last-ulp ties of the transcendentals, as in the resync test), and the whole-frame graph
    returning exactly the trajectory's rotated boxes."""
    d = _model(models)
    g = graphfile.load(d)
    img = modelgen.synth_frame(810, 1080, 40, 11)
    eng = yolort.Engine(d, 1)
    buf = _letterbox_gpu(eng, img)
    np.testing.assert_array_equal(eng.read(0, 1)[0], post.letterbox(img, 1024, 1024))
    rels, _ = fg.trajectory(eng, g, 1, [0], obb=True)
    fg.gate(rels, "obb frame")
    fops = graphfile.fuse_adds(g.ops)
    last_decode = max(k for k, op in enumerate(fops) if op.kind == "DECODEOBB")
    heads = [(eng.read(op.a)[0].astype(np.float32), eng.read(op.b)[0].astype(np.float32),
              eng.read(op.out)[0].astype(np.float32), op.stride) for op in fops if op.kind == "DECODEOBB"]
    conf, iou = _safe_thresholds(heads, 15, 0.25, 0.45)
    eng.set_thresholds(conf, iou, 300)
    eng.run_op(last_decode, 1)
    eng.run_post(1)
    want = post.detect_obb(heads, 15, conf, iou)
    traj = eng.get_obb(0)
    s, top, left = (np.float32(v) for v in eng.slot_geom(0))
    rb = want["rbox"].astype(np.float32)
    want_orig = np.stack([(rb[:, 0] - left) / s, (rb[:, 1] - top) / s, rb[:, 2] / s, rb[:, 3] / s], 1)
    print(f"obb frame: raw {eng.raw_count(0)} / {want['n_raw']}, kept {len(traj)} / {len(want['score'])}", flush=True)
    assert eng.raw_count(0) == want["n_raw"]
    assert len(traj) == len(want["score"]) > 0
    np.testing.assert_array_equal(traj[:, 6].astype(int), want["cls"])
    np.testing.assert_allclose(traj[:, 5], want["score"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(traj[:, :4], want_orig, rtol=0, atol=2e-3)
    np.testing.assert_allclose(traj[:, 4], want["theta"], rtol=0, atol=2e-6)
    eng.frame_graph([buf.ptr], [810], [1080])
    for _ in range(2):
        eng.frame_run()
        np.testing.assert_array_equal(eng.get_obb(0), traj)
    buf.free()
    eng.close()


def test_obb_batch_consistency_and_replay(models):
    d = _model(models)
    img = modelgen.synth_frame(1024, 1024, 50, 7)
    B = 2
    eng = yolort.Engine(d, B)
    bufs = [_letterbox_gpu(eng, img, s) for s in range(B)]
    eng.run(B)
    first = [eng.get_obb(s) for s in range(B)]
    assert len(first[0]) > 50
    np.testing.assert_array_equal(first[1], first[0])
    for _ in range(3):
        eng.run(B)
        for s in range(B):
            np.testing.assert_array_equal(eng.get_obb(s), first[s])
    eng.run(1)
    np.testing.assert_array_equal(eng.get_obb(0), first[0])
    for b in bufs:
        b.free()
    eng.close()
