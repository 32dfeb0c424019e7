"""Shared whole-frame checks for the GPU tests (imported by test modules; not collected).

* The trajectory gate: the frame's ops run one by one on the GPU; each op's output is
  compared with the oracle applied to that op's own GPU inputs of the same run (the per-op
  bar of test/compare.py:21-25), then decode + NMS (+ masks) must equal the oracle's exactly
  on the run's head tensors.
* The end-to-end gate (the reference's level 3, test/compare_seg.py:61-100): the frame's
  detections against the round-fp16 oracle run end to end on the same letterboxed input,
  under the reference's matching rule.  Random-init networks make whole-frame detections
  sensitive to the rounding of every fp32 accumulation, so the bound is the oracle's own
  disagreement with itself when only that rounding changes (float64 accumulation, and the
  conv sums in four other seeded orders), times two plus a small slack.  A systematic error
  far inside the per-op bar fails it: a 0.1 % gain on every conv output of the oracle moves
  the unmatched count from 1-3 to 73 on the yolo11n frame (tests/test_oracle_e2e.py).
"""
import numpy as np

import yolort
from oracle import graphfile, interp, post

TOL = 0.015   # per-op max relative deviation vs the fp32 oracle (BASELINE parity bar)


def letterbox_slots(eng, frames):
    bufs = []
    for s, f in enumerate(frames):
        b = yolort.DeviceBuffer(f.nbytes)
        eng.upload(b, f)
        eng.preprocess(b.ptr, f.shape[0], f.shape[1], s)
        bufs.append(b)
    eng.sync()
    return bufs


def to_original(eng, slot, dets):
    """Oracle boxes (letterbox space) mapped to original-image coordinates with yolo_get's
    float32 operations, so they compare with yolo_get's output directly."""
    scale, top, left = eng.slot_geom(slot)
    b = dets.astype(np.float32)
    x1 = (b[:, 0] - np.float32(left)) / np.float32(scale)
    y1 = (b[:, 1] - np.float32(top)) / np.float32(scale)
    x2 = (b[:, 2] - np.float32(left)) / np.float32(scale)
    y2 = (b[:, 3] - np.float32(top)) / np.float32(scale)
    return np.stack([x1, y1, x2, y2], 1).astype(np.float64)


def assert_dets_equal(eng, slot, got, want):
    """Exact decode + NMS parity: same count, classes and survivor order, scores within fp32
    rounding of the sigmoid, boxes from the same float32 arithmetic."""
    assert len(got) == len(want["score"]), (slot, len(got), len(want["score"]))
    np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
    np.testing.assert_allclose(got[:, 4], want["score"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(got[:, :4], to_original(eng, slot, want["box"]), rtol=0, atol=2e-3)


def trajectory(eng, g, B, check_slots, conf=0.25, iou=0.45, obb=False):
    """Runs the engine's (fused) op list op by op for B images; every op's output on
    `check_slots` is compared with the oracle applied to that op's GPU inputs.  Returns the
    per-op deviations and the oracle detections on the run's own head tensors."""
    fops = graphfile.fuse_adds(g.ops)
    assert eng.num_ops == len(fops)
    ref = interp.Interp(g, len(check_slots))
    rels = []
    for k, op in enumerate(fops):
        info = eng.op_info(k)
        assert info["kind"] == op.kind and info["a"] == op.a and info["out"] == op.out, (k, info, op)
        ins = [t for t in ((op.a, op.b) if op.kind in ("CONV", "ADD") else (op.a,)) if t >= 0]
        if op.kind in ("DECODESEG", "DECODEOBB"):
            ins = [op.a, op.b, op.out]
        elif op.kind == "DECODE":
            ins = [op.a, op.b]
        for t in ins:
            for j, s in enumerate(check_slots):
                ref.view(t)[j] = eng.read_slots(t, s)[0].astype(np.float32)
        eng.run_op(k, B)
        t = ref.run_op(op)
        if t is None:
            continue
        got = np.concatenate([eng.read_slots(t, s) for s in check_slots]).astype(np.float32)
        rel = post.rel_err(got, ref.view(t))
        rels.append((k, op.kind, rel))
        if k % 25 == 0:
            print(f"  op {k}/{len(fops)} {op.kind} rel {rel:.2e}", flush=True)
    eng.run_post(B)
    wants = []
    for j, s in enumerate(check_slots):
        heads = []
        for op in fops:
            if op.kind in ("DECODE", "DECODESEG", "DECODEOBB"):
                heads.append((eng.read_slots(op.a, s)[0].astype(np.float32),
                              eng.read_slots(op.b, s)[0].astype(np.float32),
                              eng.read_slots(op.out, s)[0].astype(np.float32) if op.kind != "DECODE" else None,
                              op.stride))
        wants.append(post.detect_obb(heads, g.nc, conf, iou) if obb else post.detect(heads, g.nc, conf, iou))
    return rels, wants


def gate(rels, label):
    worst = sorted(rels, key=lambda r: -r[2])[:4]
    print(f"{label}: {len(rels)} ops, worst " + ", ".join(f"op{k:03d} {kind} {r:.2e}" for k, kind, r in worst),
          flush=True)
    bad = [r for r in rels if not r[2] <= TOL]
    assert not bad, bad


# ------------------------------------------------------------------ end-to-end gate
def oracle_frame(g, x, task, iou, **kw):
    """The round-fp16 oracle run end to end on letterboxed input x [1,S,S,3]: detections in
    letterbox space (segment: with their masks)."""
    I = interp.Interp(g, 1, round_fp16=True, **kw)
    I.set_input(x)
    I.run()
    heads = [(b[0], c[0], None if m is None else m[0], s) for b, c, m, s in I.heads_in]
    det = post.detect(heads, g.nc, 0.25, iou)
    if task == "segment":
        pt = [op.a for op in g.ops if op.kind == "MASKS"][0]
        det["masks"] = post.masks(I.view(pt)[0], det["coef"], det["box"], x.shape[1], x.shape[2])
    return det


def disagreement(ref, got):
    """The reference's matching of `got` against `ref`, reduced to the figures the gate
    bounds: unmatched reference detections above the score gate, kept-count difference,
    median |dscore| of matched pairs, median mask IoU (segment)."""
    m = post.match_e2e(ref, got, ref.get("masks"), got.get("masks"))
    return {"unmatched": m["unmatched_gated"], "kept": abs(m["n_ref"] - m["n_got"]),
            "dscore_med": float(np.median(m["dscore"])) if m["dscore"] else 1.0,
            "mask_med": float(np.median(m["mask_iou"])) if m["mask_iou"] else None,
            "fails": m["fails"], "n_ref": m["n_ref"], "n_got": m["n_got"]}


def noise_floor(g, x, task, iou, ref, seeds=4):
    """The oracle's disagreement with itself when only fp32 accumulation rounding changes:
    the worst of float64 accumulation and `seeds` other conv summation orders."""
    ds = [disagreement(ref, oracle_frame(g, x, task, iou, acc64=True))]
    ds += [disagreement(ref, oracle_frame(g, x, task, iou, order_seed=s)) for s in range(seeds)]
    fl = {k: max(d[k] for d in ds) for k in ("unmatched", "kept", "dscore_med", "fails")}
    fl["mask_med"] = min(d["mask_med"] for d in ds) if task == "segment" else None
    return fl


def e2e_bound(floor):
    return {"unmatched": 2 * floor["unmatched"] + 2, "kept": 2 * floor["kept"] + 2,
            "dscore_med": 2 * floor["dscore_med"] + 1e-3,
            "mask_med": None if floor["mask_med"] is None else floor["mask_med"] - 0.05}


def within(d, bound):
    ok = d["unmatched"] <= bound["unmatched"] and d["kept"] <= bound["kept"] and d["dscore_med"] <= bound["dscore_med"]
    if bound["mask_med"] is not None:
        ok = ok and d["mask_med"] is not None and d["mask_med"] >= bound["mask_med"]
    return ok
