"""The end-to-end gate on the CPU: the reference's matching rule (test/compare_seg.py:61-100)
pinned on hand cases, the oracle's own whole-frame disagreement under fp32 rounding changes
(the noise floor the GPU frame is held to), and a planted systematic error in the oracle
that the gate must reject although every op stays far inside the per-op bar."""
import numpy as np
import pytest

import modelgen
from oracle import graphfile, interp, post

import _frame_gate as fg


def _dets(rows):
    a = np.asarray(rows, np.float64).reshape(-1, 6)
    return {"box": a[:, :4], "score": a[:, 4], "cls": a[:, 5].astype(int)}


def test_match_rule_hand_cases():
    ref = _dets([[0, 0, 10, 10, 0.9, 1],      # matched (IoU 0.81), dscore 0.01, corner 0.5
                 [20, 20, 30, 30, 0.8, 2],    # only a class-3 box there: unmatched, gated
                 [40, 40, 50, 50, 0.26, 1],   # unmatched, below the 0.27 score gate
                 [60, 60, 70, 70, 0.5, 1],    # IoU exactly 0.8 with its candidate: unmatched
                 [80, 80, 90, 90, 0.7, 4]])   # matched, |dscore| 0.03 > 0.02: pair failure
    got = _dets([[0, 0, 10, 9.5, 0.91, 1], [20, 20, 30, 30, 0.8, 3], [60, 62, 70, 70, 0.5, 1],
                 [80, 80, 90, 90, 0.73, 4]])
    m = post.match_e2e(ref, got)
    assert (m["n_ref"], m["n_got"]) == (5, 4)
    assert m["unmatched"] == 3 and m["unmatched_gated"] == 2
    assert m["pair_fail"] == 1 and m["fails"] == 3
    np.testing.assert_allclose(m["dscore"], [0.01, 0.03], atol=1e-12)
    np.testing.assert_allclose(m["dbox"], [0.5, 0.0])
    # one candidate serves one reference detection; the better IoU wins, first on ties
    ref2 = _dets([[0, 0, 10, 10, 0.9, 0], [0, 0, 10, 10, 0.8, 0]])
    got2 = _dets([[0, 0, 10, 10, 0.9, 0], [0, 0, 10, 10, 0.8, 0]])
    m2 = post.match_e2e(ref2, got2)
    assert m2["unmatched"] == 0 and m2["dscore"] == [0.0, 0.0]
    # masks: IoU below 0.95 fails the pair
    mk = np.zeros((1, 8, 8), np.uint8)
    mk[0, :4] = 1
    mg = mk.copy()
    mg[0, 4, :2] = 1
    m3 = post.match_e2e(_dets([[0, 0, 10, 10, 0.9, 0]]), _dets([[0, 0, 10, 10, 0.9, 0]]), mk, mg)
    assert m3["mask_iou"] == [32 / 34] and m3["pair_fail"] == 1


CASES = {
    "C0": ("n", "detect", lambda: modelgen.synth_frame(810, 1080, 20, 1), 0.45),
    "C2": ("m", "detect", lambda: modelgen.synth_frame(1080, 1920, 20, 2), 0.7),
    "C4": ("n", "segment", lambda: modelgen.synth_polygons(640, 640, 30, 4), 0.45),
}


@pytest.mark.parametrize("case", list(CASES))
def test_noise_floor_and_planted_error(models, case, monkeypatch):
    """The oracle against itself: identical runs agree exactly; changing only the rounding
    of fp32 accumulations moves some detections (the floor, non-zero); a 0.1 % gain on every
    conv output -- per op far inside the 1.5 % bar -- lands well outside the gate."""
    scale, task, frame, iou = CASES[case]
    g = graphfile.load(models("yolo11", scale, task))
    x = post.letterbox(frame(), 640, 640)[None].astype(np.float32)
    ref = fg.oracle_frame(g, x, task, iou)
    same = fg.disagreement(ref, fg.oracle_frame(g, x, task, iou))
    assert same["unmatched"] == 0 and same["kept"] == 0 and same["dscore_med"] == 0.0
    floor = fg.noise_floor(g, x, task, iou, ref)
    bound = fg.e2e_bound(floor)
    print(case, "floor", floor, "bound", bound, flush=True)
    assert floor["fails"] > 0            # the rounding alone changes whole-frame detections
    orig = interp.conv2d_nhwc
    monkeypatch.setattr(interp, "conv2d_nhwc", lambda *a, **k: (orig(*a, **k) * np.float32(1.001)).astype(np.float32))
    planted = fg.disagreement(ref, fg.oracle_frame(g, x, task, iou))
    print(case, "planted 0.1% conv gain", planted, flush=True)
    assert not fg.within(planted, bound)
    assert planted["unmatched"] > 3 * bound["unmatched"]
