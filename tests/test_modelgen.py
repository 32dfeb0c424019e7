"""Pins the synthetic model generator and the oracle's graph reader against numbers the
reference (and the public model cards it restates) hold: op counts (README.md:191),
channel tables (docs/specs/cls.md:29-55, seg.md:68-72, obb.md:50-52,
input-size.md:12-19) and parameter counts."""
import os

import numpy as np
import pytest

import modelgen
from oracle import graphfile, interp, post


def _count(info, kind=None):
    c = modelgen.count_ops(info)
    return c["total"] if kind is None else c.get(kind, 0)


def test_op_counts_reference():
    n = modelgen.build_model("yolo11", "n", calibrate=False)
    m = modelgen.build_model("yolo11", "m", calibrate=False)
    # README.md:191: 109 dumped ops for yolo11n, 141 for yolo11m (+3 DECODE each)
    assert _count(n) - _count(n, "DECODE") == 109
    assert _count(m) - _count(m, "DECODE") == 141
    assert _count(n, "CONV") == 87 and _count(n, "ADD") == 14 and _count(n, "ATTN") == 1
    x = modelgen.build_model("yolo11", "x", calibrate=False)
    assert _count(x) == 233 and _count(x, "CONV") == 173 and _count(x, "ATTN") == 2


@pytest.mark.parametrize("arch,scale,params", [("yolo11", "n", 2.62e6), ("yolo11", "s", 9.44e6),
                                               ("yolo11", "m", 20.09e6), ("yolo11", "l", 25.34e6),
                                               ("yolo11", "x", 56.92e6), ("yolov8", "n", 3.16e6),
                                               ("yolov8", "m", 25.90e6)])
def test_param_counts(arch, scale, params):
    """Public ultralytics parameter counts (after BN fuse, DFL excluded): within 1 %."""
    info = modelgen.build_model(arch, scale, calibrate=False)
    g = info.graph
    total = g.woff + g.boff
    assert abs(total - params) / params < 0.01, total


def test_channel_tables():
    g = modelgen.build_model("yolo11", "n", calibrate=False).graph
    convs = [op for op in g.ops if op[0] == "CONV"]
    # cls.md:33-39 (n): layer 2 cv1 32->32, bottleneck 16->8->16, cv2 48->64
    assert [(o[8], o[9]) for o in convs[2:6]] == [(32, 32), (16, 8), (8, 16), (48, 64)]
    # layer 6: cv1 128->128, C3k(cv1 64->32, ...), cv2 192->128
    l6 = [(o[8], o[9]) for o in convs[12:21]]
    assert l6[0] == (128, 128) and l6[1] == (64, 32) and l6[-1] == (192, 128)
    attn = [op for op in g.ops if op[0] == "ATTN"]
    assert [(a[3], a[4], a[5]) for a in attn] == [(2, 32, 64)]      # input-size.md:12-19
    gm = modelgen.build_model("yolo11", "m", calibrate=False).graph
    assert [(a[3], a[4], a[5]) for a in gm.ops if a[0] == "ATTN"] == [(4, 32, 64)]
    gx = modelgen.build_model("yolo11", "x", calibrate=False).graph
    assert [a[3] for a in gx.ops if a[0] == "ATTN"] == [6, 6]


@pytest.mark.parametrize("scale,npr,c4,c2,c3", [("n", 64, 32, 64, 80), ("s", 128, 32, 64, 128),
                                                ("m", 256, 64, 64, 256)])
def test_head_widths(scale, npr, c4, c2, c3):
    """seg.md:68-72 (npr, c4), obb.md:50-51 (c2 = 64; c3 = max(ch0, min(nc, 100)))."""
    g = modelgen.build_model("yolo11", scale, task="segment", calibrate=False).graph
    convs = [op for op in g.ops if op[0] == "CONV"]
    ps2 = [op for op in g.ops if op[0] == "PS2"][0]
    assert g.shape(ps2[2])[2] == npr
    dec = [op for op in g.ops if op[0] == "DECODESEG"][0]
    coef_conv = [o for o in convs if o[2] == dec[3]][0]
    assert coef_conv[8] == c4
    box_conv = [o for o in convs if o[2] == dec[1]][0]
    assert box_conv[8] == c2
    cls_conv = [o for o in convs if o[2] == dec[2]][0]
    assert cls_conv[8] == c3 and cls_conv[9] == 80


@pytest.mark.parametrize("scale,c3,c4", [("n", 64, 16), ("s", 128, 32), ("m", 256, 64)])
def test_obb_head(scale, c3, c4):
    """docs/specs/obb.md:13-61: layers 0..22 as detect, 11 head convs per level (cv2 3, cv3
    5, cv4 3), c2 = 64, c3 = max(ch0, min(nc, 100)), c4 = max(ch0 // 4, ne); cls padded to
    16 and angle to 8 channels; 16384 + 4096 + 1024 = 21504 anchors at 1024."""
    g = modelgen.build_model("yolo11", scale, task="obb", nc=15, imgsz=1024, calibrate=False).graph
    det = modelgen.build_model("yolo11", scale, calibrate=False).graph
    dec = [op for op in g.ops if op[0] == "DECODEOBB"]
    assert len(dec) == 3 and not [op for op in g.ops if op[0] == "DECODE"]
    n_conv = sum(op[0] == "CONV" for op in g.ops)
    assert n_conv == sum(op[0] == "CONV" for op in det.ops) + 9     # + cv4: 3 per level
    shapes = [g.shape(op[1]) for op in dec]
    assert [(h, w) for h, w, _ in shapes] == [(128, 128), (64, 64), (32, 32)]
    assert sum(h * w for h, w, _ in shapes) == 21504
    convs = [op for op in g.ops if op[0] == "CONV"]
    for _, box, cls, ang, st in dec:
        assert g.shape(box)[2] == 64 and g.shape(cls)[2] == 16 and g.shape(ang)[2] == 8
        cls_conv = [o for o in convs if o[2] == cls][0]
        ang_conv = [o for o in convs if o[2] == ang][0]
        assert cls_conv[8] == c3 and ang_conv[8] == c4 and ang_conv[3] == 1
    # the body (everything before the head's 3 x (8 convs + decode)) is the detect graph's
    body = len(det.ops) - 27
    assert [op[:1] + op[3:10] for op in g.ops[:body]] == [op[:1] + op[3:10] for op in det.ops[:body]]


def test_files_roundtrip(tmp_path):
    d = str(tmp_path / "n")
    info = modelgen.write_model(d, "yolo11", "n", calibrate=False) if False else \
        modelgen.write_model(d, "yolo11", "n")
    g = graphfile.load(d)
    assert len(g.ops) == len(info.graph.ops) and len(g.bufs) == len(info.graph.bufs)
    assert g.weights.size == info.graph.woff and g.bias.size == info.graph.boff
    assert os.path.getsize(os.path.join(d, "weights.f16")) == 2 * info.graph.woff
    for op in g.ops:
        if op.kind == "CONV":
            assert op.woff + op.Cout * op.k * op.k * op.Cin // op.g <= g.weights.size
            assert op.woff % 8 == 0


def test_calibrated_activations_are_unit_scale(tmp_path):
    """BN folded with measured statistics keeps every activation O(1) on a letterboxed
    frame (with running stats 0/1 the head collapses to a constant)."""
    d = str(tmp_path / "n")
    modelgen.write_model(d, "yolo11", "n")
    g = graphfile.load(d)
    I = interp.Interp(g, 1)
    I.set_input(post.letterbox(modelgen.synth_frame(810, 1080, 20, 1), 640, 640)[None])
    stds = []
    I.run(on_op=lambda k, op, t: stds.append(float(I.view(t).std())))
    assert 0.2 < min(stds[1:]) and max(stds) < 30


def test_fp16_storage_sensitivity(tmp_path):
    """Documents the noise floor the whole-frame GPU test is gated by: the oracle with
    fp16-rounded activations departs from the fp32 oracle by > 0.5 % at the class head
    after ~100 layers of random-init weights, and flips class ids."""
    d = str(tmp_path / "n")
    modelgen.write_model(d, "yolo11", "n", cls_bias=-8.0)
    g = graphfile.load(d)
    x = post.letterbox(modelgen.synth_frame(810, 1080, 20, 1), 640, 640)[None]
    runs = []
    for r16 in (False, True):
        I = interp.Interp(g, 1, round_fp16=r16)
        I.set_input(x)
        I.run()
        runs.append([(b[0], c[0], None, s) for b, c, _, s in I.heads_in])
    drift = max(post.rel_err(b[1], a[1]) for a, b in zip(runs[0], runs[1]))
    r32, r16 = post.detect(runs[0], 80), post.detect(runs[1], 80)
    n = min(len(r32["cls"]), len(r16["cls"]))
    agree = float((r32["cls"][:n] == r16["cls"][:n]).mean())
    print(f"fp16-storage drift {drift:.3e}, class agreement {agree:.3f}")
    assert drift > 5e-3 and agree < 0.95
