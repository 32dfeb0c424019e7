"""Pins the torch fp32 per-op CPU path (oracle/torchref.py, bench.py's CPU baseline) against
the numpy interpreter (oracle/interp.py): every op, fed the numpy interpreter's inputs,
agrees to fp32 rounding, and whole frames give the same detections."""
import numpy as np
import pytest
import torch

import modelgen
from oracle import graphfile, interp, post, torchref


def _nhwc(t):
    return t.permute(0, 2, 3, 1).numpy()


@pytest.mark.parametrize("scale,task,nc,imgsz", [("n", "detect", 80, 640), ("n", "segment", 80, 320),
                                                 ("n", "classify", 1000, 224), ("n", "obb", 15, 320)])
def test_every_op_matches_numpy_interp(models, scale, task, nc, imgsz):
    d = models("yolo11", scale, task, imgsz=imgsz, nc=nc)
    g = graphfile.load(d)
    x = post.letterbox(modelgen.synth_frame(300, 400, 20, 3), imgsz, imgsz)[None].astype(np.float32)
    ref = interp.Interp(g, 1)
    ref.set_input(x)
    tr = torchref.TorchRef(g, 1)
    tr.set_input(x)
    np.testing.assert_array_equal(_nhwc(tr.view(0)), ref.view(0))
    worst = 0.0
    with torch.no_grad():
        for k, op in enumerate(g.ops):
            for t in (op.a, op.b, op.out):
                if t >= 0:
                    tr.view(t).copy_(torch.from_numpy(ref.view(t)).permute(0, 3, 1, 2))
            out = ref.run_op(op)
            tr.run_op(k)
            if out is None:
                continue
            rel = post.rel_err(_nhwc(tr.view(out)), ref.view(out))
            worst = max(worst, rel)
            assert rel <= 2e-5, (k, op.kind, rel)
    print(f"{task}: worst per-op deviation {worst:.2e}")


def test_frame_detections_match_numpy_interp(models):
    d = models("yolo11", "n")
    g = graphfile.load(d)
    img = modelgen.synth_frame(810, 1080, 20, 1)
    want_x = post.letterbox(img, 640, 640)[None]
    ref = interp.Interp(g, 1)
    ref.set_input(want_x)
    ref.run()
    want = post.detect([(b[0], c[0], None, s) for b, c, _, s in ref.heads_in], 80)
    tr = torchref.TorchRef(g, 1)
    got = torchref.frame(tr, img, 640, 80)
    heads_t = tr.heads_nhwc(0)
    for (bt, ct, _, _), (bn, cn, _, _) in zip(heads_t, ref.heads_in):
        assert post.rel_err(ct, cn[0]) <= 1e-3 and post.rel_err(bt, bn[0]) <= 1e-3
    assert len(got["score"]) == len(want["score"])
    np.testing.assert_array_equal(got["cls"], want["cls"])
    np.testing.assert_allclose(got["score"], want["score"], atol=1e-4)
