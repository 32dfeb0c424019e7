"""The labeling client against the real server on the GPU (needs an MI355X): `yololabel`
labels JPEG and PNG files through a detect and a segment model; every JSONL record equals a
direct engine run on the same decoded pixels to the parity bar (same kept count, classes and
order, box IoU >= 0.99, |d score| <= 5e-3, mask IoU >= 0.99), that direct run being held to
the oracle as in test_gpu_serve.py, and the COCO export carries the same boxes (xywh in
original pixels) and masks of the image's size."""
import json
import os

import numpy as np
import pytest
from PIL import Image

import modelgen
import yololabel
import yolort
import yoloserve
from oracle import graphfile
from test_gpu_serve import FLAGS, _direct, _iou, _mask_iou

pytestmark = pytest.mark.gpu


def _write(path, bgr, fmt):
    kw = {"quality": 90} if fmt == "JPEG" else {}
    Image.fromarray(bgr[..., ::-1].copy()).save(path, format=fmt, **kw)


def test_label_client_against_real_server(models, tmp_path):
    dirs = {"det": models("yolo11", "n"), "seg": models("yolo11", "n", "segment")}
    served = [yoloserve.Model(n, yolort.Engine(d, 4, FLAGS), 4) for n, d in dirs.items()]
    direct = {n: yolort.Engine(d, 1, FLAGS) for n, d in dirs.items()}
    graphs = {n: graphfile.load(d) for n, d in dirs.items()}
    srv = yoloserve.Server(served, target_ms=20.0, log=lambda *a: None)
    gs, port = yoloserve.grpc_server(srv, "127.0.0.1:0")
    try:
        paths = []
        for i in range(6):
            p = tmp_path / (f"f{i}.jpg" if i % 3 else f"f{i}.png")
            _write(p, modelgen.synth_frame(360 + 40 * i, 480 + 32 * i, 15, 900 + i), "JPEG" if i % 3 else "PNG")
            paths.append(str(p))
        for name in ("det", "seg"):
            out, cj = tmp_path / f"{name}.jsonl", tmp_path / f"{name}.json"
            print(f"label {len(paths)} images with {name}", flush=True)
            assert yololabel.main(paths + ["--server", f"127.0.0.1:{port}", "--model", name, "-c", "6",
                                           "--out", str(out), "--coco", str(cj)]) == 0
            recs = [json.loads(line) for line in open(out)]
            doc = json.load(open(cj))
            assert [r["image"] for r in recs] == paths
            ann = {}
            for a in doc["annotations"]:
                ann.setdefault(a["image_id"], []).append(a)
            for p, rec in zip(paths, recs):
                img = yoloserve.decode_image(open(p, "rb").read())
                want = _direct(direct[name], graphs[name], img)
                wb = want["boxes"]
                assert rec["task"] == ("segment" if name == "seg" else "detect")
                assert len(rec["boxes"]) == len(wb), (p, len(rec["boxes"]), len(wb))
                for b, w in zip(rec["boxes"], wb):
                    assert b["cls"] == int(w[5]) and abs(b["score"] - w[4]) <= 5e-3
                    assert _iou((b["x1"], b["y1"], b["x2"], b["y2"]), w[:4]) >= 0.99
                if name == "seg" and rec["boxes"]:          # mask fields come with masks only
                    mh, mw = rec["mask_h"], rec["mask_w"]
                    assert len(rec["masks"]) == len(rec["boxes"])
                    for runs, wm in zip(rec["masks"], want["masks"]):
                        got = yoloserve.rle_decode(runs, mh * mw).reshape(mh, mw)
                        assert _mask_iou(got, wm) >= 0.99
                # COCO: one annotation per box, bbox = xywh of the record's box
                im = next(x for x in doc["images"] if x["file_name"] == os.path.basename(p))
                assert (im["height"], im["width"]) == img.shape[:2]
                got_ann = ann.get(im["id"], [])
                assert len(got_ann) == len(rec["boxes"])
                for a, b in zip(got_ann, rec["boxes"]):
                    np.testing.assert_allclose(a["bbox"], [b["x1"], b["y1"], b["x2"] - b["x1"], b["y2"] - b["y1"]],
                                               rtol=0, atol=0.01)
                    if name == "seg":
                        assert a["segmentation"]["size"] == list(img.shape[:2])
                        assert sum(a["segmentation"]["counts"]) == img.shape[0] * img.shape[1]
    finally:
        gs.stop(0)
        srv.stop()
        for m in served:
            m.eng.close()
        for e in direct.values():
            e.close()
