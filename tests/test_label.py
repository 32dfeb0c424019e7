"""Labeling client on the CPU: JSONL records and COCO export (client/label.py:57-71,118-163)
against the fake-engine server, COCO RLE against its column-major definition, the letterbox
mapping of masks back to original pixels, and OBB corner polygons."""
import json
import math

import numpy as np
import pytest
from PIL import Image

import yololabel
import yoloserve
from test_serve import FakeEngine, FakeServer


def _coco_rle_loop(m):
    out, cur, run = [], 0, 0
    for v in (m.T.ravel() != 0).tolist():
        if v == cur:
            run += 1
            continue
        out.append(run)
        cur, run = v, 1
    out.append(run)
    return out


@pytest.mark.parametrize("seed", range(4))
def test_coco_rle_column_major(seed):
    rng = np.random.default_rng(seed)
    m = (rng.random((9, 13)) < 0.4).astype(np.uint8)
    if seed == 3:
        m[0, 0] = 1
    r = yololabel.coco_rle(m)
    assert r["size"] == [9, 13] and r["counts"] == _coco_rle_loop(m) and sum(r["counts"]) == m.size
    # decode: runs alternate from background, column-major
    flat = np.repeat(np.arange(len(r["counts"])) % 2, r["counts"]).astype(np.uint8)
    assert np.array_equal(flat.reshape(13, 9).T, m)


def test_mask_to_original():
    rng = np.random.default_rng(1)
    m = (rng.random((10, 12)) < 0.5).astype(np.uint8)
    # scale 1, no padding: every mask pixel covers a 4x4 block of original pixels
    got = yololabel.mask_to_original(m, {"scale": 1.0, "top": 0, "left": 0}, 40, 48)
    assert np.array_equal(got, np.repeat(np.repeat(m, 4, 0), 4, 1))
    # scale 0.5 with a 8-pixel top pad: original row y sits at letterbox (y + 0.5) * 0.5 + 8
    got = yololabel.mask_to_original(m, {"scale": 0.5, "top": 8, "left": 0}, 20, 20)
    for y in (0, 7, 19):
        for x in (0, 5, 19):
            assert got[y, x] == m[int(((y + 0.5) * 0.5 + 8) // 4), int(((x + 0.5) * 0.5) // 4)]


def test_obb_corners():
    c = yololabel.obb_corners({"cx": 10.0, "cy": 20.0, "w": 4.0, "h": 2.0, "angle": 0.0})
    assert c == [(8.0, 19.0), (12.0, 19.0), (12.0, 21.0), (8.0, 21.0)]
    c = yololabel.obb_corners({"cx": 0.0, "cy": 0.0, "w": 4.0, "h": 2.0, "angle": math.pi / 2})
    xs, ys = [p[0] for p in c], [p[1] for p in c]
    assert max(xs) - min(xs) == pytest.approx(2.0) and max(ys) - min(ys) == pytest.approx(4.0)


def _write_png(path, bgr, h=12, w=16):
    img = np.zeros((h, w, 3), np.uint8)
    img[:] = bgr
    Image.fromarray(img[..., ::-1].copy()).save(path, format="PNG")


@pytest.fixture
def server():
    names = ["det", "seg", "cls", "obb"]
    engs = [FakeEngine(0), FakeEngine(3), FakeEngine(2), FakeEngine(1)]
    srv = FakeServer([yoloserve.Model(n, e, 4) for n, e in zip(names, engs)], target_ms=20.0, log=lambda *a: None)
    gs, port = yoloserve.grpc_server(srv, "127.0.0.1:0", decoders=8)
    yield f"127.0.0.1:{port}"
    gs.stop(0)
    srv.stop()


def test_label_jsonl_and_coco(server, tmp_path, capsys):
    paths = []
    for i in range(5):
        p = tmp_path / f"im{i}.png"
        _write_png(p, (3 + i, 40 + i, 70 + i), h=32, w=24)
        paths.append(str(p))
    out, cj = tmp_path / "l.jsonl", tmp_path / "c.json"
    assert yololabel.main(paths + ["--server", server, "--model", "seg", "-c", "4", "--out", str(out),
                                   "--coco", str(cj)]) == 0
    lines = [json.loads(l) for l in open(out)]
    assert [l["image"] for l in lines] == paths
    for i, l in enumerate(lines):
        b, g, r = 3 + i, 40 + i, 70 + i
        assert l["task"] == "segment" and l["mask_h"] == 8 and l["mask_w"] == 6
        assert l["letterbox"] == {"scale": 0.5, "top": b, "left": g}
        assert l["boxes"][0] == {"x1": b, "y1": g, "x2": r, "y2": r + 1, "score": 0.5, "cls": g % 80}
        assert len(l["masks"]) == 2 and sum(l["masks"][0]) == 48
    doc = json.load(open(cj))
    assert len(doc["images"]) == 5 and len(doc["annotations"]) == 10
    assert doc["images"][0]["height"] == 32 and doc["images"][0]["width"] == 24
    a = doc["annotations"][0]
    assert a["bbox"] == [3.0, 40.0, 67.0, 31.0] and a["area"] == 67.0 * 31.0 and a["category_id"] == 40 % 80
    seg = a["segmentation"]
    assert seg["size"] == [32, 24] and sum(seg["counts"]) == 32 * 24
    assert len(doc["categories"]) == 80
    # classify and obb records
    assert yololabel.main(paths[:2] + ["--server", server, "--model", "cls", "--out", str(out)]) == 0
    l0 = json.loads(open(out).readline())
    assert l0["task"] == "classify" and [c["id"] for c in l0["classes"]] == [3, 40, 70, 1, 2]
    assert yololabel.main(paths[:1] + ["--server", server, "--model", "obb", "--out", str(out), "--coco", str(cj)]) == 0
    l0 = json.loads(open(out).readline())
    assert l0["rboxes"][0]["cls"] == 3 and l0["task"] == "obb"
    doc = json.load(open(cj))
    assert len(doc["categories"]) == 15 and len(doc["annotations"][0]["segmentation"][0]) == 8
    # bench mode
    assert yololabel.main(paths[:1] + ["--server", server, "--bench", "20", "-c", "8"]) == 0
    out = capsys.readouterr().out
    assert "20 requests, 8 callers" in out and "img/s" in out and "server batch" in out
