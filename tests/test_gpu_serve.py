"""The gRPC server with real engines on the GPU: concurrent requests over 127.0.0.1 for a detect,
a segment and a classify model, served in-process and by two front-end processes sharing the
port (half the requests JPEG, decoded on the engine).  Every response is checked against a direct
engine handle run on the same decoded pixels, to the parity bar (same kept count, classes and
order; box IoU >= 0.99, |d score| <= 5e-3; mask IoU >= 0.99; same top-5), and that direct
run is itself held to the oracle: its input tensor equals the oracle's letterbox (classify:
resize + crop) of the decoded image bit for bit, its detections equal the oracle's decode +
NMS on the run's own head tensors exactly, its masks match the oracle's masks on the run's
proto (IoU >= 0.99), and its top-5 is the oracle's top-k of the run's probabilities.  (The
network between input and heads is held to the oracle op by op in test_gpu_configs.py.)"""
import io
from concurrent.futures import ThreadPoolExecutor

import grpc
import numpy as np
import pytest
from PIL import Image

import modelgen
import yolort
import yoloserve
from oracle import graphfile, post

pytestmark = pytest.mark.gpu
FLAGS = yolort.YOLO_NOTUNE


def _encode(img_bgr, fmt):
    buf = io.BytesIO()
    kw = {"quality": 92} if fmt == "JPEG" else {}
    Image.fromarray(img_bgr[..., ::-1].copy()).save(buf, format=fmt, **kw)
    return buf.getvalue()


def _to_original(geom, box):
    """Net-space boxes to original-image coordinates with yolo_get's float32 operations."""
    scale, top, left = (np.float32(v) for v in geom)
    b = box.astype(np.float32)
    return np.stack([(b[:, 0] - left) / scale, (b[:, 1] - top) / scale,
                     (b[:, 2] - left) / scale, (b[:, 3] - top) / scale], 1).astype(np.float64)


def _direct(eng, g, img):
    """One frame through a direct handle (upload, preprocess, run), checked against the oracle
    on that run's own tensors; returns the direct results."""
    dev = yolort.DeviceBuffer(img.nbytes)
    eng.upload(dev, img)
    h, w = img.shape[:2]
    if eng.task() == 2:
        eng.preprocess_cls(dev.ptr, h, w, 0)
    else:
        eng.preprocess(dev.ptr, h, w, 0)
    eng.run(1)
    S = eng.read(0, 1).shape[1]
    want_in = post.preprocess_cls(img, S) if eng.task() == 2 else post.letterbox(img, S, S)
    np.testing.assert_array_equal(eng.read(0, 1)[0], want_in)
    out = {"boxes": eng.get(0) if eng.task() != 2 else None}
    if eng.task() == 2:
        out["cls"] = eng.get_cls(0, 5)
        probs = eng.read([op.out for op in g.ops if op.kind == "SOFTMAX"][0], 1)[0, 0, 0].astype(np.float32)
        wid, wpr = post.topk(probs, 5)
        assert out["cls"][0].tolist() == wid.tolist()
        np.testing.assert_array_equal(out["cls"][1], wpr)
    else:
        heads = [(eng.read(op.a, 1)[0].astype(np.float32), eng.read(op.b, 1)[0].astype(np.float32),
                  eng.read(op.out, 1)[0].astype(np.float32) if op.kind == "DECODESEG" else None, op.stride)
                 for op in g.ops if op.kind in ("DECODE", "DECODESEG")]
        want = post.detect(heads, g.nc, 0.25, 0.45)
        got = out["boxes"]
        assert len(got) == len(want["score"])
        np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
        np.testing.assert_allclose(got[:, 4], want["score"], rtol=0, atol=2e-6)
        np.testing.assert_allclose(got[:, :4], _to_original(eng.slot_geom(0), want["box"]), rtol=0, atol=2e-3)
    if eng.task() == 3:
        out["masks"] = [eng.get_mask(0, j) for j in range(len(out["boxes"]))]
        out["geom"] = eng.slot_geom(0)
        proto = eng.read([op.a for op in g.ops if op.kind == "MASKS"][0], 1)[0].astype(np.float32)
        wm = post.masks(proto, want["coef"], want["box"], S, S)
        for j, m in enumerate(out["masks"]):
            assert _mask_iou(m, wm[j]) >= 0.99
    dev.free()
    return out


def _mask_iou(a, b):
    a, b = a != 0, b != 0
    u = int((a | b).sum())
    return 1.0 if u == 0 else int((a & b).sum()) / u


def _iou(a, b):
    ix = max(0.0, min(a[2], b[2]) - max(a[0], b[0]))
    iy = max(0.0, min(a[3], b[3]) - max(a[1], b[1]))
    inter = ix * iy
    u = (a[2] - a[0]) * (a[3] - a[1]) + (b[2] - b[0]) * (b[3] - b[1]) - inter
    return inter / u if u > 0 else 1.0


def test_batcher_queue_rules_and_stop(models):
    """The native worker's batching rules on one detect engine (max batch 4) and a target far
    in the future: requests below the max batch are held; the fourth fills the queue and the
    batch fires, each result equal to a batch-1 run of the same JPEG on a handle of the same
    max batch (so the same kernel choices); requests queued at
    stop are answered YOLO_BATCH_STOPPED (their tickets released), and later submits refused."""
    d = models("yolo11", "n")
    eng = yolort.Engine(d, 4, FLAGS)
    direct = yolort.Engine(d, 4, FLAGS)   # the same max batch: the same kernel choices
    frames = [modelgen.synth_frame(480, 640, 20, 700 + i) for i in range(6)]
    jpegs = [_encode(f, "JPEG") for f in frames]
    b = yolort.Batcher([eng], [4], target_ms=60000.0)
    try:
        for i in range(3):
            assert b.submit_jpeg(0, jpegs[i], i) == 0
        assert b.wait(300) == []                        # three of four: held
        assert b.submit_jpeg(0, jpegs[3], 3) == 0       # full: fires
        got = []
        while len(got) < 4:
            out = b.wait(5000)
            assert out, "the full batch was not answered"
            got += out
        for r in sorted(got, key=lambda r: r["tag"]):
            assert r["status"] == yolort.BATCH_OK and r["batch"] == 4 and r["model"] == 0
            img = yoloserve.decode_image(jpegs[r["tag"]])
            dev = yolort.DeviceBuffer(img.nbytes)
            direct.upload(dev, img)
            direct.preprocess(dev.ptr, img.shape[0], img.shape[1], 0)
            direct.run(1)
            want = direct.get(0)
            dev.free()
            assert r["rows"].shape == (len(want), 6)
            np.testing.assert_array_equal(r["rows"][:, :5], want[:, :5].astype(np.float32))
            np.testing.assert_array_equal(r["rows"][:, 5].astype(int), want[:, 5].astype(int))
        for i in (4, 5):
            assert b.submit_jpeg(0, jpegs[i], i) == 0
        assert b.wait(300) == []
        b.stop()
        left = []
        while True:
            out = b.wait(5000)
            if out is None:
                break
            left += out
        assert sorted(r["tag"] for r in left) == [4, 5]
        assert all(r["status"] == yolort.BATCH_STOPPED and len(r["rows"]) == 0 for r in left)
        assert b.submit_jpeg(0, jpegs[0], 9) == -1
    finally:
        b.stop()
        b.destroy()
        eng.close()
        direct.close()


@pytest.mark.parametrize("frontends,native", [(0, True), (2, True), (0, False)],
                         ids=["native", "native-frontends", "python-loop"])
def test_server_matches_direct_engine(models, frontends, native):
    dirs = {"det": models("yolo11", "n"), "seg": models("yolo11", "n", "segment"),
            "cls": models("yolo11", "n", "classify", imgsz=224, nc=1000)}
    limits = {"det": 4, "seg": 2, "cls": 3}
    served = [yoloserve.Model(n, yolort.Engine(d, limits[n], FLAGS), limits[n]) for n, d in dirs.items()]
    direct = {n: yolort.Engine(d, 1, FLAGS) for n, d in dirs.items()}
    graphs = {n: graphfile.load(d) for n, d in dirs.items()}
    srv = yoloserve.Server(served, target_ms=20.0, log=lambda *a: None, native=native)
    assert (srv.batcher is not None) == native
    gs, port = yoloserve.grpc_server(srv, "127.0.0.1:0", frontends=frontends)
    cl = yoloserve.Client(f"127.0.0.1:{port}")
    try:
        frames = [modelgen.synth_frame(480 + 40 * (i % 3), 640 + 64 * (i % 2), 20, 300 + i) for i in range(12)]
        route = [["det", "seg", "cls", ""][i % 4] for i in range(12)]
        fmt = ["JPEG" if i % 2 else "PNG" for i in range(12)]   # JPEG: decoded on the engine
        payload = [_encode(f, fm) for f, fm in zip(frames, fmt)]
        print(f"server ({frontends} front-end processes): 12 concurrent requests over det/seg/cls", flush=True)
        with ThreadPoolExecutor(12) as ex:
            resps = list(ex.map(lambda i: cl.detect(payload[i], route[i], timeout=120), range(12)))
        for i, r in enumerate(resps):
            name = route[i] or "det"
            img = yoloserve.decode_image(payload[i])          # PIL (the engine's JPEG decode equals it)
            want = _direct(direct[name], graphs[name], img)
            assert 1 <= r.batch <= limits[name]
            if name == "cls":
                assert r.task == "classify"
                ids, probs = want["cls"]
                assert [c.id for c in r.classes] == ids.tolist()
                assert np.abs(np.array([c.prob for c in r.classes]) - probs).max() <= 5e-3
                continue
            assert r.task == ("segment" if name == "seg" else "detect")
            wb = want["boxes"]
            assert len(r.boxes) == len(wb), (i, len(r.boxes), len(wb))
            for bx, w in zip(r.boxes, wb):
                assert bx.cls == int(w[5])
                assert abs(bx.score - w[4]) <= 5e-3
                assert _iou((bx.x1, bx.y1, bx.x2, bx.y2), w[:4]) >= 0.99
            if name == "seg":
                assert (r.mask_h, r.mask_w) == direct["seg"].mask_dim()
                sc, top, left = want["geom"]
                assert abs(r.lb_scale - sc) <= 1e-6 and (r.lb_top, r.lb_left) == (top, left)
                n = r.mask_h * r.mask_w
                for mk, wm in zip(r.masks, want["masks"]):
                    got = yoloserve.rle_decode(mk.rle, n).reshape(r.mask_h, r.mask_w)
                    assert _mask_iou(got, wm) >= 0.99
        # error paths through the real server
        with pytest.raises(grpc.RpcError) as ei:
            cl.detect(payload[0], "yolo-missing")
        assert ei.value.code() == grpc.StatusCode.INVALID_ARGUMENT
        with pytest.raises(grpc.RpcError) as ei:
            cl.detect(b"\x89PNG\r\n\x1a\nbroken", "det")
        assert ei.value.details() == "image decode failed"
        # a JPEG whose headers parse but whose entropy-coded data is cut short: the engine's
        # decoder refuses it, and only that request fails
        jp = payload[1]
        with pytest.raises(grpc.RpcError) as ei:
            cl.detect(jp[:len(jp) // 2], "det")
        assert ei.value.details() == "image decode failed"
        assert len(cl.detect(jp, "det").boxes) == len(_direct(direct["det"], graphs["det"],
                                                              yoloserve.decode_image(jp))["boxes"])
        # a short closed-loop load on the detect model
        stats = yoloserve.bench(f"127.0.0.1:{port}", payload[:8:4], "det", concurrency=16, seconds=2.0)
        print(f"server bench (yolo11n, 16 callers, PNG 480-560x640-704): {stats}", flush=True)
        assert stats["requests"] > 0
    finally:
        cl.close()
        gs.stop(0)
        srv.stop()
        for m in served:
            m.eng.close()
        for e in direct.values():
            e.close()
