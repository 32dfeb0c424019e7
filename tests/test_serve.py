"""Detection server on the CPU: the wire schema against hand-encoded protobuf bytes (field
numbers and types of proto/yolo.proto:9-56), RLE masks (server/serve.cpp:193-203), the
batcher's choice (server/serve.cpp:163-191), dir specs (:365-372), and a real gRPC round trip
on 127.0.0.1 with a fake engine that derives each slot's results from that slot's pixels, so
request -> slot -> response mapping, task fields and error codes are checked without a GPU."""
import io
import struct
import threading
import time
from concurrent.futures import ThreadPoolExecutor

import grpc
import numpy as np
import pytest
from PIL import Image

import yoloproto as pb
import yoloserve


# ------------------------------------------------------------------ wire format

def _varint(v):
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def _key(num, wt):
    return _varint(num << 3 | wt)


def _f32(num, x):
    return _key(num, 5) + struct.pack("<f", x)


def _vint(num, v):
    return _key(num, 0) + _varint(v & 0xFFFFFFFFFFFFFFFF)


def _ld(num, payload):
    return _key(num, 2) + _varint(len(payload)) + payload


def test_wire_request():
    got = pb.DetectRequest(image=b"\xff\xd8xyz", model="yolo11n-seg").SerializeToString()
    assert got == _ld(1, b"\xff\xd8xyz") + _ld(2, b"yolo11n-seg")
    assert pb.DetectRequest.FromString(got).model == "yolo11n-seg"


def test_wire_response_every_field():
    r = pb.DetectResponse(queue_ms=1.5, infer_ms=2.25, batch=3, task="segment", mask_h=160, mask_w=120,
                          lb_scale=0.5, lb_top=-2, lb_left=7)
    r.boxes.add(x1=1.0, y1=2.0, x2=3.0, y2=4.0, score=0.75, cls=5)
    r.rboxes.add(cx=1.0, cy=2.0, w=3.0, h=4.0, angle=0.5, score=0.25, cls=2)
    r.classes.add(id=9, prob=0.125)
    r.masks.add(rle=[0, 300, 2])
    box = _f32(1, 1.0) + _f32(2, 2.0) + _f32(3, 3.0) + _f32(4, 4.0) + _f32(5, 0.75) + _vint(6, 5)
    rbox = _f32(1, 1.0) + _f32(2, 2.0) + _f32(3, 3.0) + _f32(4, 4.0) + _f32(5, 0.5) + _f32(6, 0.25) + _vint(7, 2)
    cls = _vint(1, 9) + _f32(2, 0.125)
    mask = _ld(1, _varint(0) + _varint(300) + _varint(2))        # proto3: packed
    want = (_ld(1, box) + _f32(2, 1.5) + _f32(3, 2.25) + _vint(4, 3) + _ld(5, b"segment") + _ld(6, rbox)
            + _ld(7, cls) + _ld(8, mask) + _vint(9, 160) + _vint(10, 120) + _f32(11, 0.5) + _vint(12, -2)
            + _vint(13, 7))
    got = r.SerializeToString()
    assert got == want
    back = pb.DetectResponse.FromString(want)
    assert back.lb_top == -2 and list(back.masks[0].rle) == [0, 300, 2] and back.boxes[0].cls == 5


# ------------------------------------------------------------------ pure helpers

def _rle_loop(m):
    out, cur, run = [], 0, 0
    for v in m.ravel().tolist():
        if v == cur:
            run += 1
            continue
        out.append(run)
        cur, run = v, 1
    out.append(run)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_rle_matches_loop_and_roundtrips(seed):
    rng = np.random.default_rng(seed)
    m = (rng.random((17, 23)) < [0.0, 1.0, 0.5, 0.05, 0.95, 0.5][seed]).astype(np.uint8)
    if seed == 5:
        m[0, 0] = 1
    runs = yoloserve.rle_encode(m)
    assert runs.tolist() == _rle_loop(m)
    assert runs.sum() == m.size
    assert np.array_equal(yoloserve.rle_decode(runs, m.size).reshape(m.shape), m)


def test_rle_edges():
    assert yoloserve.rle_encode(np.zeros(0, np.uint8)).tolist() == [0]
    assert yoloserve.rle_encode(np.ones(4, np.uint8)).tolist() == [0, 4]
    assert yoloserve.rle_encode(np.array([0, 0, 1], np.uint8)).tolist() == [2, 1]
    with pytest.raises(ValueError):
        yoloserve.rle_decode([2, 1], 4)


def test_parse_dir_spec():
    assert yoloserve.parse_dir_spec("build/yolo11n", 16) == ("build/yolo11n", "yolo11n", 16)
    assert yoloserve.parse_dir_spec("build/yolo11n-seg:4", 16) == ("build/yolo11n-seg", "yolo11n-seg", 4)
    assert yoloserve.parse_dir_spec("host:1/yolo11n", 16) == ("host:1/yolo11n", "yolo11n", 16)
    assert yoloserve.parse_dir_spec("m/", 8) == ("m/", "m", 8)


def test_pick_queue():
    now = 100.0
    pick = yoloserve.pick_queue
    assert pick([(0, 0.0, 4, 1.0)], now, 50, 2) == (-1, False, float("inf"))
    # one young request: wait, with slack = 50 - 10 - 5 - 2 - 1
    i, fire, slack = pick([(1, now - 0.010, 4, 5.0)], now, 50, 2)
    assert (i, fire) == (0, False) and slack == pytest.approx(32.0)
    # full queue fires at once
    assert pick([(4, now, 4, 5.0)], now, 50, 2)[:2] == (0, True)
    # slack used up fires
    assert pick([(1, now - 0.045, 4, 5.0)], now, 50, 2)[:2] == (0, True)
    # a ready queue beats a less urgent waiting one; among ready, the least slack
    qs = [(1, now - 0.001, 4, 5.0), (4, now - 0.001, 4, 5.0), (2, now - 0.046, 8, 5.0)]
    i, fire, _ = pick(qs, now, 50, 2)
    assert fire and i == 2
    qs = [(1, now - 0.001, 4, 5.0), (4, now, 4, 5.0)]
    assert pick(qs, now, 50, 2)[:2] == (1, True)
    # both waiting: the least slack is the one to time the wait on
    qs = [(1, now - 0.001, 4, 5.0), (1, now - 0.020, 4, 5.0)]
    assert pick(qs, now, 50, 2)[:2] == (1, False)


def test_decode_image_formats():
    img = np.zeros((5, 7, 3), np.uint8)
    img[..., 0], img[..., 1], img[..., 2] = 10, 20, 30      # BGR
    buf = io.BytesIO()
    Image.fromarray(img[..., ::-1]).save(buf, format="PNG")
    got = yoloserve.decode_image(buf.getvalue())
    assert got.shape == (5, 7, 3) and np.array_equal(got, img)
    assert yoloserve.decode_image(b"not an image") is None
    assert yoloserve.decode_image(b"") is None


# ------------------------------------------------------------------ gRPC round trip, fake engine

class FakeEngine:
    """The yolort.Engine calls the server makes; results are functions of each slot's pixel."""

    def __init__(self, task):
        self._task = task
        self.staged, self.done, self.batches = {}, {}, []
        self.lock = threading.Lock()
        self.worker_threads = set()

    def task(self):
        return self._task

    def mask_dim(self):
        return (8, 6)

    def exec_ms(self, B):
        return 0.5

    def stage(self, slot, img):
        self.worker_threads.add(threading.get_ident())
        self.staged[slot] = img

    def run_async(self, B):
        self.worker_threads.add(threading.get_ident())
        self.batches.append(B)
        self.pending = {s: self.staged.get(s) for s in range(B)}

    def sync(self):
        self.done = self.pending

    def _bgr(self, slot):
        return [int(v) for v in self.done[slot][0, 0]]

    def get(self, slot):
        b, g, r = self._bgr(slot)
        return np.array([[b, g, r, r + 1.0, 0.5, g % 80], [b + 1.0, g, r, r + 2.0, 0.25, 1]], np.float64)

    def get_obb(self, slot):
        b, g, r = self._bgr(slot)
        return np.array([[b, g, r, 4.0, 0.5, 0.75, 3]], np.float64)

    def get_cls(self, slot, k):
        b, g, r = self._bgr(slot)
        return np.array([b, g, r, 1, 2][:k], np.int32), np.array([0.5, 0.25, 0.125, 0.0625, 0.03125][:k], np.float32)

    def slot_geom(self, slot):
        b, g, r = self._bgr(slot)
        return 0.5, b, g

    def get_mask(self, slot, j):
        b = self._bgr(slot)[0]
        m = np.zeros((8, 6), np.uint8)
        m[: (b + j) % 8] = 1
        return m


class FakeServer(yoloserve.Server):
    def _stage(self, m, slot, img):
        m.eng.stage(slot, img)


def _png(bgr):
    img = np.zeros((12, 16, 3), np.uint8)
    img[:] = bgr
    buf = io.BytesIO()
    Image.fromarray(img[..., ::-1].copy()).save(buf, format="PNG")
    return buf.getvalue()


def test_grpc_roundtrip_fake_engines():
    names = ["det", "seg", "cls", "obb"]
    engs = [FakeEngine(0), FakeEngine(3), FakeEngine(2), FakeEngine(1)]
    models = [yoloserve.Model(n, e, 4) for n, e in zip(names, engs)]
    srv = FakeServer(models, target_ms=40.0, log=lambda *a: None)
    gs, port = yoloserve.grpc_server(srv, "127.0.0.1:0", workers=48)
    cl = yoloserve.Client(f"127.0.0.1:{port}")
    try:
        colors = [(10 + i, 20 + 2 * i, 30 + 3 * i) for i in range(24)]
        route = ["" if i % 8 == 0 else names[i % 4] for i in range(24)]
        with ThreadPoolExecutor(24) as ex:
            resps = list(ex.map(lambda i: cl.detect(_png(colors[i]), route[i]), range(24)))
        for i, r in enumerate(resps):
            b, g, rr = colors[i]
            task = {"": "detect", "det": "detect", "seg": "segment", "cls": "classify", "obb": "obb"}[route[i]]
            assert r.task == task
            assert 1 <= r.batch <= 4 and r.queue_ms >= 0 and r.infer_ms >= 0
            if task in ("detect", "segment"):
                assert len(r.boxes) == 2 and not r.rboxes and not r.classes
                bx = r.boxes[0]
                assert (bx.x1, bx.y1, bx.x2, bx.y2, bx.cls) == (b, g, rr, rr + 1, g % 80)
                assert bx.score == 0.5
            if task == "segment":
                assert (r.mask_h, r.mask_w, r.lb_scale, r.lb_top, r.lb_left) == (8, 6, 0.5, b, g)
                assert len(r.masks) == 2
                for j, mk in enumerate(r.masks):
                    want = np.zeros((8, 6), np.uint8)
                    want[: (b + j) % 8] = 1
                    assert np.array_equal(yoloserve.rle_decode(mk.rle, 48).reshape(8, 6), want)
            elif task == "detect":
                assert not r.masks and r.mask_h == 0
            if task == "classify":
                assert [c.id for c in r.classes] == [b, g, rr, 1, 2] and not r.boxes
                assert r.classes[0].prob == 0.5
            if task == "obb":
                rb = r.rboxes[0]
                assert (rb.cx, rb.cy, rb.w, rb.h, rb.angle, rb.score, rb.cls) == (b, g, rr, 4, 0.5, 0.75, 3)
        # batches: never above a model's limit, and concurrent requests were batched together
        allb = [bb for e in engs for bb in e.batches]
        assert max(allb) <= 4 and sum(allb) == 24 and max(allb) > 1
        # every engine call came from the one worker thread
        assert len(set().union(*[e.worker_threads for e in engs])) == 1
        # errors: unknown model, undecodable image
        with pytest.raises(grpc.RpcError) as ei:
            cl.detect(_png((1, 2, 3)), "nope")
        assert ei.value.code() == grpc.StatusCode.INVALID_ARGUMENT and "unknown model: nope" in ei.value.details()
        with pytest.raises(grpc.RpcError) as ei:
            cl.detect(b"\x00garbage", "det")
        assert ei.value.code() == grpc.StatusCode.INVALID_ARGUMENT and ei.value.details() == "image decode failed"
        # a JPEG goes through the same decoder (lossy: colours within a few levels)
        buf = io.BytesIO()
        Image.fromarray(np.full((32, 32, 3), (90, 60, 30), np.uint8)).save(buf, format="JPEG", quality=95)
        r = cl.detect(buf.getvalue(), "det")
        assert abs(r.boxes[0].x1 - 30) <= 3 and abs(r.boxes[0].y2 - 90) <= 3
    finally:
        cl.close()
        gs.stop(0)
        srv.stop()
    # after stop, submissions fail fast instead of hanging
    req = srv.submit(_png((1, 1, 1)), "det")
    assert req.done.wait(1.0) and req.error == "server shutting down"


def test_deadline_fires_partial_batch():
    """A lone request is answered once its slack is used up, not when a batch fills."""
    eng = FakeEngine(0)
    srv = FakeServer([yoloserve.Model("det", eng, 16)], target_ms=30.0, log=lambda *a: None)
    try:
        t0 = time.monotonic()
        req = srv.submit(_png((5, 6, 7)))
        assert req.done.wait(5.0) and req.error is None
        waited = (time.monotonic() - t0) * 1e3
        assert eng.batches == [1]
        # fired after about target - exec - decode estimate - margin (30 - 0.5 - 2 - 1 ms)
        assert 15.0 <= waited <= 2000.0
        assert req.resp.batch == 1 and req.resp.boxes[0].x1 == 5
    finally:
        srv.stop()
