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


class _ArrayPool:
    """The pinned pool's take/give over plain numpy buffers."""

    class Buf:
        def __init__(self, n):
            self.array = np.full(n, 77, np.uint8)

    def __init__(self):
        self.out = 0

    def take(self, n):
        self.out += 1
        return self.Buf(n + 13)            # larger than asked, as pooled buffers are

    def give(self, b):
        self.out -= 1


@pytest.mark.parametrize("mode", ["RGB", "L", "RGBA", "P"])
@pytest.mark.parametrize("zero_copy", [True, False])
def test_decode_rgbx_into(mode, zero_copy, monkeypatch):
    rng = np.random.default_rng(5)
    rgb = rng.integers(0, 256, (9, 13, 3), dtype=np.uint8)
    im = Image.fromarray(rgb)
    im = im.convert(mode) if mode != "RGBA" else Image.fromarray(np.dstack([rgb, rgb[..., :1]]), "RGBA")
    buf = io.BytesIO()
    im.save(buf, format="PNG")
    want_rgb = np.asarray(im.convert("RGB"))
    if not zero_copy:
        monkeypatch.setattr(yoloserve, "_rgbx_view", lambda im, n: None)
    else:
        assert yoloserve._rgbx_view(im.convert("RGB"), 9 * 13) is not None   # PIL exports it here
    pool = _ArrayPool()
    got = yoloserve.decode_rgbx_into(buf.getvalue(), pool)
    assert got is not None and pool.out == 1
    b, hw = got
    assert hw == (9, 13)
    px = b.array[:9 * 13 * 4].reshape(9, 13, 4)
    assert np.array_equal(px[..., :3], want_rgb)
    # the same pixels as the BGR decode, channel-reversed
    assert np.array_equal(px[..., 2::-1], yoloserve.decode_image(buf.getvalue()))
    assert np.all(b.array[9 * 13 * 4:] == 77)                         # nothing past the frame


def test_decode_rgbx_into_jpeg_and_failures():
    rng = np.random.default_rng(6)
    rgb = rng.integers(0, 256, (40, 56, 3), dtype=np.uint8)
    buf = io.BytesIO()
    Image.fromarray(rgb).save(buf, format="JPEG", quality=85)
    pool = _ArrayPool()
    b, hw = yoloserve.decode_rgbx_into(buf.getvalue(), pool)
    assert hw == (40, 56)
    px = b.array[:40 * 56 * 4].reshape(40, 56, 4)
    assert np.array_equal(px[..., 2::-1], yoloserve.decode_image(buf.getvalue()))
    pool = _ArrayPool()
    assert yoloserve.decode_rgbx_into(b"not an image", pool) is None
    assert yoloserve.decode_rgbx_into(b"", pool) is None
    assert pool.out == 0


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


@pytest.mark.parametrize("frontends", [0, 2])
def test_grpc_roundtrip_fake_engines(frontends):
    """In-process asyncio server (frontends=0) and two front-end processes sharing the port
    (requests and results over pipes to this process, which keeps the engines)."""
    names = ["det", "seg", "cls", "obb"]
    engs = [FakeEngine(0), FakeEngine(3), FakeEngine(2), FakeEngine(1)]
    models = [yoloserve.Model(n, e, 4) for n, e in zip(names, engs)]
    srv = FakeServer(models, target_ms=40.0, log=lambda *a: None)
    gs, port = yoloserve.grpc_server(srv, "127.0.0.1:0", decoders=4, frontends=frontends)
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
        got = req.message()
        assert got.batch == 1 and got.boxes[0].x1 == 5
    finally:
        srv.stop()


def test_wire_boxes_match_protobuf():
    """The numpy wire encoding of boxes / rotated boxes parses to the same messages as the
    protobuf-built ones: 1- and 2-byte class varints, zeros, negatives, fp32 rounding, empty
    lists; ids beyond two varint bytes fall back (None)."""
    rng = np.random.default_rng(3)
    for n in (0, 1, 7, 300):
        d = rng.normal(0, 500, (n, 6))
        d[:, 5] = rng.integers(0, 1024, n)
        if n:
            d[0, :5] = 0.0
            d[-1, 5] = 127
        want = pb.DetectResponse(task="detect", batch=3)
        for x1, y1, x2, y2, s, c in d.tolist():
            want.boxes.add(x1=x1, y1=y1, x2=x2, y2=y2, score=s, cls=int(c))
        got = pb.DetectResponse.FromString(pb.DetectResponse(task="detect", batch=3).SerializeToString() +
                                           yoloserve.boxes_wire(d))
        assert got == want
        rb = rng.normal(0, 100, (n, 7))
        rb[:, 6] = rng.integers(0, 200, n)
        want = pb.DetectResponse()
        for cx, cy, w, h, a, s, c in rb.tolist():
            want.rboxes.add(cx=cx, cy=cy, w=w, h=h, angle=a, score=s, cls=int(c))
        got = pb.DetectResponse.FromString(yoloserve.rboxes_wire(rb))
        assert got == want
    assert yoloserve.boxes_wire(np.array([[0, 0, 1, 1, 0.5, 1 << 14]], float)) is None
    assert yoloserve.boxes_wire(np.array([[0, 0, 1, 1, 0.5, -1]], float)) is None


class _FailingEngine(FakeEngine):
    """Raises while fetching the results of its second batch."""

    def get(self, slot):
        if len(self.batches) >= 2:
            raise RuntimeError("device lost")
        return super().get(slot)


def test_engine_failure_answers_every_request():
    """An engine failure while finishing a batch answers that batch and the one collected
    behind it with an error (no handler waits forever), and later requests fail fast."""
    eng = _FailingEngine(0)
    srv = FakeServer([yoloserve.Model("det", eng, 2)], target_ms=5.0, log=lambda *a: None)
    try:
        reqs = [srv.submit(_png((i, i, i))) for i in range(8)]
        for r in reqs:
            assert r.done.wait(10.0)
        errs = [r.error for r in reqs]
        assert any(e and e.startswith("engine failure") for e in errs)
        assert all(e is None or e.startswith("engine failure") or e == "server shutting down" for e in errs)
        late = srv.submit(_png((1, 2, 3)))
        assert late.done.wait(1.0) and late.error == "server shutting down"
    finally:
        srv.stop()


def test_frontend_connection_malformed_message():
    """A malformed message on a front-end connection closes that connection (the front-end
    sees EOF and answers UNAVAILABLE) instead of stopping its reader silently; a valid request
    on another connection is still served."""
    import socket as _socket
    from multiprocessing.connection import Connection
    logs = []
    srv = FakeServer([yoloserve.Model("det", FakeEngine(0), 4)], target_ms=5.0, log=logs.append)
    try:
        a, b = _socket.socketpair()
        mine, theirs = Connection(a.detach()), Connection(b.detach())
        srv.serve_frontend(mine)
        theirs.send_bytes(b"\x01\x02")                     # not a request header
        assert theirs.poll(5.0)
        with pytest.raises(EOFError):
            theirs.recv_bytes()
        assert any("front-end connection closed" in l for l in logs)
        a2, b2 = _socket.socketpair()
        mine2, theirs2 = Connection(a2.detach()), Connection(b2.detach())
        srv.serve_frontend(mine2)
        img = np.full((12, 16, 3), (7, 8, 9), np.uint8)
        theirs2.send_bytes(yoloserve._REQ.pack(5, yoloserve.KIND_BGR, 0, 0, 12, 16))
        theirs2.send_bytes(img.tobytes())
        assert theirs2.poll(10.0)
        msg = theirs2.recv_bytes()
        rid, code, obb, _, n, nresp = yoloserve._RSP.unpack_from(msg)
        assert (rid, code, obb, n) == (5, yoloserve.CODE_OK, 0, 2)
        rows = np.frombuffer(msg, np.float32, n * 6, yoloserve._RSP.size).reshape(n, 6)
        assert rows[0].tolist() == [7, 8, 9, 10, 0.5, 8]
        theirs2.close()
    finally:
        srv.stop()


class _TicketEngine(FakeEngine):
    """A fake engine whose batch JPEG decode fails as a whole."""

    def decode_tickets(self, tickets, first_slot=0):
        raise RuntimeError("yolo_decode_tickets failed")


def test_ticket_decode_failure_fails_only_its_requests():
    """A batch decode of engine-decoded JPEG streams that fails (e.g. a batch too large to
    stage) answers those requests with a decode error; the server keeps running and serves
    the next request."""
    eng = _TicketEngine(0)
    m = yoloserve.Model("det", eng, 4)
    srv = FakeServer([m], target_ms=5.0, log=lambda *a: None)
    try:
        reqs = [yoloserve._Request() for _ in range(3)]
        for r in reqs:
            r.ticket = object()
        srv._decode_tickets(m, reqs)
        assert all(r.error == "image decode failed" and r.ticket is None for r in reqs)
        assert not srv._stop
        r = srv.submit(_png((5, 6, 7)))
        assert r.done.wait(10.0) and r.error is None
        assert r.message().boxes[0].x1 == 5
    finally:
        srv.stop()
