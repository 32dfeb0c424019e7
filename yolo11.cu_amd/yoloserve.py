"""Detection server: the gRPC service `yolo.Yolo/Detect` over the engine's C ABI.

    python yolo11.cu_amd/yoloserve.py --dir models/yolo11n[:maxB] [--dir ...] \
        [--addr 0.0.0.0:50051] [--max-batch 16] [--target-ms 50] [--frontends N]
    python yolo11.cu_amd/yoloserve.py bench --addr 127.0.0.1:50051 --image a.jpg [--model name]

Behaviour of the reference server (server/serve.cpp), on this image's stack (Python gRPC over
the same C ABI; gRPC C++ and protoc are not available here):

* one engine handle per model dir; requests route by `DetectRequest.model` (the dir basename;
  empty = the first dir; anything else is INVALID_ARGUMENT "unknown model: ...")
  (server/serve.cpp:308-317, 361-381);
* deadline-aware dynamic batching per model: a queue fires when it is full or when its oldest
  request would miss `--target-ms` if the batcher waited for a full batch, given that model's
  calibrated `yolo_exec_ms(maxB)`, a decode-time EMA and a 1 ms margin; batches never mix
  models (server/serve.cpp:163-191);
* decoding overlaps the GPU (server/serve.cpp:71-131,264-302), here from the moment a request
  arrives: a JPEG the engine decodes (baseline / extended Huffman, 8-bit, grayscale or YCbCr)
  is handed to the library at once (`yolo_jpeg_submit`: entropy decoding on its decoder
  threads), and the worker runs the GPU half for the whole batch (`yolo_decode_tickets`: copies,
  IDCT and colour on the engine's decode stream, beside the previous batch's network), as the
  reference does with nvJPEG; any other image is decoded by PIL on a decode pool thread
  straight into pinned memory, in PIL's own R, G, B, X layout (the reference uses stb).  The
  worker then reads the previous batch's results (every slot in one call), letterboxes the
  batch in one launch and starts it.  An undecodable image is answered at once and never takes
  a batch slot;
* responses carry the task's fields -- boxes, rotated boxes, top-5 classes, or boxes plus
  RLE masks at proto resolution with the letterbox geometry -- and queue_ms, infer_ms and
  the batch size (server/serve.cpp:193-256); an undecodable image is INVALID_ARGUMENT
  "image decode failed".  Detection lists are encoded with numpy outside the worker.  The
  slack formula's decode term is an EMA of the worker's per-batch staging time.

The gRPC layer is grpc.aio, in this process or, with `--frontends N`, in N front-end
processes sharing the port (SO_REUSEPORT) that pass images and results to this one over
socket pairs.  All engine calls happen on the one worker thread (the engine handle is not
thread-safe).
"""
from __future__ import annotations

import argparse
import asyncio
import collections
import ctypes
import io
import itertools
import json
import os
import queue
import socket
import struct
import subprocess
import sys
import threading
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

import yoloproto as pb

TASK_NAMES = {0: "detect", 1: "obb", 2: "classify", 3: "segment"}
PIXEL_RGBX = 1           # yolo_stage_frames layout R, G, B, X (YOLO_PIXEL_RGBX)
MAX_MSG = 64 << 20       # request size limit (server/serve.cpp:395)
SAFETY_MS = 1.0


# ------------------------------------------------------------------ pure helpers

def rle_encode(mask: np.ndarray) -> np.ndarray:
    """Alternating 0/1 run lengths of a binary mask, row-major, starting with a 0-run (a
    mask whose first pixel is set starts with a run of length 0) -- server/serve.cpp:193-203."""
    flat = np.asarray(mask).ravel() != 0
    if flat.size == 0:
        return np.zeros(1, np.uint32)
    cuts = np.flatnonzero(flat[1:] != flat[:-1]) + 1
    runs = np.diff(np.concatenate(([0], cuts, [flat.size])))
    if flat[0]:
        runs = np.concatenate(([0], runs))
    return runs.astype(np.uint32)


def rle_decode(runs, n: int) -> np.ndarray:
    """Inverse of rle_encode for a mask of n pixels (u8 0/1)."""
    runs = np.asarray(runs, np.int64)
    vals = np.arange(runs.size) % 2
    out = np.repeat(vals, runs).astype(np.uint8)
    if out.size != n:
        raise ValueError(f"runs cover {out.size} pixels, expected {n}")
    return out


def decode_image(data: bytes) -> np.ndarray | None:
    """HxWx3 BGR u8 (the engine's input layout) from encoded image bytes, None if undecodable.
    PIL packs the decoded RGB image as BGR in one pass (its raw "BGR" mode)."""
    try:
        from PIL import Image
        with Image.open(io.BytesIO(data)) as im:
            if im.mode != "RGB":
                im = im.convert("RGB")
            w, h = im.size
            if h < 1 or w < 1:
                return None
            return np.frombuffer(im.tobytes("raw", "BGR"), np.uint8).reshape(h, w, 3)
    except Exception:
        return None


# The Apache Arrow C data interface (its published, stable C ABI).  PIL (11.2+) exports an
# RGB image's pixel memory through it without copying, as a fixed-size list of four u8 per
# pixel (R, G, B, X): the server copies that straight into pinned memory, GIL released,
# instead of packing BGR under the GIL (PIL's tobytes holds it for ~0.5 ms per 640x640 image,
# which capped the whole server near 1.2k images/s).
class _ArrowSchema(ctypes.Structure):
    pass


_ArrowSchema._fields_ = [("format", ctypes.c_char_p), ("name", ctypes.c_char_p), ("metadata", ctypes.c_char_p),
                         ("flags", ctypes.c_int64), ("n_children", ctypes.c_int64),
                         ("children", ctypes.POINTER(ctypes.POINTER(_ArrowSchema))),
                         ("dictionary", ctypes.c_void_p), ("release", ctypes.c_void_p),
                         ("private_data", ctypes.c_void_p)]


class _ArrowArray(ctypes.Structure):
    pass


_ArrowArray._fields_ = [("length", ctypes.c_int64), ("null_count", ctypes.c_int64), ("offset", ctypes.c_int64),
                        ("n_buffers", ctypes.c_int64), ("n_children", ctypes.c_int64),
                        ("buffers", ctypes.POINTER(ctypes.c_void_p)),
                        ("children", ctypes.POINTER(ctypes.POINTER(_ArrowArray))),
                        ("dictionary", ctypes.c_void_p), ("release", ctypes.c_void_p),
                        ("private_data", ctypes.c_void_p)]

_capsule_ptr = ctypes.pythonapi.PyCapsule_GetPointer
_capsule_ptr.restype = ctypes.c_void_p
_capsule_ptr.argtypes = [ctypes.py_object, ctypes.c_char_p]


def _rgbx_view(im, npix: int):
    """(keepalive, u8 view of npix * 4 bytes) of an RGB PIL image's pixel memory, zero-copy;
    None when PIL does not export it (older PIL, or an image held in several blocks).  The
    view is valid while `keepalive` (the exported capsules, which release the export when
    collected) is referenced."""
    try:
        caps = im.__arrow_c_array__()
    except Exception:
        return None
    sch = _ArrowSchema.from_address(_capsule_ptr(caps[0], b"arrow_schema"))
    arr = _ArrowArray.from_address(_capsule_ptr(caps[1], b"arrow_array"))
    if sch.format != b"+w:4" or sch.n_children != 1 or sch.children[0].contents.format != b"C":
        return None
    if arr.length != npix or arr.null_count != 0 or arr.n_children != 1:
        return None
    ch = arr.children[0].contents
    if ch.n_buffers != 2 or ch.null_count != 0 or not ch.buffers[1] or ch.length < (arr.offset + npix) * 4:
        return None
    ptr = ch.buffers[1] + ch.offset + arr.offset * 4
    return caps, np.ctypeslib.as_array((ctypes.c_uint8 * (npix * 4)).from_address(ptr))


def decode_rgbx_into(data: bytes, pool) -> tuple | None:
    """Decodes encoded image bytes into a buffer taken from `pool` as R, G, B, X u8 HWC;
    (buffer, (h, w)), or None if undecodable (the buffer then goes back)."""
    try:
        from PIL import Image
        with Image.open(io.BytesIO(data)) as im:
            if im.mode != "RGB":
                im = im.convert("RGB")
            w, h = im.size
            if h < 1 or w < 1:
                return None
            im.load()                    # the decode itself runs with the GIL released
            n = h * w * 4
            buf = pool.take(n)
            try:
                view = _rgbx_view(im, h * w)
                if view is not None:
                    np.copyto(buf.array[:n], view[1])
                    del view
                else:
                    np.copyto(buf.array[:n], np.frombuffer(im.tobytes("raw", "RGBX"), np.uint8))
            except BaseException:
                pool.give(buf)
                raise
            return buf, (h, w)
    except Exception:
        return None


# Wire encoding of the repeated Box / RBox messages (proto/yolo.proto:14-33), built with numpy
# instead of one protobuf object per detection: each entry is the field-1 (boxes) or field-6
# (rboxes) tag, the submessage length, every float field as tag + 4 little-endian bytes and
# the class as tag + varint.  Fields at their default value are written out too, which proto3
# parsers accept.  Appending these bytes to a serialized DetectResponse adds the entries.
def _entries_wire(outer_tag: int, floats: np.ndarray, cls: np.ndarray) -> bytes | None:
    n, nf = floats.shape
    if n == 0:
        return b""
    c = cls.astype(np.int64)
    if c.min() < 0 or c.max() >= 1 << 14:
        return None                       # 1- and 2-byte varints only
    two = c >= 128
    width = 2 + 5 * nf + 3
    rows = np.zeros((n, width), np.uint8)
    rows[:, 0] = outer_tag
    rows[:, 1] = np.where(two, 5 * nf + 3, 5 * nf + 2)
    f = np.ascontiguousarray(floats, dtype="<f4").view(np.uint8).reshape(n, nf, 4)
    for q in range(nf):
        rows[:, 2 + 5 * q] = ((q + 1) << 3) | 5            # fixed32
        rows[:, 3 + 5 * q:7 + 5 * q] = f[:, q]
    rows[:, 2 + 5 * nf] = (nf + 1) << 3                     # varint
    rows[:, 3 + 5 * nf] = np.where(two, (c & 0x7F) | 0x80, c)
    rows[:, 4 + 5 * nf] = c >> 7
    keep = np.ones((n, width), bool)
    keep[~two, width - 1] = False
    return rows[keep].tobytes()


def boxes_wire(dets: np.ndarray) -> bytes | None:
    """`DetectResponse.boxes` entries for rows (x1, y1, x2, y2, score, cls); None if a class
    id needs more than two varint bytes (the caller then uses protobuf)."""
    return _entries_wire(0x0A, dets[:, :5], dets[:, 5])


def rboxes_wire(rb: np.ndarray) -> bytes | None:
    """`DetectResponse.rboxes` entries for rows (cx, cy, w, h, angle, score, cls)."""
    return _entries_wire(0x32, rb[:, :6], rb[:, 6])


def pick_queue(queues, now: float, target_ms: float, decode_ms: float, safety_ms: float = SAFETY_MS):
    """The batcher's choice (server/serve.cpp:163-191).  `queues` holds one
    (length, oldest arrival [s], max batch, exec_ms at max batch) per model.  A queue is ready
    when full or when its slack -- target minus the oldest request's age, the full-batch
    execution time, the decode estimate and the margin -- is used up.  Returns (index, fire,
    slack_ms): the most urgent ready queue (fire=True), else the queue with the least slack
    (fire=False, wait at most that long), else (-1, False, inf) when every queue is empty."""
    pick, fire, min_slack = -1, False, float("inf")
    for i, (n, t0, maxb, ex) in enumerate(queues):
        if n == 0:
            continue
        slack = target_ms - (now - t0) * 1e3 - max(ex, 0.0) - decode_ms - safety_ms
        ready = n >= maxb or slack <= 0
        if (ready and not fire) or (ready == fire and slack < min_slack):
            pick, min_slack, fire = i, slack, fire or ready
    return pick, fire, min_slack


def parse_dir_spec(spec: str, max_batch: int) -> tuple[str, str, int]:
    """'path/name[:B]' -> (path, name, B); the suffix only counts after the last '/'
    (server/serve.cpp:365-372)."""
    b = max_batch
    colon = spec.rfind(":")
    if colon != -1 and colon > spec.rfind("/"):
        b = int(spec[colon + 1:])
        spec = spec[:colon]
    path = spec.rstrip("/")
    return spec, os.path.basename(path), b


# ------------------------------------------------------------------ server

def response_bytes(resp: bytes, rows, obb: bool) -> bytes:
    """A serialized DetectResponse: `resp` (its other fields, serialized) plus the detection
    rows (boxes, or rotated boxes if `obb`) appended as repeated-field entries."""
    if rows is None or len(rows) == 0:
        return resp
    wire = (rboxes_wire if obb else boxes_wire)(rows)
    if wire is not None:
        return resp + wire
    m = pb.DetectResponse.FromString(resp)      # class ids beyond two varint bytes
    if obb:
        for cx, cy, w, h, a, sc, c in np.asarray(rows, np.float64).tolist():
            m.rboxes.add(cx=cx, cy=cy, w=w, h=h, angle=a, score=sc, cls=int(c))
    else:
        for x1, y1, x2, y2, sc, c in np.asarray(rows, np.float64).tolist():
            m.boxes.add(x1=x1, y1=y1, x2=x2, y2=y2, score=sc, cls=int(c))
    return m.SerializeToString()


class _PinnedPool:
    """Pinned host buffers for decoded frames: a request's pixels go straight from the
    decoder into one (on its handler thread), the worker stages a whole batch from them
    with one asynchronous copy per frame, and they return here once the batch is done."""

    def __init__(self):
        self.free: list = []
        self.lock = threading.Lock()

    def take(self, nbytes: int):
        with self.lock:
            for i, b in enumerate(self.free):
                if b.array.nbytes >= nbytes:
                    return self.free.pop(i)
        import yolort
        return yolort.PinnedBuffer((max(nbytes, 1 << 20),))

    def give(self, b):
        with self.lock:
            self.free.append(b)

    def close(self):
        with self.lock:
            for b in self.free:
                b.free()
            self.free.clear()


class _Request:
    """`resp` holds the response's small fields; `rows` the detections (boxes, or rotated
    boxes if `obb`) that `payload()` encodes on the caller's thread, so the engine worker
    never does it.  `payload()` is the serialized response, `message()` the parsed one.
    The image is `ticket` (a JPEG stream whose entropy decoding the engine library started
    at arrival), or decoded pixels:
    `img` (numpy) or, with a pinned pool, `host` + `hw`."""
    __slots__ = ("img", "host", "ticket", "hw", "arrival", "resp", "rows", "obb", "error", "done", "on_done")

    def __init__(self, on_done=None):
        self.on_done = on_done
        self.img = None
        self.ticket = None
        self.host = None
        self.hw = (0, 0)
        self.arrival = time.monotonic()
        self.resp = pb.DetectResponse()
        self.rows = None
        self.obb = False
        self.error = None
        self.done = threading.Event()

    def finish(self):
        """Marks the response (or error) ready: sets `done`, then calls `on_done` (the event
        loop's wake-up for an asynchronous handler) if one was given."""
        self.done.set()
        if self.on_done is not None:
            self.on_done()

    def payload(self) -> bytes:
        return response_bytes(self.resp.SerializeToString(), self.rows, self.obb)

    def message(self):
        return pb.DetectResponse.FromString(self.payload())


class Model:
    """One served model: its engine handle (the yolort.Engine API), batch limit and queue."""

    def __init__(self, name: str, engine, max_batch: int):
        self.name = name
        self.eng = engine
        self.max_batch = max_batch
        self.task = engine.task()
        self.task_name = TASK_NAMES.get(self.task, "detect")
        self.mask_hw = engine.mask_dim() if self.task == 3 else (0, 0)
        self.exec_ms = float(engine.exec_ms(max_batch))
        self.queue: collections.deque[_Request] = collections.deque()


class Server:
    """Batcher + engine worker.  `submit` (decode + enqueue) is called from any thread.

    With real engines the batcher and the per-batch loop are the library's native batch
    worker (yolo_batcher_*: collect, decode, fetch the previous batch, stage, launch on a
    library thread); this object only queues requests into it and turns its finished
    records into responses on a completion thread.  Engines without the C ABI (test fakes)
    run the same loop in Python (`_work`)."""

    def __init__(self, models: list[Model], target_ms: float = 50.0, log=print, native: bool = True):
        if not models:
            raise ValueError("no models")
        self.models = models
        self.by_name = {m.name: i for i, m in enumerate(models)}
        self.target_ms = float(target_ms)
        self.stage_ema = 1.0
        self.log = log
        self.cv = threading.Condition()
        self.buffers: dict[int, object] = {}
        self.served = 0
        # batch staging from pinned memory when every engine offers it (test fakes do not),
        # and JPEG streams decoded by the engines themselves when they all can
        self.pool = _PinnedPool() if all(hasattr(m.eng, "stage_frames") for m in models) else None
        self.engine_jpeg = self.pool is not None and all(hasattr(m.eng, "decode_tickets") for m in models)
        self._stop = False
        self.batcher = None
        if native and self.engine_jpeg:
            import yolort
            self.batcher = yolort.Batcher([m.eng for m in models], [m.max_batch for m in models], self.target_ms)
            self._tags = itertools.count(1)
            self._pending: dict[int, tuple] = {}
            self._plock = threading.Lock()
            self._worker = threading.Thread(target=self._drain, name="yoloserve-completion", daemon=True)
        else:
            self._worker = threading.Thread(target=self._work, name="yoloserve-worker", daemon=True)
        self._worker.start()

    # -- the native batch worker
    def _native_submit(self, r: _Request, mi: int, jpeg: bytes | None = None) -> bool:
        """Queues r on the native batcher: a JPEG stream the engine decodes (`jpeg`), or the
        pixels in r.host.  False if the engine does not decode the stream (nothing queued)."""
        tag = next(self._tags)
        with self._plock:
            self._pending[tag] = (r, mi)
        if jpeg is not None:
            rc = self.batcher.submit_jpeg(mi, jpeg, tag)
        else:
            rc = self.batcher.submit_frame(mi, r.host.ptr, r.hw[0], r.hw[1], tag)
        if rc == 0:
            return True
        with self._plock:
            self._pending.pop(tag, None)
        if rc == 1:
            return False
        r.error = "server shutting down"
        r.resp.task = self.models[mi].task_name
        self._release([r])
        r.finish()
        return True

    def _drain(self):
        """Completion thread: finished records of the native batcher -> responses."""
        while True:
            recs = self.batcher.wait(200)
            if recs is None:
                break
            for rec in recs:
                with self._plock:
                    r, mi = self._pending.pop(rec["tag"])
                self._complete(r, self.models[mi], rec)
            if recs:
                before = self.served
                self.served += len(recs)
                if self.served // 5000 != before // 5000:
                    self.log(f"[serve] {self.served} imgs, B={recs[-1]['batch']} gpu {recs[-1]['infer_ms']:.2f} ms")

    def _complete(self, r: _Request, m: Model, rec: dict):
        resp = r.resp
        resp.task = m.task_name
        self._release([r])                # the batch has run: its frame buffer is free
        if rec["status"] != 0:
            import yolort                 # loaded already: this path runs with a native batcher
            r.error = {yolort.BATCH_DECODE_FAILED: "image decode failed",
                       yolort.BATCH_STOPPED: "server shutting down"}.get(rec["status"], "batch failed")
            r.finish()
            return
        resp.queue_ms = rec["queue_ms"]
        resp.infer_ms = rec["infer_ms"]
        resp.batch = rec["batch"]
        rows = rec["rows"]
        if m.task == 2:
            for c, p in rows.tolist():
                resp.classes.add(id=int(c), prob=float(p))
        else:
            r.rows = rows
            r.obb = m.task == 1
            if m.task == 3:
                resp.mask_h, resp.mask_w = rec["mask_hw"]
                resp.lb_scale, resp.lb_top, resp.lb_left = rec["geom"]
                runs, at = rec["rle"], 0
                for n in rec["rle_len"].tolist():
                    resp.masks.add(rle=runs[at:at + n].tolist())
                    at += n
        r.finish()

    # -- engine-side steps (device staging is separate so tests can drive a fake engine)
    def _device_buffer(self, slot: int, nbytes: int):
        import yolort
        b = self.buffers.get(slot)
        if b is None or b.nbytes < nbytes:
            if b is not None:
                b.free()
            b = self.buffers[slot] = yolort.DeviceBuffer(nbytes)
        return b

    def _stage(self, m: Model, slot: int, img: np.ndarray):
        buf = self._device_buffer(slot, img.nbytes)
        m.eng.upload(buf, img)
        h, w = img.shape[:2]
        if m.task == 2:
            m.eng.preprocess_cls(buf.ptr, h, w, slot)
        else:
            m.eng.preprocess(buf.ptr, h, w, slot)

    # -- request side
    def model_index(self, name: str) -> int:
        if not name:
            return 0
        if name not in self.by_name:
            raise KeyError(name)
        return self.by_name[name]

    def submit_jpeg(self, image: bytes, model: str = "", on_done=None):
        """Queues a JPEG stream the engines decode themselves, its entropy decoding started on
        the library's decoder threads now (a few µs here); None if the engines do not decode
        this stream (submit it instead: PIL decodes it)."""
        if not self.engine_jpeg or image[:2] != b"\xff\xd8":
            return None
        mi = self.model_index(model)
        if self.batcher is not None:
            r = _Request(on_done)
            return r if self._native_submit(r, mi, image) else None
        import yolort
        ticket = yolort.jpeg_submit(image)
        if ticket is None:
            return None
        r = _Request(on_done)
        r.ticket = ticket
        return self._queue(r, mi)

    def submit(self, image: bytes, model: str = "", on_done=None) -> _Request:
        """Decodes on the calling thread, then queues; the returned request's `done` is set,
        and `on_done()` called from the thread that completes it, when its response (or
        error) is ready."""
        mi = self.model_index(model)
        r = _Request(on_done)
        if self.pool is not None:
            got = decode_rgbx_into(image, self.pool)
            if got is not None:
                r.host, r.hw = got
        else:
            r.img = decode_image(image)
        if r.ticket is None and r.host is None and r.img is None:
            r.error = "image decode failed"
            r.resp.task = self.models[mi].task_name
            r.finish()
            return r
        return self._queue(r, mi)

    def _queue(self, r: _Request, mi: int) -> _Request:
        if self.batcher is not None:      # decoded pixels (r.host) into the native batcher
            self._native_submit(r, mi)
            return r
        with self.cv:
            if self._stop:
                r.error = "server shutting down"
                self._release([r])
                r.finish()
                return r
            q = self.models[mi].queue
            q.append(r)
            # only a queue that starts (its slack now counts) or fills can change the
            # batcher's decision; it sleeps until the least slack runs out otherwise
            if len(q) == 1 or len(q) >= self.models[mi].max_batch:
                self.cv.notify_all()
        return r

    # -- requests from front-end processes
    def serve_frontend(self, conn):
        """Serves one front-end process's connection (see `grpc_server(frontends=...)`): a
        reader thread queues its requests, a sender thread encodes and returns the results.
        Returns the two threads; both end when the connection closes."""
        sendq = queue.SimpleQueue()

        def reader():
            try:
                while True:
                    hdr = conn.recv_bytes()
                    rid, kind, mi, _, h, w = _REQ.unpack(hdr)
                    data = conn.recv_bytes()
                    r = _Request()
                    r.on_done = lambda rid=rid, r=r: sendq.put((rid, r))
                    if not 0 <= mi < len(self.models):
                        r.error = "unknown model"
                        r.finish()
                        continue
                    if kind == KIND_JPEG and self.batcher is not None:
                        if self._native_submit(r, mi, data):
                            continue
                        got = decode_rgbx_into(data, self.pool)    # the header check said yes
                        if got is None:
                            r.error = "image decode failed"
                            r.finish()
                            continue
                        r.host, r.hw = got
                    elif kind == KIND_JPEG and self.engine_jpeg:
                        import yolort
                        r.ticket = yolort.jpeg_submit(data)
                        if r.ticket is None:      # the front-end's header check said yes
                            got = decode_rgbx_into(data, self.pool)
                            if got is None:
                                r.error = "image decode failed"
                                r.finish()
                                continue
                            r.host, r.hw = got
                    elif kind == KIND_RGBX and self.pool is not None:
                        r.host, r.hw = self.pool.take(h * w * 4), (h, w)
                        np.copyto(r.host.array[:h * w * 4], np.frombuffer(data, np.uint8))
                    elif kind == KIND_BGR and self.pool is None:
                        r.img = np.frombuffer(data, np.uint8).reshape(h, w, 3)
                    else:
                        r.error = "image decode failed"
                        r.finish()
                        continue
                    self._queue(r, mi)
            except (EOFError, OSError):
                pass
            except Exception as ex:       # a malformed message: drop the connection
                self.log(f"[serve] front-end connection closed: {ex!r}")
                try:
                    conn.close()
                except OSError:
                    pass
            finally:
                sendq.put(None)

        def sender():
            while True:
                item = sendq.get()
                if item is None:
                    return
                rid, r = item
                try:
                    conn.send_bytes(_encode_result(rid, r))
                except (EOFError, OSError, BrokenPipeError):
                    return

        ts = [threading.Thread(target=reader, name="yoloserve-fe-reader", daemon=True),
              threading.Thread(target=sender, name="yoloserve-fe-sender", daemon=True)]
        for t in ts:
            t.start()
        return ts

    # -- worker side
    def _collect(self):
        with self.cv:
            while True:
                if self._stop:
                    return None
                qs = [(len(m.queue), m.queue[0].arrival if m.queue else 0.0, m.max_batch, m.exec_ms)
                      for m in self.models]
                pick, fire, slack = pick_queue(qs, time.monotonic(), self.target_ms, self.stage_ema)
                if pick >= 0 and fire:
                    break
                self.cv.wait(None if pick < 0 else max(slack, 0.0) * 1e-3)
            m = self.models[pick]
            batch = [m.queue.popleft() for _ in range(min(len(m.queue), m.max_batch))]
        return pick, batch

    def _work(self):
        prev = None
        batch = None          # collected and not yet launched
        try:
            while True:
                got = self._collect()
                if got is None:
                    break
                mi, batch = got
                m = self.models[mi]
                t0 = time.monotonic()
                jp = []
                if self.pool is not None:
                    # engine-decoded JPEG streams take the first slots, decoded pixels the
                    # rest.  Their entropy decoding started at arrival; the coefficient
                    # copies and the GPU half queue now, behind the previous batch; the
                    # letterbox (which sets the slots' geometry, still the previous batch's
                    # until its results are read) waits for _finish.
                    jp = [r for r in batch if r.ticket is not None]
                    px = [r for r in batch if r.ticket is None]
                    batch = jp + px
                    if jp:
                        self._decode_tickets(m, jp)
                stage_ms = (time.monotonic() - t0) * 1e3
                if prev is not None:
                    self._finish(*prev)
                    prev = None
                t1 = time.monotonic()
                if self.pool is not None:
                    if jp:
                        m.eng.letterbox_decoded(len(jp), 0)
                    if px:                # one call: async copies + one letterbox launch
                        m.eng.stage_frames([r.host.ptr for r in px], [r.hw[0] for r in px],
                                           [r.hw[1] for r in px], PIXEL_RGBX, len(jp))
                else:
                    for i, r in enumerate(batch):
                        self._stage(m, i, r.img)
                        r.img = None
                launch = time.monotonic()
                stage_ms += (launch - t1) * 1e3
                self.stage_ema = 0.9 * self.stage_ema + 0.1 * stage_ms
                m.eng.run_async(len(batch))
                prev = (mi, batch, launch)
                batch = None
                with self.cv:
                    idle = all(not q.queue for q in self.models)
                if idle:                  # no traffic behind it: answer now
                    self._finish(*prev)
                    prev = None
        except Exception as ex:        # an engine failure fails everything in flight
            self.log(f"[serve] worker stopped: {ex!r}")
            failed = (prev[1] if prev is not None else []) + (batch or [])
            for r in failed:
                r.error = f"engine failure: {ex}"
                r.finish()
            self._release(failed)
            batch = None
            with self.cv:
                self._stop = True
            prev = None
        if prev is not None:
            self._finish(*prev)
        with self.cv:
            for m in self.models:
                while m.queue:
                    r = m.queue.popleft()
                    r.error = "server shutting down"
                    self._release([r])
                    r.finish()

    def _decode_tickets(self, m: Model, jp: list):
        """Queues the GPU half of the batch's engine-decoded JPEG streams (slots 0..len-1).
        A stream the engine does not stage (corrupt, or past what one batch decode holds)
        fails its own request; a call that fails as a whole fails these requests only, and
        the rest of the batch goes on (their slots run on whatever they held, and their
        results are not read).  The worker stops only for failures of the batch itself."""
        tickets = [r.ticket for r in jp]
        for r in jp:
            r.ticket = None               # consumed by the call, whatever happens
        try:
            res = m.eng.decode_tickets(tickets, 0)
        except Exception as ex:
            self.log(f"[serve] JPEG batch decode failed: {ex!r}")
            for r in jp:
                r.error = "image decode failed"
            return
        for r, (st, _, _) in zip(jp, res):
            if st != 0:
                r.error = "image decode failed"

    def _release(self, batch: list):
        for r in batch:
            if r.host is not None and self.pool is not None:
                self.pool.give(r.host)
                r.host = None
            if r.ticket is not None:
                import yolort
                yolort.jpeg_release(r.ticket)
                r.ticket = None

    def _finish(self, mi: int, batch: list, launch: float):
        m = self.models[mi]
        m.eng.sync()
        infer_ms = (time.monotonic() - launch) * 1e3
        self._release(batch)              # the stream has passed the staged frames
        rows = None                       # every slot's records in one call
        if self.pool is not None and m.task in (0, 3):
            rows = m.eng.get_batch(len(batch))
        elif self.pool is not None and m.task == 1:
            rows = m.eng.get_obb_batch(len(batch))
        for i, r in enumerate(batch):
            resp = r.resp
            resp.task = m.task_name
            if r.error:                   # its slot ran on whatever it held
                r.finish()
                continue
            r.rows = self._fill(m, i, resp, None if rows is None else rows[i])
            r.obb = m.task == 1
            resp.queue_ms = (launch - r.arrival) * 1e3
            resp.infer_ms = infer_ms
            resp.batch = len(batch)
            r.finish()
        before = self.served
        self.served += len(batch)
        if self.served // 5000 != before // 5000:
            self.log(f"[serve] {self.served} imgs, B={len(batch)} gpu {infer_ms:.2f} ms "
                     f"({len(batch) * 1e3 / max(infer_ms, 1e-6):.0f} img/s in-batch)")

    @staticmethod
    def _fill(m: Model, slot: int, resp, rows=None):
        """Reads what the response needs from the engine (worker thread): sets the classes,
        masks and letterbox geometry on `resp` and returns the detection rows (None for
        classify).  `rows`: the slot's records when already fetched for the whole batch."""
        eng = m.eng
        if m.task == 2:
            ids, probs = eng.get_cls(slot, 5)
            for c, p in zip(ids.tolist(), probs.tolist()):
                resp.classes.add(id=int(c), prob=float(p))
            return None
        if m.task == 1:
            return np.asarray(eng.get_obb(slot) if rows is None else rows)
        dets = np.asarray(eng.get(slot) if rows is None else rows)
        if m.task == 3:
            resp.mask_h, resp.mask_w = m.mask_hw
            resp.lb_scale, resp.lb_top, resp.lb_left = eng.slot_geom(slot)
            for j in range(len(dets)):
                mk = eng.get_mask(slot, j)
                if mk is None:
                    resp.masks.add()
                else:
                    resp.masks.add(rle=rle_encode(mk).tolist())
        return dets

    def stop(self):
        with self.cv:
            self._stop = True
            self.cv.notify_all()
        if self.batcher is not None:
            self.batcher.stop()           # queued requests are answered; the drain thread ends
        self._worker.join()
        if self.batcher is not None:
            self.batcher.destroy()
        for b in self.buffers.values():
            b.free()
        self.buffers.clear()
        if self.pool is not None:
            self.pool.close()


# ------------------------------------------------------------------ gRPC glue

# ------------------------------------------------------------------ front-end processes
# A front-end is a process of its own (its own GIL and event loop) running the gRPC service on
# the server's port with SO_REUSEPORT, so the kernel spreads client connections over the
# front-ends.  It answers routing and decode errors itself, hands each image to the engine
# process over a pipe (JPEG streams the engines decode, as they are; other formats decoded
# here by PIL into R,G,B,X pixels), and encodes the response from the result the engine
# process returns.  Engine calls, batching and the GPU stay in the engine process.  A
# front-end never loads the HIP runtime: it reads JPEG headers with libyolo11_jpeg.so.
_REQ = struct.Struct("<QBBHII")      # request id, kind, model index, 0, height, width
_RSP = struct.Struct("<QBBHII")      # request id, code, obb, 0, rows, response-field bytes
KIND_JPEG, KIND_RGBX, KIND_BGR = 0, 1, 2
CODE_OK, CODE_INVALID, CODE_UNAVAILABLE = 0, 1, 2


def _encode_result(rid: int, r: _Request) -> bytes:
    """A finished request as the engine process returns it to a front-end: the header, the
    detection rows (float32), then the serialized response fields (or the error text)."""
    if r.error:
        code = CODE_INVALID if r.error == "image decode failed" else CODE_UNAVAILABLE
        msg = r.error.encode()
        return _RSP.pack(rid, code, 0, 0, 0, len(msg)) + msg
    rows, n = b"", 0
    if r.rows is not None and len(r.rows):
        a = np.ascontiguousarray(r.rows, np.float32)
        rows, n = a.tobytes(), a.shape[0]
    resp = r.resp.SerializeToString()
    return _RSP.pack(rid, CODE_OK, 1 if r.obb else 0, 0, n, len(resp)) + rows + resp


_JPEG_LIB = None


def jpeg_dims(data: bytes):
    """(height, width) if the engine decodes this JPEG stream itself, else None -- from the
    headers, with the host-only libyolo11_jpeg.so (no HIP runtime in the calling process)."""
    global _JPEG_LIB
    if _JPEG_LIB is None:
        lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "libyolo11_jpeg.so"))
        lib.yolo_jpeg_probe.restype = ctypes.c_int
        lib.yolo_jpeg_probe.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int),
                                        ctypes.POINTER(ctypes.c_int)]
        _JPEG_LIB = lib
    h, w = ctypes.c_int(0), ctypes.c_int(0)
    ok = _JPEG_LIB.yolo_jpeg_probe(data, len(data), ctypes.byref(h), ctypes.byref(w))
    return (h.value, w.value) if ok == 1 else None


def _frontend_decode(image: bytes, rgbx: bool):
    """(kind, height, width, pixel bytes) decoded by PIL, or None if undecodable."""
    if not rgbx:
        img = decode_image(image)
        return None if img is None else (KIND_BGR, img.shape[0], img.shape[1], img.tobytes())
    try:
        from PIL import Image
        with Image.open(io.BytesIO(image)) as im:
            if im.mode != "RGB":
                im = im.convert("RGB")
            w, h = im.size
            if h < 1 or w < 1:
                return None
            im.load()
            view = _rgbx_view(im, h * w)
            data = view[1].tobytes() if view is not None else im.tobytes("raw", "RGBX")
            return KIND_RGBX, h, w, data
    except Exception:
        return None


def _frontend_main(addr: str, conn, names: list, engine_jpeg: bool, rgbx: bool, decoders: int):
    asyncio.run(_frontend(addr, conn, names, engine_jpeg, rgbx, decoders))


async def _frontend(addr: str, conn, names: list, engine_jpeg: bool, rgbx: bool, decoders: int):
    """engine_jpeg: JPEG streams inside the engines' decoder go to the engine process as they
    are; rgbx: other images are sent as R,G,B,X pixels (the engine process stages them from
    pinned memory) instead of BGR."""
    import grpc
    loop = asyncio.get_running_loop()
    pending: dict[int, asyncio.Future] = {}
    ids = itertools.count()
    outq: queue.SimpleQueue = queue.SimpleQueue()
    pool = ThreadPoolExecutor(max_workers=decoders, thread_name_prefix="yoloserve-fe-decode")
    stopping = asyncio.Event()

    def deliver(rid, msg):
        fut = pending.pop(rid, None)
        if fut is not None and not fut.done():
            fut.set_result(msg)

    def engine_gone():
        for fut in pending.values():
            if not fut.done():
                fut.set_result(None)
        pending.clear()
        stopping.set()

    def reader():                         # results from the engine process
        try:
            while True:
                msg = conn.recv_bytes()
                loop.call_soon_threadsafe(deliver, _RSP.unpack_from(msg)[0], msg)
        except Exception:                 # closed, or a malformed message: stop serving
            pass
        try:
            loop.call_soon_threadsafe(engine_gone)
        except RuntimeError:
            pass

    def writer():                         # requests to the engine process
        while True:
            item = outq.get()
            if item is None:
                return
            try:
                conn.send_bytes(item[0])
                conn.send_bytes(item[1])
            except (EOFError, OSError):
                return

    async def detect(request, context):
        model = request.model
        if model and model not in names:
            await context.abort(grpc.StatusCode.INVALID_ARGUMENT, f"unknown model: {model}")
        mi = names.index(model) if model else 0
        image = request.image
        hw = jpeg_dims(image) if engine_jpeg and image[:2] == b"\xff\xd8" else None
        if hw is not None:
            kind, (h, w), data = KIND_JPEG, hw, image
        else:
            got = await loop.run_in_executor(pool, _frontend_decode, image, rgbx)
            if got is None:
                await context.abort(grpc.StatusCode.INVALID_ARGUMENT, "image decode failed")
            kind, h, w, data = got
        if stopping.is_set():
            await context.abort(grpc.StatusCode.UNAVAILABLE, "engine process gone")
        rid = next(ids)
        fut = loop.create_future()
        pending[rid] = fut
        outq.put((_REQ.pack(rid, kind, mi, 0, h, w), data))
        msg = await fut
        if msg is None:
            await context.abort(grpc.StatusCode.UNAVAILABLE, "engine process gone")
        _, code, obb, _, n, nresp = _RSP.unpack_from(msg)
        if code != CODE_OK:
            err = msg[_RSP.size:_RSP.size + nresp].decode()
            await context.abort(grpc.StatusCode.INVALID_ARGUMENT if code == CODE_INVALID
                                else grpc.StatusCode.UNAVAILABLE, err)
        ncol = 7 if obb else 6
        rows = np.frombuffer(msg, np.float32, n * ncol, _RSP.size).reshape(n, ncol) if n else None
        off = _RSP.size + n * ncol * 4
        return response_bytes(msg[off:off + nresp], rows, bool(obb))

    handler = grpc.method_handlers_generic_handler(pb.SERVICE, {
        pb.METHOD: grpc.unary_unary_rpc_method_handler(
            detect, request_deserializer=pb.DetectRequest.FromString, response_serializer=None)})
    srv = grpc.aio.server(options=[("grpc.max_receive_message_length", MAX_MSG),
                                   ("grpc.max_send_message_length", MAX_MSG), ("grpc.so_reuseport", 1)])
    srv.add_generic_rpc_handlers((handler,))
    try:
        port = srv.add_insecure_port(addr)
    except Exception as ex:
        port, err = 0, repr(ex)
    else:
        err = f"cannot bind {addr}"
    if port == 0:
        conn.send_bytes(b"E" + err.encode())
        return
    await srv.start()
    threading.Thread(target=reader, name="yoloserve-fe-results", daemon=True).start()
    threading.Thread(target=writer, name="yoloserve-fe-requests", daemon=True).start()
    conn.send_bytes(b"R%d" % port)
    await stopping.wait()
    await srv.stop(1.0)
    outq.put(None)
    pool.shutdown(wait=False)


def _free_port(host: str) -> int:
    fam = socket.AF_INET6 if ":" in host.strip("[]") else socket.AF_INET
    with socket.socket(fam, socket.SOCK_STREAM) as sk:
        sk.bind((host.strip("[]") if host not in ("", "0.0.0.0") else "", 0))
        return sk.getsockname()[1]


class _Frontends:
    """`n` front-end processes serving `server` on one port: child programs
    (`yoloserve.py frontend ...`) that share nothing with this process but a socket pair each;
    grpc.Server's `stop(grace)` and `wait_for_termination()`."""

    def __init__(self, server: Server, addr: str, n: int, decoders: int):
        from multiprocessing.connection import Connection
        host, port = addr.rsplit(":", 1)
        if int(port) == 0:
            port = str(_free_port(host))
        addr = f"{host}:{port}"
        self.procs, self.conns = [], []
        try:
            for _ in range(n):
                mine, theirs = socket.socketpair()
                cmd = [sys.executable, os.path.abspath(__file__), "frontend", "--fd", str(theirs.fileno()),
                       "--addr", addr, "--decoders", str(decoders), "--engine-jpeg", str(int(server.engine_jpeg)),
                       "--rgbx", str(int(server.pool is not None))]
                for m in server.models:
                    cmd += ["--model", m.name]
                self.procs.append(subprocess.Popen(cmd, pass_fds=(theirs.fileno(),)))
                theirs.close()
                self.conns.append(Connection(mine.detach()))
            for c, p in zip(self.conns, self.procs):
                while not c.poll(0.5):
                    if p.poll() is not None:
                        raise RuntimeError(f"front-end process exited ({p.returncode}) before serving")
                msg = c.recv_bytes()
                if msg[:1] != b"R":
                    raise RuntimeError(f"front-end failed: {msg[1:].decode()}")
        except BaseException:
            self.stop()
            raise
        self.port = int(port)
        self.threads = [t for c in self.conns for t in server.serve_frontend(c)]

    def stop(self, grace: float | None = None):
        for c in self.conns:              # wakes both ends' readers: the front-ends shut down
            try:
                socket.socket(fileno=os.dup(c.fileno())).shutdown(socket.SHUT_RDWR)
            except OSError:
                pass
        for p in self.procs:
            try:
                p.wait(timeout=(grace or 0) + 15)
            except subprocess.TimeoutExpired:
                p.kill()
                p.wait(5)
        for c in self.conns:
            c.close()
        self.conns, self.procs = [], []

    def wait_for_termination(self, timeout: float | None = None) -> bool:
        try:
            for p in self.procs:
                p.wait(timeout)
        except subprocess.TimeoutExpired:
            return False
        return True


def _default_decoders() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 4
    return max(4, min(n, 32))


class _AioServer:
    """A grpc.aio server on an event-loop thread of its own.  Each RPC decodes on a thread of
    the decode pool (PIL's decode and the pixel copy run with the GIL released), waits for
    its batch on the loop without holding a thread, and returns the response bytes the
    request serialized.  `stop(grace)` and `wait_for_termination()` follow grpc.Server."""

    def __init__(self, server: Server, addr: str, decoders: int):
        self.server = server
        self.decoders = ThreadPoolExecutor(max_workers=decoders, thread_name_prefix="yoloserve-decode")
        self.loop = asyncio.new_event_loop()
        self.port = 0
        self._aio = None
        self._error = None
        started = threading.Event()
        self._thread = threading.Thread(target=self._run, args=(addr, started), name="yoloserve-grpc", daemon=True)
        self._thread.start()
        started.wait()
        if self._error is not None:
            self._thread.join()
            self.decoders.shutdown(wait=False)
            raise self._error

    def _run(self, addr: str, started: threading.Event):
        asyncio.set_event_loop(self.loop)
        try:
            self.loop.run_until_complete(self._start(addr))
        except BaseException as ex:
            self._error = ex if isinstance(ex, Exception) else RuntimeError(repr(ex))
            started.set()
            self.loop.close()
            return
        started.set()
        try:
            self.loop.run_forever()
        finally:
            self.loop.close()

    async def _start(self, addr: str):
        import grpc
        server, decoders = self.server, self.decoders

        async def detect(request, context):
            loop = asyncio.get_running_loop()
            ready = loop.create_future()

            def wake():                   # from the thread that completes the request
                try:
                    loop.call_soon_threadsafe(_resolve, ready)
                except RuntimeError:      # the loop has already closed
                    pass
            try:
                # a JPEG the engine decodes: its decoding starts on the library's threads
                r = server.submit_jpeg(request.image, request.model, wake)
                if r is None:
                    r = await loop.run_in_executor(decoders, server.submit, request.image, request.model, wake)
            except KeyError:
                await context.abort(grpc.StatusCode.INVALID_ARGUMENT, f"unknown model: {request.model}")
            await ready
            if r.error == "image decode failed":
                await context.abort(grpc.StatusCode.INVALID_ARGUMENT, r.error)
            elif r.error:
                await context.abort(grpc.StatusCode.UNAVAILABLE, r.error)
            return r.payload()

        # responses leave the handler already serialized (bytes pass through unchanged)
        handler = grpc.method_handlers_generic_handler(pb.SERVICE, {
            pb.METHOD: grpc.unary_unary_rpc_method_handler(
                detect, request_deserializer=pb.DetectRequest.FromString, response_serializer=None)})
        self._aio = grpc.aio.server(options=[("grpc.max_receive_message_length", MAX_MSG),
                                             ("grpc.max_send_message_length", MAX_MSG)])
        self._aio.add_generic_rpc_handlers((handler,))
        self.port = self._aio.add_insecure_port(addr)
        if self.port == 0:
            raise RuntimeError(f"cannot bind {addr}")
        await self._aio.start()

    def stop(self, grace: float | None = None):
        if self.loop.is_closed():
            return
        try:
            asyncio.run_coroutine_threadsafe(self._aio.stop(grace), self.loop).result(timeout=(grace or 0) + 30)
        finally:
            self.loop.call_soon_threadsafe(self.loop.stop)
            self._thread.join()
            self.decoders.shutdown(wait=True)

    def wait_for_termination(self, timeout: float | None = None) -> bool:
        self._thread.join(timeout)
        return not self._thread.is_alive()


def _resolve(fut):
    if not fut.done():
        fut.set_result(None)


def grpc_server(server: Server, addr: str, decoders: int | None = None, frontends: int = 0):
    """A started gRPC server exposing `server` at `addr`; returns (server handle, bound port).
    frontends = 0: grpc.aio on an event-loop thread of this process, decoding on a pool of
    `decoders` threads.  frontends = n: n front-end processes on the same port (each with
    `decoders` PIL threads, default the CPUs split between them), this process keeping the
    engines.  The handle has grpc.Server's `stop(grace)` and `wait_for_termination()`."""
    if frontends > 0:
        fe = _Frontends(server, addr, frontends, decoders or max(2, _default_decoders() // frontends))
        return fe, fe.port
    gs = _AioServer(server, addr, decoders or _default_decoders())
    return gs, gs.port


def load_models(specs: list[str], max_batch: int, log=print) -> list[Model]:
    import yolort
    models = []
    for spec in specs:
        path, name, b = parse_dir_spec(spec, max_batch)
        m = Model(name, yolort.Engine(path, b), b)
        log(f"model '{name}': task={m.task_name} max-batch={b}")
        models.append(m)
    return models


class Client:
    """Minimal client of the service (any client generated from the same contract works)."""

    def __init__(self, addr: str):
        import grpc
        self.channel = grpc.insecure_channel(addr, options=[("grpc.max_send_message_length", MAX_MSG),
                                                            ("grpc.max_receive_message_length", MAX_MSG)])
        self._call = self.channel.unary_unary(pb.FULL_METHOD, request_serializer=pb.DetectRequest.SerializeToString,
                                              response_deserializer=pb.DetectResponse.FromString)

    def detect(self, image: bytes, model: str = "", timeout: float | None = 60.0):
        return self._call(pb.DetectRequest(image=image, model=model), timeout=timeout)

    def close(self):
        self.channel.close()


def bench(addr: str, images: list[bytes], model: str = "", concurrency: int = 32, seconds: float = 10.0) -> dict:
    """Closed-loop load: `concurrency` callers (coroutines on one grpc.aio channel) each send
    the next image as soon as the last answer arrives; returns throughput and latency
    percentiles."""
    import grpc

    async def run():
        lat, batches = [], []
        async with grpc.aio.insecure_channel(addr, options=[("grpc.max_send_message_length", MAX_MSG),
                                                            ("grpc.max_receive_message_length", MAX_MSG)]) as ch:
            call = ch.unary_unary(pb.FULL_METHOD, request_serializer=pb.DetectRequest.SerializeToString,
                                  response_deserializer=pb.DetectResponse.FromString)
            reqs = [pb.DetectRequest(image=im, model=model) for im in images]
            stop_at = time.monotonic() + seconds

            async def caller(k):
                i = k
                while time.monotonic() < stop_at:
                    t0 = time.monotonic()
                    r = await call(reqs[i % len(reqs)], timeout=60.0)
                    lat.append((time.monotonic() - t0) * 1e3)
                    batches.append(r.batch)
                    i += concurrency

            t0 = time.monotonic()
            await asyncio.gather(*(caller(k) for k in range(concurrency)))
            return lat, batches, time.monotonic() - t0

    lat, batches, wall = asyncio.run(run())
    a = np.array(lat)
    return dict(requests=int(a.size), img_per_s=a.size / wall, p50_ms=float(np.percentile(a, 50)),
                p99_ms=float(np.percentile(a, 99)), mean_batch=float(np.mean(batches)), concurrency=concurrency)


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    if argv and argv[0] == "frontend":    # started by grpc_server(frontends=n)
        from multiprocessing.connection import Connection
        ap = argparse.ArgumentParser(prog="yoloserve frontend")
        ap.add_argument("--fd", type=int, required=True)
        ap.add_argument("--addr", required=True)
        ap.add_argument("--decoders", type=int, default=4)
        ap.add_argument("--engine-jpeg", type=int, default=0)
        ap.add_argument("--rgbx", type=int, default=0)
        ap.add_argument("--model", action="append", default=[])
        a = ap.parse_args(argv[1:])
        _frontend_main(a.addr, Connection(a.fd), a.model, bool(a.engine_jpeg), bool(a.rgbx), a.decoders)
        return 0
    if argv and argv[0] == "bench":
        ap = argparse.ArgumentParser(prog="yoloserve bench")
        ap.add_argument("--addr", default="127.0.0.1:50051")
        ap.add_argument("--image", action="append", required=True)
        ap.add_argument("--model", default="")
        ap.add_argument("--concurrency", type=int, default=32)
        ap.add_argument("--seconds", type=float, default=10.0)
        a = ap.parse_args(argv[1:])
        imgs = [open(p, "rb").read() for p in a.image]
        print(json.dumps(bench(a.addr, imgs, a.model, a.concurrency, a.seconds)), flush=True)
        return 0
    ap = argparse.ArgumentParser(prog="yoloserve", description="gRPC yolo.Yolo/Detect server")
    ap.add_argument("--dir", action="append", default=[], help="model dir[:max batch]; repeatable")
    ap.add_argument("--addr", default="0.0.0.0:50051")
    ap.add_argument("--max-batch", type=int, default=16)
    ap.add_argument("--target-ms", type=float, default=50.0)
    ap.add_argument("--frontends", type=int, default=0,
                    help="gRPC front-end processes sharing the port (0: serve in this process)")
    a = ap.parse_args(argv)
    specs = a.dir or ["build/yolo11n"]
    models = load_models(specs, a.max_batch)
    srv = Server(models, a.target_ms)
    gs, port = grpc_server(srv, a.addr, frontends=a.frontends)
    print(f"yoloserve listening on {a.addr} (port {port}, {len(models)} models, target={a.target_ms:.0f} ms)",
          flush=True)
    try:
        gs.wait_for_termination()
    except KeyboardInterrupt:
        pass
    gs.stop(1.0)
    srv.stop()
    for m in models:
        m.eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
