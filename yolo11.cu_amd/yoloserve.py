"""Detection server: the gRPC service `yolo.Yolo/Detect` over the engine's C ABI.

    python yolo11.cu_amd/yoloserve.py --dir models/yolo11n[:maxB] [--dir ...] \
        [--addr 0.0.0.0:50051] [--max-batch 16] [--target-ms 50]
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
* decode overlaps the GPU (server/serve.cpp:264-302), here one step earlier: every request
  is decoded on its own gRPC handler thread as it arrives, so the batcher collects ready
  pixels and the worker only stages them and launches, while the next batch's images decode
  during the current batch's GPU time.  The decoder is PIL for every format (the reference
  decodes JPEG with nvJPEG and PNG with stb; pixel values of a lossy JPEG can differ by
  decoder).  An undecodable image is answered at once and never takes a batch slot;
* responses carry the task's fields -- boxes, rotated boxes, top-5 classes, or boxes plus
  RLE masks at proto resolution with the letterbox geometry -- and queue_ms, infer_ms and
  the batch size (server/serve.cpp:193-256); an undecodable image is INVALID_ARGUMENT
  "image decode failed".  The slack formula's decode term is an EMA of the worker's per-batch
  staging time (upload + preprocess).

All engine calls happen on the one worker thread (the engine handle is not thread-safe);
gRPC handler threads only enqueue and wait.
"""
from __future__ import annotations

import argparse
import collections
import io
import json
import os
import sys
import threading
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

import yoloproto as pb

TASK_NAMES = {0: "detect", 1: "obb", 2: "classify", 3: "segment"}
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
    """HxWx3 BGR u8 (the engine's input layout) from encoded image bytes, None if undecodable."""
    try:
        from PIL import Image
        with Image.open(io.BytesIO(data)) as im:
            if im.mode != "RGB":
                im = im.convert("RGB")
            w, h = im.size
            rgb = np.frombuffer(im.tobytes(), np.uint8).reshape(h, w, 3)
        if h < 1 or w < 1:
            return None
        # three plane copies: numpy runs them without the GIL, unlike a reversed-stride copy
        bgr = np.empty_like(rgb)
        bgr[..., 0] = rgb[..., 2]
        bgr[..., 1] = rgb[..., 1]
        bgr[..., 2] = rgb[..., 0]
        return bgr
    except Exception:
        return None


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

class _Request:
    __slots__ = ("img", "arrival", "resp", "error", "done")

    def __init__(self):
        self.img = None
        self.arrival = time.monotonic()
        self.resp = pb.DetectResponse()
        self.error = None
        self.done = threading.Event()


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
    """Batcher + engine worker.  `submit` (decode + enqueue) is called from any thread."""

    def __init__(self, models: list[Model], target_ms: float = 50.0, log=print):
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
        self._stop = False
        self._worker = threading.Thread(target=self._work, name="yoloserve-worker", daemon=True)
        self._worker.start()

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

    def submit(self, image: bytes, model: str = "") -> _Request:
        """Decodes on the calling thread, then queues; the returned request's `done` is set
        when its response (or error) is ready."""
        mi = self.model_index(model)
        r = _Request()
        r.img = decode_image(image)
        if r.img is None:
            r.error = "image decode failed"
            r.resp.task = self.models[mi].task_name
            r.done.set()
            return r
        with self.cv:
            if self._stop:
                r.error = "server shutting down"
                r.done.set()
                return r
            self.models[mi].queue.append(r)
            self.cv.notify_all()
        return r

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
                self.cv.wait(None if pick < 0 else min(max(slack, 0.0) * 1e-3, 2e-4))
            m = self.models[pick]
            batch = [m.queue.popleft() for _ in range(min(len(m.queue), m.max_batch))]
        return pick, batch

    def _work(self):
        prev = None
        try:
            while True:
                got = self._collect()
                if got is None:
                    break
                mi, batch = got
                if prev is not None:
                    self._finish(*prev)
                    prev = None
                m = self.models[mi]
                t0 = time.monotonic()
                for i, r in enumerate(batch):
                    self._stage(m, i, r.img)
                    r.img = None
                launch = time.monotonic()
                self.stage_ema = 0.9 * self.stage_ema + 0.1 * (launch - t0) * 1e3
                m.eng.run_async(len(batch))
                prev = (mi, batch, launch)
                with self.cv:
                    idle = all(not q.queue for q in self.models)
                if idle:                  # no traffic behind it: answer now
                    self._finish(*prev)
                    prev = None
        except Exception as ex:        # an engine failure fails everything in flight
            self.log(f"[serve] worker stopped: {ex!r}")
            if prev is not None:
                for r in prev[1]:
                    r.error = f"engine failure: {ex}"
                    r.done.set()
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
                    r.done.set()

    def _finish(self, mi: int, batch: list, launch: float):
        m = self.models[mi]
        m.eng.sync()
        infer_ms = (time.monotonic() - launch) * 1e3
        for i, r in enumerate(batch):
            resp = r.resp
            resp.task = m.task_name
            self._fill(m, i, resp)
            resp.queue_ms = (launch - r.arrival) * 1e3
            resp.infer_ms = infer_ms
            resp.batch = len(batch)
            r.done.set()
        before = self.served
        self.served += len(batch)
        if self.served // 5000 != before // 5000:
            self.log(f"[serve] {self.served} imgs, B={len(batch)} gpu {infer_ms:.2f} ms "
                     f"({len(batch) * 1e3 / max(infer_ms, 1e-6):.0f} img/s in-batch)")

    @staticmethod
    def _fill(m: Model, slot: int, resp):
        eng = m.eng
        if m.task == 2:
            ids, probs = eng.get_cls(slot, 5)
            for c, p in zip(ids.tolist(), probs.tolist()):
                resp.classes.add(id=int(c), prob=float(p))
        elif m.task == 1:
            for cx, cy, w, h, a, s, c in eng.get_obb(slot).tolist():
                resp.rboxes.add(cx=cx, cy=cy, w=w, h=h, angle=a, score=s, cls=int(c))
        else:
            dets = eng.get(slot)
            for x1, y1, x2, y2, s, c in dets.tolist():
                resp.boxes.add(x1=x1, y1=y1, x2=x2, y2=y2, score=s, cls=int(c))
            if m.task == 3:
                resp.mask_h, resp.mask_w = m.mask_hw
                resp.lb_scale, resp.lb_top, resp.lb_left = eng.slot_geom(slot)
                for j in range(len(dets)):
                    mk = eng.get_mask(slot, j)
                    if mk is None:
                        resp.masks.add()
                    else:
                        resp.masks.add(rle=rle_encode(mk).tolist())

    def stop(self):
        with self.cv:
            self._stop = True
            self.cv.notify_all()
        self._worker.join()
        for b in self.buffers.values():
            b.free()
        self.buffers.clear()


# ------------------------------------------------------------------ gRPC glue

def grpc_server(server: Server, addr: str, workers: int | None = None):
    """A started grpc.Server exposing `server` at `addr`; returns (grpc server, bound port)."""
    import grpc

    def detect(request, context):
        try:
            r = server.submit(request.image, request.model)
        except KeyError:
            context.abort(grpc.StatusCode.INVALID_ARGUMENT, f"unknown model: {request.model}")
        r.done.wait()
        if r.error == "image decode failed":
            context.abort(grpc.StatusCode.INVALID_ARGUMENT, r.error)
        elif r.error:
            context.abort(grpc.StatusCode.UNAVAILABLE, r.error)
        return r.resp

    handler = grpc.method_handlers_generic_handler(pb.SERVICE, {
        pb.METHOD: grpc.unary_unary_rpc_method_handler(
            detect, request_deserializer=pb.DetectRequest.FromString,
            response_serializer=pb.DetectResponse.SerializeToString)})
    # every in-flight request holds a handler thread while it waits for its batch
    nthreads = workers or max(64, 4 * sum(m.max_batch for m in server.models))
    gs = grpc.server(ThreadPoolExecutor(max_workers=nthreads),
                     options=[("grpc.max_receive_message_length", MAX_MSG),
                              ("grpc.max_send_message_length", MAX_MSG)])
    gs.add_generic_rpc_handlers((handler,))
    port = gs.add_insecure_port(addr)
    if port == 0:
        raise RuntimeError(f"cannot bind {addr}")
    gs.start()
    return gs, port


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
    """Closed-loop load: `concurrency` callers each send the next image as soon as the last
    answer arrives; returns throughput and latency percentiles."""
    cl = Client(addr)
    lat, batches, lock = [], [], threading.Lock()
    stop_at = time.monotonic() + seconds

    def caller(k):
        i = k
        while time.monotonic() < stop_at:
            t0 = time.monotonic()
            r = cl.detect(images[i % len(images)], model)
            dt = (time.monotonic() - t0) * 1e3
            with lock:
                lat.append(dt)
                batches.append(r.batch)
            i += concurrency

    t0 = time.monotonic()
    with ThreadPoolExecutor(max_workers=concurrency) as ex:
        list(ex.map(caller, range(concurrency)))
    wall = time.monotonic() - t0
    cl.close()
    a = np.array(lat)
    return dict(requests=int(a.size), img_per_s=a.size / wall, p50_ms=float(np.percentile(a, 50)),
                p99_ms=float(np.percentile(a, 99)), mean_batch=float(np.mean(batches)), concurrency=concurrency)


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
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
    a = ap.parse_args(argv)
    specs = a.dir or ["build/yolo11n"]
    models = load_models(specs, a.max_batch)
    srv = Server(models, a.target_ms)
    gs, port = grpc_server(srv, a.addr)
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
