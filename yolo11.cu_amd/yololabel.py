"""Labeling client for the detection server (the CLI of the reference's client/label.py).

    python yolo11.cu_amd/yololabel.py imgs/*.jpg --out labels.jsonl      # JSONL, one line per image
    python yolo11.cu_amd/yololabel.py imgs/*.jpg --coco labels.json      # COCO annotations
    python yolo11.cu_amd/yololabel.py bus.jpg --bench 2000 -c 64          # throughput / latency

Talks to `yolo.Yolo/Detect` through the run-time schema (no generated stubs or grpc_tools).

Outputs keep the reference client's formats, since other tools read them: the JSONL record
keys per task (client/label.py:63-76) and the COCO field names and class tables
(client/label.py:86-101,118-163).  The code is this module's own:

* a response becomes a record through one table, RESULT_FIELDS (repeated response field ->
  the message fields copied), the first non-empty repeated field naming the record's kind;
* COCO annotations are built per record kind; OBB corners come from one rotation of the
  half-extent corners (numpy); segment masks -- instead of OpenCV contour polygons, which
  need cv2 -- are COCO uncompressed RLE in original-image pixels: each original pixel maps
  through the letterbox (x * scale + left, at 4 letterbox pixels per mask pixel) to the mask
  pixel that covers it, counts column-major as COCO defines them;
* --bench runs `concurrency` closed-loop callers that share one request counter and report
  per-request latency percentiles and the server's mean batch size.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import threading
import time

import numpy as np

import yoloproto as pb

# standard class-name tables of the two label sets the models are trained on
COCO80 = ("person bicycle car motorcycle airplane bus train truck boat traffic_light fire_hydrant stop_sign "
          "parking_meter bench bird cat dog horse sheep cow elephant bear zebra giraffe backpack umbrella "
          "handbag tie suitcase frisbee skis snowboard sports_ball kite baseball_bat baseball_glove skateboard "
          "surfboard tennis_racket bottle wine_glass cup fork knife spoon bowl banana apple sandwich orange "
          "broccoli carrot hot_dog pizza donut cake chair couch potted_plant bed dining_table toilet tv laptop "
          "mouse remote keyboard cell_phone microwave oven toaster sink refrigerator book clock vase scissors "
          "teddy_bear hair_drier toothbrush").split()
DOTA15 = ("plane ship storage_tank baseball_diamond tennis_court basketball_court ground_track_field harbor "
          "bridge large_vehicle small_vehicle helicopter roundabout soccer_ball_field swimming_pool").split()
PROTO_STRIDE = 4          # letterbox pixels per proto-mask pixel

# repeated response field -> message fields copied into the record, in precedence order: a
# response carries exactly one kind of result (classify, obb, detect/segment)
RESULT_FIELDS = (
    ("classes", ("id", "prob")),
    ("rboxes", ("cx", "cy", "w", "h", "angle", "score", "cls")),
    ("boxes", ("x1", "y1", "x2", "y2", "score", "cls")),
)


def record(resp) -> dict:
    """The JSONL record of one response (without the image path)."""
    rec = {"task": resp.task or "detect"}
    for name, keys in RESULT_FIELDS:
        msgs = getattr(resp, name)
        if len(msgs) or name == "boxes":
            rec[name] = [dict(zip(keys, (getattr(m, k) for k in keys))) for m in msgs]
            break
    if "boxes" in rec and len(resp.masks):
        rec.update(mask_h=resp.mask_h, mask_w=resp.mask_w,
                   letterbox={"scale": resp.lb_scale, "top": resp.lb_top, "left": resp.lb_left},
                   masks=[list(m.rle) for m in resp.masks])
    return rec


def rle_to_mask(runs, h: int, w: int) -> np.ndarray:
    vals = np.arange(len(runs)) % 2
    m = np.repeat(vals, np.asarray(runs, np.int64)).astype(np.uint8)
    if m.size != h * w:
        raise ValueError(f"runs cover {m.size} pixels, expected {h * w}")
    return m.reshape(h, w)


def mask_to_original(mask: np.ndarray, lb: dict, img_h: int, img_w: int) -> np.ndarray:
    """Proto-resolution letterbox-space mask -> mask over the original image's pixels."""
    mh, mw = mask.shape
    ys = ((np.arange(img_h) + 0.5) * lb["scale"] + lb["top"]) / PROTO_STRIDE
    xs = ((np.arange(img_w) + 0.5) * lb["scale"] + lb["left"]) / PROTO_STRIDE
    iy = np.clip(np.floor(ys).astype(np.int64), 0, mh - 1)
    ix = np.clip(np.floor(xs).astype(np.int64), 0, mw - 1)
    return mask[iy[:, None], ix[None, :]]


def coco_rle(mask: np.ndarray) -> dict:
    """COCO uncompressed RLE: column-major runs starting with background."""
    flat = mask.T.ravel() != 0
    if flat.size == 0:
        return {"counts": [0], "size": list(mask.shape)}
    cuts = np.flatnonzero(flat[1:] != flat[:-1]) + 1
    runs = np.diff(np.concatenate(([0], cuts, [flat.size])))
    if flat[0]:
        runs = np.concatenate(([0], runs))
    return {"counts": runs.astype(int).tolist(), "size": [int(mask.shape[0]), int(mask.shape[1])]}


# half-extent signs of the four corners, counter-clockwise from the (-w/2, -h/2) corner
_CORNER_SIGNS = np.array([[-1.0, -1.0], [1.0, -1.0], [1.0, 1.0], [-1.0, 1.0]])


def obb_corners(b: dict):
    """Corners of a rotated box (cx, cy, w, h, angle in radians) as four (x, y) tuples."""
    c, s = np.cos(b["angle"]), np.sin(b["angle"])
    rot = np.array([[c, -s], [s, c]])
    pts = (_CORNER_SIGNS * (0.5 * np.array([b["w"], b["h"]]))) @ rot.T + np.array([b["cx"], b["cy"]])
    return [(float(x), float(y)) for x, y in pts]


def _xywh(x0, y0, x1, y1) -> list:
    return [round(float(v), 2) for v in (x0, y0, x1 - x0, y1 - y0)]


def _box_annotations(res: dict, hw: tuple[int, int]):
    """(category, score, bbox, area, segmentation | None) per box of a detect/segment record."""
    for j, b in enumerate(res.get("boxes", [])):
        bbox = _xywh(b["x1"], b["y1"], b["x2"], b["y2"])
        seg = None
        if "masks" in res:
            m = rle_to_mask(res["masks"][j], res["mask_h"], res["mask_w"])
            seg = coco_rle(mask_to_original(m, res["letterbox"], *hw))
        yield b["cls"], b["score"], bbox, round((b["x2"] - b["x1"]) * (b["y2"] - b["y1"]), 2), seg


def _rbox_annotations(res: dict, hw: tuple[int, int]):
    """The same for an OBB record: the corner polygon and its axis-aligned bounds."""
    for b in res.get("rboxes", []):
        pts = np.array(obb_corners(b))
        lo, hi = pts.min(0), pts.max(0)
        poly = [round(float(v), 2) for v in pts.ravel()]
        yield b["cls"], b["score"], _xywh(lo[0], lo[1], hi[0], hi[1]), round(b["w"] * b["h"], 2), [poly]


def coco(results: dict, sizes: dict) -> dict:
    """COCO annotations for {path: record}; `sizes` maps path -> (h, w) of the original image."""
    images, anns = [], []
    for iid, path in enumerate(sorted(results), 1):
        res, hw = results[path], sizes[path]
        images.append({"id": iid, "file_name": os.path.basename(path), "height": hw[0], "width": hw[1]})
        for gen in (_box_annotations, _rbox_annotations):
            for cat, score, bbox, area, seg in gen(res, hw):
                a = {"id": len(anns) + 1, "image_id": iid, "category_id": cat, "iscrowd": 0,
                     "score": round(score, 4), "bbox": bbox, "area": area}
                if seg is not None:
                    a["segmentation"] = seg
                anns.append(a)
    names = DOTA15 if any(r.get("task") == "obb" for r in results.values()) else COCO80
    return {"images": images, "annotations": anns,
            "categories": [{"id": i, "name": n} for i, n in enumerate(names)]}


def image_size(path: str) -> tuple[int, int]:
    from PIL import Image
    with Image.open(path) as im:
        return im.size[1], im.size[0]


class _Load:
    """Closed-loop load: `callers` threads take request numbers from one shared counter
    until `total` requests were sent; each records its latency and the batch it rode in."""

    def __init__(self, call, request, total: int, callers: int):
        self.call, self.request, self.total, self.callers = call, request, total, callers
        self.lock = threading.Lock()
        self.sent = 0
        self.lat_ms = np.zeros(total)
        self.batch = np.zeros(total)

    def _caller(self):
        while True:
            with self.lock:
                i = self.sent
                if i >= self.total:
                    return
                self.sent += 1
            t = time.perf_counter()
            resp = self.call(self.request)
            self.lat_ms[i] = (time.perf_counter() - t) * 1e3
            self.batch[i] = resp.batch

    def run(self) -> dict:
        threads = [threading.Thread(target=self._caller, daemon=True) for _ in range(self.callers)]
        t = time.perf_counter()
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        wall = time.perf_counter() - t
        p50, p95, p99 = np.percentile(self.lat_ms, [50, 95, 99])
        return {"requests": self.total, "seconds": wall, "img_per_s": self.total / wall, "p50_ms": p50,
                "p95_ms": p95, "p99_ms": p99, "mean_batch": float(self.batch.mean())}


def _label_all(call, model: str, paths: list[str], callers: int) -> dict:
    """One request per image over `callers` threads; {path: record}."""
    out, lock, todo = {}, threading.Lock(), list(reversed(paths))

    def worker():
        while True:
            with lock:
                if not todo:
                    return
                p = todo.pop()
            with open(p, "rb") as f:
                rec = record(call(pb.DetectRequest(image=f.read(), model=model)))
            with lock:
                out[p] = rec

    threads = [threading.Thread(target=worker, daemon=True) for _ in range(max(1, min(callers, len(paths))))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="yololabel")
    ap.add_argument("images", nargs="+")
    ap.add_argument("--server", default="localhost:50051")
    ap.add_argument("--model", default="", help="model name on multi-model servers (dir basename)")
    ap.add_argument("-c", "--concurrency", type=int, default=64, help="requests in flight (feeds the batcher)")
    ap.add_argument("--out", default=None, help="write results as JSONL")
    ap.add_argument("--coco", default=None, help="write results as COCO annotations JSON")
    ap.add_argument("--bench", type=int, default=0, help="benchmark: send the first image N times")
    a = ap.parse_args(argv)

    import grpc
    ch = grpc.insecure_channel(a.server, [("grpc.max_receive_message_length", 64 << 20),
                                          ("grpc.max_send_message_length", 64 << 20)])
    call = ch.unary_unary(pb.FULL_METHOD, request_serializer=pb.DetectRequest.SerializeToString,
                          response_deserializer=pb.DetectResponse.FromString)
    try:
        if a.bench:
            with open(a.images[0], "rb") as f:
                req = pb.DetectRequest(image=f.read(), model=a.model)
            call(req)                                             # connection + graph warm-up
            st = _Load(call, req, a.bench, a.concurrency).run()
            print(f"bench {a.images[0]}: {st['requests']} requests, {a.concurrency} callers, "
                  f"{st['seconds']:.2f} s -> {st['img_per_s']:,.0f} img/s | latency ms p50 {st['p50_ms']:.1f} "
                  f"p95 {st['p95_ms']:.1f} p99 {st['p99_ms']:.1f} | server batch {st['mean_batch']:.1f}",
                  flush=True)
            return 0
        t = time.perf_counter()
        results = _label_all(call, a.model, a.images, a.concurrency)
        wall = time.perf_counter() - t
    finally:
        ch.close()
    print(f"{len(results)} images -> {a.server} in {wall:.2f} s ({len(results) / wall:,.0f} img/s)", flush=True)
    if a.coco:
        doc = coco(results, {p: image_size(p) for p in results})
        with open(a.coco, "w") as f:
            json.dump(doc, f)
        print(f"COCO: {a.coco}, {len(doc['images'])} images, {len(doc['annotations'])} annotations")
    if a.out:
        with open(a.out, "w") as f:
            f.writelines(json.dumps({"image": p, **results[p]}) + "\n" for p in a.images)
        print(f"JSONL: {a.out}, {len(a.images)} records")
    return 0


if __name__ == "__main__":
    sys.exit(main())
