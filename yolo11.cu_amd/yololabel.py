"""Labeling client for the detection server (the reference's client/label.py, same CLI).

    python yolo11.cu_amd/yololabel.py imgs/*.jpg --out labels.jsonl      # JSONL, one line per image
    python yolo11.cu_amd/yololabel.py imgs/*.jpg --coco labels.json      # COCO annotations
    python yolo11.cu_amd/yololabel.py bus.jpg --bench 2000 -c 64          # throughput / latency

Talks to `yolo.Yolo/Detect` through the run-time schema (no generated stubs or grpc_tools).
JSONL records carry the task and its fields as the reference client writes them
(client/label.py:57-71).  COCO export (client/label.py:118-163): boxes as xywh, OBB as the
4-corner polygon plus its axis-aligned box, and -- instead of cv2 contour polygons, which need
OpenCV -- segment masks as COCO uncompressed RLE in original-image pixels: each original pixel
maps through the letterbox (x * scale + left, at 4 letterbox pixels per mask pixel) to the
mask pixel that covers it; counts are column-major as COCO defines them.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

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


def record(resp) -> dict:
    """The JSONL record of one response (without the image path)."""
    out = {"task": resp.task or "detect"}
    if resp.classes:
        out["classes"] = [{"id": c.id, "prob": c.prob} for c in resp.classes]
    elif resp.rboxes:
        out["rboxes"] = [{"cx": b.cx, "cy": b.cy, "w": b.w, "h": b.h, "angle": b.angle, "score": b.score,
                          "cls": b.cls} for b in resp.rboxes]
    else:
        out["boxes"] = [{"x1": b.x1, "y1": b.y1, "x2": b.x2, "y2": b.y2, "score": b.score, "cls": b.cls}
                        for b in resp.boxes]
        if resp.masks:
            out["mask_h"], out["mask_w"] = resp.mask_h, resp.mask_w
            out["letterbox"] = {"scale": resp.lb_scale, "top": resp.lb_top, "left": resp.lb_left}
            out["masks"] = [list(m.rle) for m in resp.masks]
    return out


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


def obb_corners(b: dict):
    ca, sa = math.cos(b["angle"]), math.sin(b["angle"])
    hw, hh = b["w"] / 2, b["h"] / 2
    return [(b["cx"] + dx * ca - dy * sa, b["cy"] + dx * sa + dy * ca)
            for dx, dy in ((-hw, -hh), (hw, -hh), (hw, hh), (-hw, hh))]


def coco(results: dict, sizes: dict) -> dict:
    """COCO annotations for {path: record}; `sizes` maps path -> (h, w) of the original image."""
    images, anns = [], []
    aid = 1
    for iid, (path, res) in enumerate(sorted(results.items()), 1):
        h, w = sizes[path]
        images.append({"id": iid, "file_name": os.path.basename(path), "height": h, "width": w})
        for j, b in enumerate(res.get("boxes", [])):
            bw, bh = b["x2"] - b["x1"], b["y2"] - b["y1"]
            a = {"id": aid, "image_id": iid, "category_id": b["cls"], "iscrowd": 0, "score": round(b["score"], 4),
                 "bbox": [round(b["x1"], 2), round(b["y1"], 2), round(bw, 2), round(bh, 2)],
                 "area": round(bw * bh, 2)}
            if "masks" in res:
                m = rle_to_mask(res["masks"][j], res["mask_h"], res["mask_w"])
                a["segmentation"] = coco_rle(mask_to_original(m, res["letterbox"], h, w))
            anns.append(a)
            aid += 1
        for b in res.get("rboxes", []):
            pts = obb_corners(b)
            xs, ys = [p[0] for p in pts], [p[1] for p in pts]
            anns.append({"id": aid, "image_id": iid, "category_id": b["cls"], "iscrowd": 0,
                         "score": round(b["score"], 4),
                         "segmentation": [[round(v, 2) for p in pts for v in p]],
                         "bbox": [round(min(xs), 2), round(min(ys), 2), round(max(xs) - min(xs), 2),
                                  round(max(ys) - min(ys), 2)],
                         "area": round(b["w"] * b["h"], 2)})
            aid += 1
    names = DOTA15 if any(r.get("task") == "obb" for r in results.values()) else COCO80
    return {"images": images, "annotations": anns, "categories": [{"id": i, "name": n} for i, n in enumerate(names)]}


def image_size(path: str) -> tuple[int, int]:
    from PIL import Image
    with Image.open(path) as im:
        return im.size[1], im.size[0]


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

    if a.bench:
        data = open(a.images[0], "rb").read()
        call(pb.DetectRequest(image=data, model=a.model))          # warm-up
        lat, batches = [], []

        def one(_):
            t0 = time.perf_counter()
            r = call(pb.DetectRequest(image=data, model=a.model))
            lat.append((time.perf_counter() - t0) * 1e3)
            batches.append(r.batch)

        t0 = time.perf_counter()
        with ThreadPoolExecutor(a.concurrency) as ex:
            list(ex.map(one, range(a.bench)))
        dt = time.perf_counter() - t0
        q = np.percentile(np.array(lat), [50, 95, 99])
        print(f"{len(lat)} imgs in {dt:.2f}s = {len(lat) / dt:,.0f} img/s   latency p50={q[0]:.1f} "
              f"p95={q[1]:.1f} p99={q[2]:.1f} ms   avg batch={np.mean(batches):.1f}", flush=True)
        ch.close()
        return 0

    results = {}

    def label(path):
        r = call(pb.DetectRequest(image=open(path, "rb").read(), model=a.model))
        results[path] = record(r)

    t0 = time.perf_counter()
    with ThreadPoolExecutor(a.concurrency) as ex:
        list(ex.map(label, a.images))
    dt = time.perf_counter() - t0
    ch.close()
    print(f"labeled {len(a.images)} images in {dt:.2f}s ({len(a.images) / dt:,.0f} img/s)", flush=True)
    if a.coco:
        doc = coco(results, {p: image_size(p) for p in results})
        with open(a.coco, "w") as f:
            json.dump(doc, f)
        print(f"wrote {a.coco} ({len(doc['annotations'])} annotations)")
    if a.out:
        with open(a.out, "w") as f:
            for p in a.images:
                f.write(json.dumps({"image": p, **results[p]}) + "\n")
        print(f"wrote {a.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
