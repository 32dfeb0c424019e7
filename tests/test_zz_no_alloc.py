"""The entry point that allocates nothing (yolo_detect_static) against the engine's own
decode + NMS (the DECODE ops + yolo_run_post of a detect handle), through the C ABI: two
calls in a row, the second with a smaller batch, must give exactly the engine's
detections, raw counts and kept counts (needs an MI355X)."""
import ctypes as C

import numpy as np
import pytest

import modelgen
import yolort
from oracle import graphfile, post

pytestmark = pytest.mark.gpu


def _strided(arr, stride, off):
    """[B,H,W,C] -> [B,H,W,stride] with the channels at off..off+C (other channels hold a
    fill value the kernels must never read)."""
    out = np.full(arr.shape[:3] + (stride,), 7.0, np.float16)
    out[..., off:off + arr.shape[3]] = arr
    return out


def test_detect_static_matches_engine(models):
    d = models("yolo11", "n")
    g = graphfile.load(d)
    B = 4
    frames = [modelgen.synth_frame(810, 1080, 20, 1), modelgen.synth_frame(640, 640, 50, 100),
              modelgen.synth_frame(1080, 1920, 20, 2), modelgen.synth_frame(720, 1280, 30, 9)]
    eng = yolort.Engine(d, B)
    bufs = []
    for s, f in enumerate(frames):
        b = yolort.DeviceBuffer(f.nbytes)
        eng.upload(b, f)
        eng.preprocess(b.ptr, f.shape[0], f.shape[1], s)
        bufs.append(b)
    eng.run(B)
    want = [eng.get(s) for s in range(B)]
    want_raw = [eng.raw_count(s) for s in range(B)]
    geoms = [eng.slot_geom(s) for s in range(B)]
    assert all(len(w) > 0 for w in want)

    # the engine's head tensors, re-laid out in caller buffers with strides and offsets
    dec = [op for op in g.ops if op.kind == "DECODE"]
    dev, levels = [], []
    heads_host = []
    for i, op in enumerate(dec):
        box = eng.read(op.a, B)
        cls = eng.read(op.b, B)
        heads_host.append((box, cls, op.stride))
        bs, bo = (72, 8) if i == 0 else (64, 0)
        cs, co = (96, 16) if i == 1 else (80, 0)
        hb, hc = _strided(box, bs, bo), _strided(cls, cs, co)
        db, dc = yolort.DeviceBuffer(hb.nbytes), yolort.DeviceBuffer(hc.nbytes)
        eng.upload(db, hb)
        eng.upload(dc, hc)
        dev += [db, dc]
        H, W = box.shape[1:3]
        levels.append([db.ptr, dc.ptr, H, W, op.stride, bs, bo, cs, co])
    dets = yolort.DeviceBuffer(B * 300 * 6 * 4)
    cnt = yolort.DeviceBuffer(B * 4)
    raw = yolort.DeviceBuffer(B * 4)
    stream = eng.lib.yolo_stream(eng.h)

    def fetch(n):
        hd = np.empty((n, 300, 6), np.float32)
        hcnt = np.empty(n, np.int32)
        hraw = np.empty(n, np.int32)
        for host, buf in ((hd, dets), (hcnt, cnt), (hraw, raw)):
            assert eng.lib.yolo_copy_d2h(eng.h, host.ctypes.data, buf.ptr, host.nbytes) == 0
        return hd, hcnt, hraw

    def check(slot_of, n):
        hd, hcnt, hraw = fetch(n)
        for i in range(n):
            s = slot_of[i]
            scale, top, left = geoms[s]
            k = int(hcnt[i])
            r = hd[i, :k]
            # yolo_get's un-letterbox, in the same float32 operations
            x1 = (r[:, 0] - np.float32(left)) / np.float32(scale)
            y1 = (r[:, 1] - np.float32(top)) / np.float32(scale)
            x2 = (r[:, 2] - np.float32(left)) / np.float32(scale)
            y2 = (r[:, 3] - np.float32(top)) / np.float32(scale)
            got = np.stack([x1, y1, x2, y2, r[:, 4], r[:, 5]], 1).astype(np.float64)
            print(f"call B={n} image {i} (slot {s}): kept {k} raw {int(hraw[i])}", flush=True)
            assert int(hraw[i]) == want_raw[s]
            assert k == len(want[s])
            np.testing.assert_array_equal(got, want[s])
            # and the oracle's decode + NMS on the same heads
            o = post.detect([(bx[s].astype(np.float32), cl[s].astype(np.float32), None, st)
                             for bx, cl, st in heads_host], 80)
            np.testing.assert_array_equal(r[:, 5].astype(int), o["cls"])
            np.testing.assert_allclose(r[:, 4], o["score"], rtol=0, atol=2e-6)

    # call 1: the whole batch
    assert yolort.detect_static(levels, B, 80, 0.25, 0.45, 300, dets.ptr, cnt.ptr, raw.ptr, stream) == 0
    check(list(range(B)), B)
    # call 2: one image (slot 2), a smaller input than the first call, in the same scratch
    one = []
    for lv in levels:
        db, dc, H, W, st, bs, bo, cs, co = lv
        one.append([db + 2 * H * W * bs * 2, dc + 2 * H * W * cs * 2, H, W, st, bs, bo, cs, co])
    dets_before = fetch(B)[0]
    assert yolort.detect_static(one, 1, 80, 0.25, 0.45, 300, dets.ptr, cnt.ptr, raw.ptr, stream) == 0
    check([2], 1)
    # only image 0's output records were rewritten
    np.testing.assert_array_equal(fetch(B)[0][1:], dets_before[1:])
    # inputs beyond the stated maximum are refused before any launch
    big = [[lv[0], lv[1], 128, 128, 8, lv[5], lv[6], lv[7], lv[8]] for lv in levels[:1]]
    assert yolort.detect_static(big, 16, 80, 0.25, 0.45, 300, dets.ptr, cnt.ptr, raw.ptr, stream) == -1
    for b in dev + bufs + [dets, cnt, raw]:
        b.free()
    eng.close()
