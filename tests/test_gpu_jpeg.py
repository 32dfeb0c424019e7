"""JPEG decode on the engine (needs an MI355X): yolo_stage_jpeg's input tensors against the
letterbox (classify: resize + crop) of PIL's decode of the same bytes, bit for bit -- PIL being
the decoder the CPU oracle (oracle/jpeg.py) is pinned to pixel for pixel in test_jpeg.py --
over sizes, qualities, chroma subsamplings, restart intervals and grayscale, with unsupported
and corrupt streams in the same batch and a staging offset."""
import io

import numpy as np
import pytest
from PIL import Image

import modelgen
import yolort
from oracle import post

pytestmark = pytest.mark.gpu


def _jpeg(h, w, seed, mode="RGB", **kw):
    rng = np.random.default_rng(seed)
    img = modelgen.synth_frame(h, w, max(1, (h * w) // 4000), seed)[..., ::-1]
    img = np.clip(img.astype(np.int32) + rng.integers(-12, 13, img.shape), 0, 255).astype(np.uint8)
    im = Image.fromarray(img)
    if mode == "L":
        im = im.convert("L")
    buf = io.BytesIO()
    im.save(buf, "JPEG", **kw)
    return buf.getvalue()


def _pil_bgr(data):
    with Image.open(io.BytesIO(data)) as im:
        return np.ascontiguousarray(np.asarray(im.convert("RGB"))[..., ::-1])


STREAMS = [
    dict(h=480, w=640, quality=90, subsampling=2),
    dict(h=1080, w=1920, quality=85, subsampling=2),
    dict(h=333, w=517, quality=95, subsampling=0),
    dict(h=641, w=479, quality=75, subsampling=1),
    dict(h=200, w=300, quality=80, mode="L"),
    dict(h=640, w=640, quality=90, subsampling=2, restart_marker_blocks=5),
    dict(h=97, w=131, quality=100, subsampling=2, optimize=True),
]


def _streams():
    out = []
    for i, s in enumerate(STREAMS):
        s = dict(s)
        out.append(_jpeg(s.pop("h"), s.pop("w"), 70 + i, **s))
    return out


@pytest.mark.parametrize("task", ["detect", "classify"])
def test_stage_jpeg_matches_pil(models, task):
    if task == "detect":
        d, S = models("yolo11", "n"), 640
        want_fn = lambda im: post.letterbox(im, S, S)
    else:
        d, S = models("yolo11", "n", "classify", imgsz=224, nc=1000), 224
        want_fn = lambda im: post.preprocess_cls(im, S)
    good = _streams()
    prog = _jpeg(120, 160, 5, quality=90, progressive=True)
    trunc = good[0][:len(good[0]) // 2]
    batch = good[:3] + [prog] + good[3:5] + [trunc] + good[5:]
    eng = yolort.Engine(d, len(batch), yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    print(f"stage_jpeg {task}: {len(batch)} streams", flush=True)
    res = eng.stage_jpeg(batch)
    eng.sync()
    got = eng.read(0, len(batch))
    for i, (st, h, w) in enumerate(res):
        if i == 3:
            assert st == yolort.JPEG_UNSUPPORTED
            continue
        if i == 6:
            assert st == yolort.JPEG_INVALID
            continue
        assert st == yolort.JPEG_STAGED, (i, st)
        img = _pil_bgr(batch[i])
        assert (h, w) == img.shape[:2]
        np.testing.assert_array_equal(got[i], want_fn(img), err_msg=f"stream {i}")
        if task == "detect":
            scale, top, left = eng.slot_geom(i)
            assert (np.float32(scale), top, left) == post.letterbox_geom(S, S, h, w)[:3]
    # a second call at an offset restages slots 2 and 3 only, the others keep their inputs
    before = got.copy()
    res2 = eng.stage_jpeg([good[6], good[4]], first_slot=2)
    eng.sync()
    after = eng.read(0, len(batch))
    assert [r[0] for r in res2] == [yolort.JPEG_STAGED] * 2
    np.testing.assert_array_equal(after[2], want_fn(_pil_bgr(good[6])))
    np.testing.assert_array_equal(after[3], want_fn(_pil_bgr(good[4])))
    keep = [s for s in range(len(batch)) if s not in (2, 3)]
    np.testing.assert_array_equal(after[keep], before[keep])
    eng.close()


def test_stage_jpeg_detections_equal_pixel_staging(models):
    """The whole frame (decode on the engine + network + NMS) returns the same detections as
    staging PIL's pixels."""
    d = models("yolo11", "n")
    streams = _streams()[:4]
    eng = yolort.Engine(d, 4, yolort.YOLO_NOTUNE)
    assert all(r[0] == yolort.JPEG_STAGED for r in eng.stage_jpeg(streams))
    eng.run(4)
    a = [eng.get(s) for s in range(4)]
    bufs = []
    for im in (_pil_bgr(s) for s in streams):
        b = yolort.PinnedBuffer(im.shape)
        b.array[...] = im
        bufs.append((b, im.shape[:2]))
    eng.stage_frames([b.ptr for b, _ in bufs], [hw[0] for _, hw in bufs], [hw[1] for _, hw in bufs])
    eng.run(4)
    for s in range(4):
        np.testing.assert_array_equal(eng.get(s), a[s])
    for b, _ in bufs:
        b.free()
    eng.close()


def test_decode_next_batch_keeps_results(models):
    """yolo_decode_jpeg of the next batch leaves the current batch's results and slot geometry
    alone (the server decodes batch k+1 while reading batch k); yolo_letterbox_decoded then
    stages exactly what yolo_stage_jpeg would."""
    d = models("yolo11", "n")
    streams = _streams()
    a, b = streams[:3], [streams[4], streams[6], streams[2]]
    eng = yolort.Engine(d, 3, yolort.YOLO_NOTUNE)
    assert all(r[0] == yolort.JPEG_STAGED for r in eng.stage_jpeg(a))
    eng.run(3)
    got_a = [eng.get(s) for s in range(3)]
    geom_a = [eng.slot_geom(s) for s in range(3)]
    print("decode next batch", flush=True)
    assert all(r[0] == yolort.JPEG_STAGED for r in eng.decode_jpeg(b))
    eng.sync()
    for s in range(3):
        np.testing.assert_array_equal(eng.get(s), got_a[s])
        assert eng.slot_geom(s) == geom_a[s]
    assert eng.letterbox_decoded(3) == 3
    eng.run(3)
    got_b = [eng.get(s) for s in range(3)]
    inp_b = eng.read(0, 3)
    for s in range(3):
        np.testing.assert_array_equal(inp_b[s], post.letterbox(_pil_bgr(b[s]), 640, 640))
    assert all(r[0] == yolort.JPEG_STAGED for r in eng.stage_jpeg(b))
    eng.run(3)
    for s in range(3):
        np.testing.assert_array_equal(eng.get(s), got_b[s])
    # staging pixels into a slot forgets the frame decoded there
    img = _pil_bgr(b[0])
    pb = yolort.PinnedBuffer(img.shape)
    pb.array[...] = img
    eng.stage_frames([pb.ptr], [img.shape[0]], [img.shape[1]], yolort.PIXEL_BGR, 1)
    assert eng.letterbox_decoded(3) == 2
    eng.sync()
    pb.free()
    eng.close()


def test_tickets_equal_stage_jpeg(models):
    """Streams submitted at arrival (entropy decoding started at once on the library's threads)
    and decoded later by yolo_decode_tickets stage exactly what yolo_stage_jpeg does; a
    truncated stream is reported corrupt, a progressive one gets no ticket, and released
    tickets and repeated rounds recycle the pinned buffers."""
    d = models("yolo11", "n")
    streams = _streams()
    trunc = streams[0][:len(streams[0]) // 2]
    assert yolort.jpeg_submit(_jpeg(120, 160, 5, quality=90, progressive=True)) is None
    eng = yolort.Engine(d, len(streams) + 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    want = [post.letterbox(_pil_bgr(s), 640, 640) for s in streams]
    for rnd in range(3):
        spare = [yolort.jpeg_submit(s) for s in streams[:2]]
        for t in spare:
            yolort.jpeg_release(t)
        order = streams[rnd:] + streams[:rnd]
        wants = want[rnd:] + want[:rnd]
        tickets = [yolort.jpeg_submit(s) for s in order] + [yolort.jpeg_submit(trunc)]
        assert all(t is not None for t in tickets)
        print(f"round {rnd}: decode {len(tickets)} tickets", flush=True)
        res = eng.decode_tickets(tickets)
        assert [r[0] for r in res] == [yolort.JPEG_STAGED] * len(order) + [yolort.JPEG_INVALID]
        assert eng.letterbox_decoded(len(tickets)) == len(order)
        eng.sync()
        got = eng.read(0, len(tickets))
        for s in range(len(order)):
            np.testing.assert_array_equal(got[s], wants[s], err_msg=f"round {rnd} slot {s}")
    eng.close()
