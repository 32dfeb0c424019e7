"""GPU frame-level parity through the C ABI (needs an MI355X).

  * letterbox: the device kernel against the oracle's fp32 restatement (bit-exact target)
  * batch self-consistency (engine/engine.cu:1914-1936) and graph-replay determinism
(the whole frame of each BASELINE configuration against the oracle: test_gpu_configs.py)
"""
import numpy as np
import pytest

import modelgen
import yolort
from oracle import graphfile, interp, post

pytestmark = pytest.mark.gpu


def _letterbox_gpu(eng, img, slot=0):
    buf = yolort.DeviceBuffer(img.nbytes)
    eng.upload(buf, img)
    eng.preprocess(buf.ptr, img.shape[0], img.shape[1], slot)
    eng.sync()
    return buf


@pytest.mark.parametrize("hw", [(810, 1080), (1080, 1920), (640, 640), (480, 640), (333, 517), (1200, 700)])
def test_letterbox_exact(models, hw):
    d = models("yolo11", "n")
    img = modelgen.synth_frame(hw[0], hw[1], 20, hw[0] + hw[1])
    eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    buf = _letterbox_gpu(eng, img)
    got = eng.read(0, 1)[0]
    want = post.letterbox(img, 640, 640)
    diff = np.abs(got.astype(np.float32) - want.astype(np.float32))
    exact = float((got == want).mean())
    print(f"letterbox {hw}: exact {exact:.6f} max diff {diff.max():.3e}", flush=True)
    scale, top, left = eng.slot_geom(0)
    s2, t2, l2, _, _ = post.letterbox_geom(640, 640, hw[0], hw[1])
    assert (np.float32(scale), top, left) == (s2, t2, l2)
    np.testing.assert_array_equal(got, want)     # bit-exact: same fp32 arithmetic, same order
    buf.free()
    eng.close()


def test_batch_consistency_and_replay(models):
    """B identical frames -> identical per-slot results; repeated graph launches agree."""
    d = models("yolo11", "n")
    img = modelgen.synth_frame(810, 1080, 20, 1)
    B = 4
    eng = yolort.Engine(d, B)
    bufs = [_letterbox_gpu(eng, img, s) for s in range(B)]
    eng.run(B)
    first = [eng.get(s) for s in range(B)]
    for s in range(1, B):
        np.testing.assert_array_equal(first[s], first[0])
    for _ in range(3):
        eng.run(B)
        for s in range(B):
            np.testing.assert_array_equal(eng.get(s), first[s])
    # batch-1 graph on slot 0 gives the same result as the batch-4 graph
    eng.run(1)
    np.testing.assert_array_equal(eng.get(0), first[0])
    for b in bufs:
        b.free()
    eng.close()


def test_frame_graph_pipeline(models):
    """The whole-frame graph (H2D + letterbox + net + decode + NMS) equals the
    preprocess-then-run path of the same handle, bit for bit, over several replays with new
    frame contents in the same pinned buffers (no re-capture)."""
    d = models("yolo11", "n")
    eng = yolort.Engine(d, 2)
    imgs = [modelgen.synth_frame(810, 1080, 20, 1), modelgen.synth_frame(720, 1280, 20, 9)]
    pins = [yolort.PinnedBuffer(im.shape) for im in imgs]
    devs = [yolort.DeviceBuffer(im.nbytes) for im in imgs]
    for p, im in zip(pins, imgs):
        p.array[...] = im
    eng.frame_graph([b.ptr for b in devs], [im.shape[0] for im in imgs], [im.shape[1] for im in imgs],
                    [p.ptr for p in pins])
    for rep in range(3):
        if rep == 2:   # new contents in the same pinned buffers, no re-capture
            pins[0].array[...] = modelgen.synth_frame(810, 1080, 25, 77)
        eng.frame_run()
        got = [eng.get(s) for s in range(2)]
        raw = [eng.raw_count(s) for s in range(2)]
        # the same frames through per-slot letterbox + the batch-2 graph of this handle
        bufs = [_letterbox_gpu(eng, np.ascontiguousarray(pins[s].array), s) for s in range(2)]
        eng.run(2)
        for s in range(2):
            assert eng.raw_count(s) == raw[s]
            np.testing.assert_array_equal(eng.get(s), got[s])
        for b in bufs:
            b.free()
    for p in pins:
        p.free()
    eng.close()


def test_thresholds_runtime(models):
    """conf / IoU / max_det are device parameters: graphs pick them up without re-capture."""
    d = models("yolo11", "n")
    img = modelgen.synth_frame(810, 1080, 20, 1)
    eng = yolort.Engine(d, 1)
    buf = _letterbox_gpu(eng, img)
    for conf, iou, md in [(0.25, 0.45, 300), (0.25, 0.7, 300), (0.5, 0.45, 300), (0.25, 0.45, 7),
                          (0.0, 0.45, 300), (0.0, 0.7, 100), (0.001, 0.5, 300)]:
        eng.set_thresholds(conf, iou, md)
        eng.run(1)
        got = eng.get(0)
        g = graphfile.load(d)
        I = interp.Interp(g, 1, round_fp16=True)
        I.set_input(eng.read(0, 1).astype(np.float32))
        # decode/NMS parity on the GPU's own head tensors
        heads = []
        for op in [o for o in g.ops if o.kind == "DECODE"]:
            heads.append((eng.read(op.a)[0].astype(np.float32), eng.read(op.b)[0].astype(np.float32), None, op.stride))
        want = post.detect(heads, 80, conf, iou, md)
        print(f"conf {conf} iou {iou} max_det {md}: kept {len(got)} (oracle {len(want['score'])})", flush=True)
        assert len(got) == len(want["score"])
        np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
    buf.free()
    eng.close()


@pytest.mark.skip(reason="branch-concurrent graph capture is switched off: capturing the "
                  "fork/join plan crashed inside hipStreamEndCapture and the cause is not isolated")
def test_concurrent_branches_equal_serial(models):
    """The multi-stream plan (independent branches on side streams) must give bit-identical
    tensors and detections to the single-stream order, on every graph replay."""
    pytest.skip("disabled")


@pytest.mark.parametrize("task", ["detect", "segment"])
def test_dag_graph_equals_serial_graph(models, task):
    """Graphs built as a dependency DAG of per-op nodes (independent branches run
    concurrently) give bit-identical detections and masks to the single-stream graph, over
    replays; the frame graph too."""
    d = models("yolo11", "n", task)
    img = modelgen.synth_frame(810, 1080, 20, 3)
    res = {}
    for name, flags in (("dag", yolort.YOLO_NOTUNE | yolort.YOLO_DAGGRAPH), ("serial", yolort.YOLO_NOTUNE)):
        eng = yolort.Engine(d, 2, flags)
        bufs = [_letterbox_gpu(eng, img, s) for s in range(2)]
        outs = []
        for _ in range(3):
            eng.run(2)
            outs.append([eng.get(s) for s in range(2)])
        if task == "segment":
            outs.append([eng.get_mask(0, i) for i in range(min(3, len(outs[0][0])))])
        dev = yolort.DeviceBuffer(img.nbytes)
        eng.upload(dev, img)
        eng.frame_graph([dev.ptr], [img.shape[0]], [img.shape[1]])
        eng.frame_run()
        outs.append([eng.get(0)])
        res[name] = outs
        dev.free()
        for b in bufs:
            b.free()
        eng.close()
    for a, b in zip(res["dag"], res["serial"]):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    assert len(res["dag"][0][0]) > 0


@pytest.mark.parametrize("scale,B", [("n", 2), ("x", 3)])
def test_attention_carries_v_copies(models, scale, B):
    """C2PSA's V-gather copies run as trailing blocks of the attention launch (one launch
    unit with the ATTN op); every tensor and the detections equal a one-op-per-launch
    engine's (YOLO_NOGROUP) bit for bit."""
    d = models("yolo11", scale)
    g = graphfile.load(d)
    imgs = [modelgen.synth_frame(640, 640, 30, 40 + s) for s in range(B)]
    res = {}
    for name, flags in (("carried", 0), ("single", yolort.YOLO_NOGROUP)):
        eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH | flags)
        kinds = [eng.op_info(k)["kind"] for k in range(eng.num_ops)]
        attn = [k for k, kd in enumerate(kinds) if kd == "ATTN"]
        copies = [k for k, kd in enumerate(kinds) if kd == "COPYC"]
        assert attn and copies
        if name == "carried":
            # each attention's unit holds the copies just before it
            for a in attn:
                mine = [k for k in copies if k < a and eng.op_unit(k) == eng.op_unit(a)]
                assert mine, (a, [eng.op_unit(k) for k in copies], eng.op_unit(a))
            assert all(eng.op_unit(k) in {eng.op_unit(a) for a in attn} for k in copies)
        else:
            assert len({eng.op_unit(k) for k in copies + attn}) == len(copies + attn)
        bufs = [_letterbox_gpu(eng, im, s) for s, im in enumerate(imgs)]
        eng.run(B)
        res[name] = [eng.get(s) for s in range(B)] + [eng.read(t, B) for t in range(len(g.tens))]
        for b in bufs:
            b.free()
        eng.close()
    for x, y in zip(res["carried"], res["single"]):
        np.testing.assert_array_equal(x, y)
    assert sum(len(r) for r in res["carried"][:B]) > 0


def test_frame_graph_nms_variants(models):
    """The frame graph holds both NMS variants and picks by the previous frame's candidate
    count: a sparse frame (294 candidates) and a crowded one (conf 0.05: thousands) alternate
    on one handle; every run must equal a YOLO_NMS_BLOCK handle's run of the same frame."""
    d = models("yolo11", "n")
    img = modelgen.synth_frame(810, 1080, 20, 1)
    engs = [yolort.Engine(d, 1), yolort.Engine(d, 1, yolort.YOLO_NMS_BLOCK)]
    bufs = []
    for e in engs:
        b = yolort.DeviceBuffer(img.nbytes)
        e.upload(b, img)
        e.frame_graph([b.ptr], [810], [1080])
        bufs.append(b)
    raws = {}
    for conf in (0.25, 0.05, 0.05, 0.25, 0.25, 0.05):
        outs = []
        for e in engs:
            e.set_thresholds(conf, 0.45, 300)
            e.frame_run()
            outs.append((e.get(0), e.raw_count(0)))
        print(f"conf {conf}: raw {outs[0][1]}, kept {len(outs[0][0])}", flush=True)
        assert outs[0][1] == outs[1][1]
        np.testing.assert_array_equal(outs[0][0], outs[1][0])
        raws[conf] = outs[0][1]
    assert raws[0.25] <= 512 < raws[0.05]   # both variants were taken
    for b, e in zip(bufs, engs):
        b.free()
        e.close()


@pytest.mark.parametrize("task", ["detect", "classify"])
def test_stage_frames_layouts(models, task):
    """yolo_stage_frames (the server's batch staging from pinned memory) letterboxes -- or, for
    a classify handle, resizes and crops -- every slot exactly as the oracle does, from BGR
    and from R, G, B, X frames alike; a later call with larger frames regrows the staging."""
    if task == "detect":
        d, S = models("yolo11", "n"), 640
        want_fn = lambda im: post.letterbox(im, S, S)
    else:
        d, S = models("yolo11", "n", "classify", imgsz=224, nc=1000), 224
        want_fn = lambda im: post.preprocess_cls(im, S)
    eng = yolort.Engine(d, 4, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    pinned = []
    for sizes in ([(333, 517), (640, 640), (810, 1080), (200, 90)],
                  [(1080, 1920), (1200, 700), (480, 640)]):
        frames = [modelgen.synth_frame(h, w, 12, h + 3 * w) for h, w in sizes]
        want = [want_fn(im) for im in frames]
        for fmt in (yolort.PIXEL_BGR, yolort.PIXEL_RGBX):
            bufs = []
            for im in frames:
                if fmt == yolort.PIXEL_RGBX:
                    im = np.concatenate([im[..., ::-1], np.full(im.shape[:2] + (1,), 201, np.uint8)], axis=2)
                b = yolort.PinnedBuffer(im.shape)
                b.array[...] = im
                bufs.append(b)
            print(f"stage {task} fmt {fmt} sizes {sizes}", flush=True)
            eng.stage_frames([b.ptr for b in bufs], [h for h, _ in sizes], [w for _, w in sizes], fmt)
            eng.sync()
            got = eng.read(0, len(sizes))
            for s in range(len(sizes)):
                np.testing.assert_array_equal(got[s], want[s])
                if task == "detect":
                    g2 = post.letterbox_geom(S, S, *sizes[s])
                    scale, top, left = eng.slot_geom(s)
                    assert (np.float32(scale), top, left) == g2[:3]
            pinned += bufs
    with pytest.raises(RuntimeError):
        eng.stage_frames([pinned[0].ptr], [333], [517], 7)      # unknown layout
    for b in pinned:
        b.free()
    eng.close()
