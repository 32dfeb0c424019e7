"""GPU per-op parity through the C ABI (needs an MI355X).

The isolated-kernel check of the reference (its `dump` mode, engine/engine.cu:1843-1888,
and test/compare.py): every op runs alone on the GPU with inputs that equal the oracle's
fp16-rounded activations (each GPU output is overwritten with the oracle's before the
next op), and the op's output must satisfy max|gpu - ref| / max|ref| <= 1.5 %.
"""
import numpy as np
import pytest

import modelgen
import yolort
from oracle import graphfile, interp, post

TOL = 0.015   # per-op max relative deviation vs the fp32 oracle (BASELINE parity bar)

pytestmark = pytest.mark.gpu


def _resync_run(model_dir, x, B=1):
    """Runs every op of the unfused graph on the GPU with oracle resync; returns
    [(k, kind, rel)] and the engine (for post-processing checks)."""
    g = graphfile.load(model_dir)
    ref = interp.Interp(g, B, round_fp16=True)
    ref.set_input(x)
    eng = yolort.Engine(model_dir, B, yolort.YOLO_NOFUSE | yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.write(0, ref.view(0))
    assert eng.num_ops == len(g.ops)
    rels = []
    for k, op in enumerate(g.ops):
        t = ref.run_op(op)
        eng.run_op(k, B)
        if t is None:
            continue
        want = ref.view(t)
        got = eng.read(t, B).astype(np.float32)
        rel = post.rel_err(got, want)
        rels.append((k, op.kind, rel))
        eng.write(t, want)
    return rels, eng, ref


def _print_worst(rels, n=5):
    worst = sorted(rels, key=lambda r: -r[2])[:n]
    print("worst ops:", ", ".join(f"op{k:03d} {kind} {rel:.2e}" for k, kind, rel in worst), flush=True)


def test_yolo11n_ops_resync(models):
    d = models("yolo11", "n")
    img = modelgen.synth_frame(810, 1080, 20, 1)
    x = post.letterbox(img, 640, 640)[None]
    rels, eng, ref = _resync_run(d, x)
    _print_worst(rels)
    assert len(rels) == 109          # the reference's dumped-op count for yolo11n (README.md:191)
    bad = [r for r in rels if not r[2] <= TOL]
    assert not bad, bad
    # decode + NMS on identical head tensors: exact same survivors, order and classes
    eng.run_post(1)
    want = post.detect([(b[0], c[0], None, s) for b, c, _, s in ref.heads_in], 80)
    got = eng.get(0)
    assert eng.raw_count(0) == want["n_raw"]
    assert len(got) == len(want["score"]), (len(got), len(want["score"]))
    np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
    np.testing.assert_allclose(got[:, 4], want["score"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(got[:, :4], want["box"], rtol=0, atol=2e-3)
    eng.close()


def test_yolo11n_seg_ops_resync(models):
    d = models("yolo11", "n", "segment")
    img = modelgen.synth_polygons(640, 640, 30, 4)
    x = post.letterbox(img, 640, 640)[None]
    rels, eng, ref = _resync_run(d, x)
    _print_worst(rels)
    bad = [r for r in rels if not r[2] <= TOL]
    assert not bad, bad
    eng.run_post(1)
    heads = [(b[0], c[0], m[0], s) for b, c, m, s in ref.heads_in]
    want = post.detect(heads, 80)
    got = eng.get(0)
    assert len(got) == len(want["score"])
    np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
    g = graphfile.load(d)
    proto_t = [op.a for op in g.ops if op.kind == "MASKS"][0]
    proto = ref.view(proto_t)[0]
    wm = post.masks(proto, want["coef"], want["box"], 640, 640)
    agree = []
    for i in range(len(got)):
        gm = eng.get_mask(0, i)
        inter = np.logical_and(gm, wm[i]).sum()
        union = np.logical_or(gm, wm[i]).sum()
        agree.append(1.0 if union == 0 else inter / union)
    print("mask IoU min %.4f" % (min(agree) if agree else 1.0), flush=True)
    assert not agree or min(agree) >= 0.99
    eng.close()


@pytest.mark.parametrize("nm", [16, 32, 64])
def test_seg_masks_nm(tmp_path, nm):
    """Mask assembly with 16 mask coefficients (the per-lane kernel) and 32 or 64 (the MFMA
    kernel, one or two 32-channel steps): on resynced heads, decode + NMS exactly the oracle's,
    then every survivor's mask at IoU >= 0.99 against the oracle's masks."""
    d = str(tmp_path / f"seg{nm}")
    modelgen.build_model("yolo11", "n", "segment", 80, 640, 0, -8.0, nm=nm).graph.write(d, "segment", 80, 640)
    img = modelgen.synth_polygons(640, 640, 30, 4)
    x = post.letterbox(img, 640, 640)[None]
    rels, eng, ref = _resync_run(d, x)
    assert not [r for r in rels if not r[2] <= TOL]
    eng.run_post(1)
    want = post.detect([(b[0], c[0], m[0], s) for b, c, m, s in ref.heads_in], 80)
    got = eng.get(0)
    assert len(got) == len(want["score"]) and len(got) > 0
    np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
    g = graphfile.load(d)
    proto = ref.view([op.a for op in g.ops if op.kind == "MASKS"][0])[0]
    assert proto.shape[-1] == nm
    wm = post.masks(proto, want["coef"], want["box"], 640, 640)
    ious = []
    for i in range(len(got)):
        gm = eng.get_mask(0, i)
        union = np.logical_or(gm, wm[i]).sum()
        ious.append(1.0 if union == 0 else np.logical_and(gm, wm[i]).sum() / union)
    print(f"nm {nm}: {len(got)} survivors, mask IoU min {min(ious):.4f}", flush=True)
    assert min(ious) >= 0.99
    eng.close()


@pytest.mark.parametrize("B", [1, 32])
@pytest.mark.parametrize("shape", [
    (80, 80, 256, 256, 3, 1), (80, 80, 256, 512, 3, 2), (40, 40, 512, 256, 1, 1),
    (20, 20, 512, 512, 3, 1), (20, 20, 1024, 512, 1, 1), (40, 40, 96, 192, 3, 1)])
def test_conv_sweep(tmp_path, shape, B):
    """Config 1: the isolated conv sweep, bias + SiLU epilogue, every tile config; the last
    shape is N = 192 exactly with Cin not a multiple of 64 (tap-straddling K stages)."""
    H, W, cin, cout, k, s = shape
    d = str(tmp_path / "conv")
    modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=7)
    g = graphfile.load(d)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((B, H, W, cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.write(0, x)
    # the oracle on two images (images are independent; first and last cover the batch)
    pick = [0, B - 1] if B > 1 else [0]
    ref = interp.Interp(g, len(pick))
    ref.set_input(x[pick].astype(np.float32))
    ref.run_op(g.ops[0])
    want = ref.view(g.ops[0].out)
    for cfg in range(len(yolort.tile_configs())):
        try:
            eng.set_op_config(0, cfg)
        except ValueError:
            continue
        eng.run_op(0, B)
        got = eng.read(g.ops[0].out, B)[pick].astype(np.float32)
        rel = post.rel_err(got, want)
        print(f"shape {shape} B={B} cfg {cfg}: rel {rel:.2e}", flush=True)
        assert rel <= TOL, (cfg, rel)
    eng.close()


@pytest.mark.parametrize("shape,B,cfg", [((80, 80, 256, 256, 3, 1), 32, 31), ((80, 80, 96, 192, 3, 1), 32, 31),
                                         ((80, 80, 512, 256, 1, 1), 32, 2), ((80, 80, 768, 768, 3, 2), 16, 5)])
def test_conv_tail_retile(tmp_path, shape, B, cfg):
    """Tail retile (the rows past the last whole chip wave under a smaller tile of the same
    BK, in a second launch): for every tail config that applies, the output is bit-identical
    to the plain tile config, which is itself within the oracle tolerance.  Covers the
    channel-block walk (3x3 stride 1 and 2), the per-lane walk (Cin 96 with BK 64) and 1x1."""
    H, W, cin, cout, k, s = shape
    d = str(tmp_path / "tail")
    modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=5)
    g = graphfile.load(d)
    x = np.random.default_rng(9).standard_normal((B, H, W, cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.write(0, x)
    eng.set_op_config(0, cfg)
    assert eng.op_tail(0) == -1
    eng.run_op(0, B)
    plain = eng.read(g.ops[0].out, B)
    pick = [0, B - 1]
    ref = interp.Interp(g, len(pick))
    ref.set_input(x[pick].astype(np.float32))
    ref.run_op(g.ops[0])
    rel = post.rel_err(plain[pick].astype(np.float32), ref.view(g.ops[0].out))
    assert rel <= TOL, rel
    tried = []
    for tail in range(len(yolort.tile_configs())):
        try:
            eng.set_op_tail(0, tail)
        except ValueError:
            continue
        assert eng.op_tail(0) == tail
        eng.write(g.ops[0].out, np.zeros_like(plain))
        eng.run_op(0, B)
        got = eng.read(g.ops[0].out, B)
        diff = int(np.count_nonzero(got.view(np.uint16) != plain.view(np.uint16)))
        print(f"shape {shape} B={B} cfg {cfg} tail {tail}: {diff} differing values", flush=True)
        assert diff == 0, (tail, diff)
        tried.append(tail)
    assert tried, "no tail config applies"
    eng.set_op_tail(0, -1)
    assert eng.op_tail(0) == -1
    eng.close()


def test_conv_tail_rejects(tmp_path):
    """The tail override is refused for tiles with another BK or no smaller area, for special
    kernels, split ops and non-GEMM ops."""
    d = str(tmp_path / "tr")
    modelgen.write_single_conv(d, 80, 80, 256, 256, 3, 1, seed=5)
    eng = yolort.Engine(d, 32, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.set_op_config(0, 31)                      # 256x256, BK 64
    for tail in (2, 5, 13, 31, 20, -5 + 100):     # BK 32, BK 32, BK 128, itself, same area, out of range
        with pytest.raises(ValueError):
            eng.set_op_tail(0, tail)
    eng.set_op_tail(0, 6)                         # 128x128, BK 64
    eng.set_op_split(0, 2)                        # a split clears the tail
    assert eng.op_tail(0) == -1
    with pytest.raises(ValueError):
        eng.set_op_tail(0, 6)
    eng.close()


@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("shape", [(20, 20, 8, 16, 3, 1), (13, 17, 24, 40, 3, 2), (7, 9, 16, 8, 1, 1),
                                   (33, 31, 64, 24, 3, 1), (16, 16, 32, 32, 3, 1)])
def test_conv_edge_shapes(tmp_path, shape, res):
    """Ragged M/N/K edges (M not a tile multiple, Cin 8/24, Cout 8/24/40) and residuals."""
    H, W, cin, cout, k, s = shape
    if res and (s != 1 or cin != cout):
        pytest.skip("residual needs matching shapes")
    d = str(tmp_path / "edge")
    modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=3, residual=res)
    g = graphfile.load(d)
    B = 3
    x = np.random.default_rng(5).standard_normal((B, H, W, cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    assert eng.num_ops == len(ops)
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    for op in ops:
        ref.run_op(op)
    want = ref.view(ops[0].out)
    for cfg in range(len(yolort.tile_configs())):
        try:
            eng.set_op_config(0, cfg)
        except ValueError:
            continue
        eng.write(0, x)
        eng.run_op(0, B)
        got = eng.read(ops[0].out, B).astype(np.float32)
        rel = post.rel_err(got, want)
        assert rel <= TOL, (shape, cfg, rel)
    eng.close()


@pytest.mark.parametrize("H,W,heads,B", [(20, 20, 2, 2), (7, 7, 3, 2), (20, 20, 6, 2), (32, 32, 2, 2),
                                         (5, 13, 1, 2), (20, 20, 6, 8), (20, 20, 6, 24), (7, 7, 3, 40)])
def test_attention_op(tmp_path, H, W, heads, B):
    """ATTN alone: N = 400 (640 input), N = 49 / 65 (ragged key chunks, key parts with no
    chunk), N = 1024 (streamed keys); grids of up to 128 / 512 / more blocks (4, 2 and 1 key
    parts per query group)."""
    kd, hd = 32, 64
    d = str(tmp_path / "attn")
    modelgen.write_attention(d, H, W, heads, kd, hd)
    g = graphfile.load(d)
    x = (np.random.default_rng(H * W).standard_normal((B, H, W, heads * (2 * kd + hd)), dtype=np.float32)
         * 2).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    op = g.ops[0]
    eng.write(op.a, x)
    eng.run_op(0, B)
    got = eng.read(op.out, B).astype(np.float32)
    want = interp.attention(x.astype(np.float32), heads, kd, hd)
    rel = post.rel_err(got, want)
    print(f"attention {H}x{W} heads={heads} B={B}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    eng.close()


@pytest.mark.parametrize("scale,B,imgsz", [("n", 1, 640), ("n", 3, 640), ("n", 32, 640), ("x", 16, 640),
                                           ("x", 24, 320)])
def test_sppf_pool_chain(models, scale, B, imgsz):
    """The fused SPPF pool chain (one launch for three MAXPOOL5) is bit-exact against the
    oracle's mp5, mp5(mp5), mp5(mp5(mp5)) on random activations, and the standalone
    MAXPOOL5 of a chain follower (what the per-op harness runs) is exact too.  The cases
    cover one 8-channel group per block (yolo11n b1, b3), two (yolo11n b32, yolo11x b16 at
    20x20) and four (yolo11x b24 at 320: a 10x10 plane)."""
    d = models("yolo11", scale, "detect", imgsz=imgsz)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    kinds = [eng.op_info(k) for k in range(eng.num_ops)]
    head = next(k for k in range(len(kinds) - 2)
                if all(kinds[k + i]["kind"] == "MAXPOOL5" for i in range(3)))
    x = (np.random.default_rng(B).standard_normal((B,) + eng.tensor_shape(kinds[head]["a"]),
                                                  dtype=np.float32) * 3).astype(np.float16)
    eng.write(kinds[head]["a"], x)
    eng.run_op(head, B)
    want = x.astype(np.float32)
    for i in range(3):
        want = interp.maxpool5(want)
        got = eng.read(kinds[head + i]["out"], B).astype(np.float32)
        assert np.array_equal(got, want), (i, np.abs(got - want).max())
    # follower alone: mp5 of the chain head's output
    eng.run_op(head + 1, B)
    got = eng.read(kinds[head + 1]["out"], B).astype(np.float32)
    assert np.array_equal(got, interp.maxpool5(eng.read(kinds[head]["out"], B).astype(np.float32)))
    eng.close()


@pytest.mark.parametrize("shape", [(20, 20, 512, 256, 3, 1), (40, 40, 128, 64, 3, 2),
                                   (20, 20, 1024, 512, 1, 1), (13, 17, 96, 40, 3, 1)])
def test_conv_split_k(tmp_path, shape):
    """Split-K: every split count a tile admits gives the oracle's result within the per-op
    bar, is bit-identical across launches (fixed reduction order, counters re-armed by the
    kernel) and across the tile's first and second use of the workspace."""
    H, W, cin, cout, k, s = shape
    d = str(tmp_path / "splitk")
    modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=5)
    g = graphfile.load(d)
    B = 1
    x = np.random.default_rng(7).standard_normal((B, H, W, cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.write(0, x)
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    ref.run_op(g.ops[0])
    want = ref.view(g.ops[0].out)
    tried = 0
    for cfg in (13, 16, 17, 12, 7):
        eng.set_op_config(0, cfg)
        eng.run_op(0, B)
        base = eng.read(g.ops[0].out, B)
        for S in (2, 3, 4, 8, 16):
            try:
                eng.set_op_split(0, S)
            except ValueError:
                continue            # tile/K combination leaves a split empty
            assert eng.op_split(0) == S
            eng.run_op(0, B)
            got1 = eng.read(g.ops[0].out, B)
            eng.run_op(0, B)
            got2 = eng.read(g.ops[0].out, B)
            assert np.array_equal(got1, got2), (cfg, S)
            rel = post.rel_err(got1.astype(np.float32), want)
            print(f"shape {shape} cfg {cfg} S {S}: rel {rel:.2e}", flush=True)
            assert rel <= TOL, (cfg, S, rel)
            # against the unsplit launch: only fp32 summation order differs
            assert post.rel_err(got1.astype(np.float32), base.astype(np.float32)) <= 2e-3
            tried += 1
        eng.set_op_config(0, cfg)   # back to split 1 for the next tile
    assert tried >= 4
    eng.close()


def test_conv_tail_split(tmp_path):
    """Tail split (negative split factor): the tiles of whole chip waves run unsplit and only
    the part-empty last wave is split, at the max batch (4) and at smaller batches that reuse
    the same setting (1 and 3: grids of less than a wave).  Every result is within the
    per-op bar of the oracle, bit-identical across launches, and within fp32 summation-order
    noise of the unsplit launch."""
    H, W, cin, cout, k, s = 80, 80, 64, 64, 3, 1
    d = str(tmp_path / "tail")
    modelgen.write_single_conv(d, H, W, cin, cout, k, s, seed=9)
    g = graphfile.load(d)
    Bmax = 4
    x = np.random.default_rng(3).standard_normal((Bmax, H, W, cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, Bmax, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.write(0, x)
    ref = interp.Interp(g, Bmax)
    ref.set_input(x.astype(np.float32))
    ref.run_op(g.ops[0])
    want = ref.view(g.ops[0].out)
    tried = 0
    for cfg in (17, 12, 7, 5, 16):
        for B in (Bmax, 1, 3):
            eng.set_op_config(0, cfg)
            eng.run_op(0, B)
            base = eng.read(g.ops[0].out, B)
            for S in (-2, -3, -5, -8):
                try:
                    eng.set_op_split(0, S)
                except ValueError:
                    continue
                assert eng.op_split(0) == S
                eng.run_op(0, B)
                got1 = eng.read(g.ops[0].out, B)
                eng.run_op(0, B)
                got2 = eng.read(g.ops[0].out, B)
                assert np.array_equal(got1, got2), (cfg, B, S)
                rel = post.rel_err(got1.astype(np.float32), want[:B])
                print(f"cfg {cfg} B {B} S {S}: rel {rel:.2e}", flush=True)
                assert rel <= TOL, (cfg, B, S, rel)
                assert post.rel_err(got1.astype(np.float32), base.astype(np.float32)) <= 2e-3
                tried += 1
    assert tried >= 20
    eng.close()


@pytest.mark.parametrize("HW", [(37, 48), (37, 45)])
@pytest.mark.parametrize("cout", [16, 32, 48, 96, 160, 256, 24])
def test_conv_first(tmp_path, cout, HW):
    """The stem conv (Cin 3, 3x3 s2): the MFMA kernel (Cout % 16 == 0 and input rows of whole
    16-byte vectors, W % 8 == 0; paired 16-byte stores when Cout % 32 == 0) and the direct
    kernel (Cout 24, or W = 45) against the oracle, with ragged image edges and a batch."""
    (H, W), B = HW, 2
    d = str(tmp_path / "stem")
    modelgen.write_single_conv(d, H, W, 3, cout, 3, 2, seed=cout)
    g = graphfile.load(d)
    x = np.random.default_rng(cout).uniform(0, 1, (B, H, W, 3)).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.write(0, x)
    eng.run_op(0, B)
    got = eng.read(g.ops[0].out, B).astype(np.float32)
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    ref.run_op(g.ops[0])
    rel = post.rel_err(got, ref.view(g.ops[0].out))
    print(f"stem Cout {cout}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    eng.close()


@pytest.mark.parametrize("H,W,C,s,B,res", [(80, 80, 384, 1, 16, False), (41, 43, 256, 1, 16, True),
                                            (81, 79, 128, 2, 32, False), (20, 21, 64, 1, 2, True),
                                            (13, 11, 32, 2, 3, False)])
def test_dwconv(tmp_path, H, W, C, s, B, res):
    """Depthwise 3x3 (bias, SiLU, optional residual): the 4-pixels-per-thread kernel (large
    launches: stride 1 and 2, widths not a multiple of 4) and the one-pixel kernel (small
    launches) against the oracle on the first and last image of the batch."""
    d = str(tmp_path / "dw")
    modelgen.write_single_conv(d, H, W, C, C, 3, s, seed=C + s, dw=True, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(C).standard_normal((B, H, W, C), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    assert eng.num_ops == len(ops) == 1
    eng.write(0, x)
    eng.run_op(0, B)
    pick = [0, B - 1]
    got = eng.read(ops[0].out, B)[pick].astype(np.float32)
    ref = interp.Interp(g, len(pick))
    ref.set_input(x[pick].astype(np.float32))
    for op in ops:
        ref.run_op(op)
    rel = post.rel_err(got, ref.view(ops[0].out))
    print(f"dwconv {H}x{W}x{C} s{s} b{B} res={res}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    eng.close()


@pytest.mark.parametrize("H,W,C,s,B,res", [(41, 43, 256, 1, 16, True), (80, 80, 384, 1, 16, False),
                                            (81, 79, 128, 2, 32, False)])
def test_dwconv_kernels_bit_identical(tmp_path, H, W, C, s, B, res):
    """The depthwise kernels a launch size selects (four pixels per thread for large launches,
    one pixel per thread for small ones) give the same bits: images of a large batch against
    batch-1 runs of each image, so a frame's result does not depend on its batch."""
    d = str(tmp_path / "dwb")
    modelgen.write_single_conv(d, H, W, C, C, 3, s, seed=C + 7 * s, dw=True, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(C + s).standard_normal((B, H, W, C), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    out = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)][0].out
    eng.write(0, x)
    eng.run_op(0, B)
    big = eng.read(out, B)
    for i in (0, B // 2, B - 1):
        eng.write(0, x[i:i + 1])
        eng.run_op(0, 1)
        one = eng.read(out, 1)[0]
        diff = int(np.count_nonzero(one.view(np.uint16) != big[i].view(np.uint16)))
        print(f"dw {H}x{W}x{C} s{s}: image {i} of {B} vs alone: {diff} differing values", flush=True)
        assert diff == 0
    eng.close()


@pytest.mark.parametrize("H,W,Cin,Cout,B,res", [(160, 160, 48, 48, 2, False), (37, 45, 32, 32, 3, True),
                                                (20, 21, 64, 64, 2, True), (8, 8, 8, 16, 1, False),
                                                (33, 17, 24, 48, 2, False), (40, 40, 64, 16, 2, False)])
def test_conv_halo(tmp_path, H, W, Cin, Cout, B, res):
    """The LDS-halo 3x3 kernel (op config CFG_HALO): ragged 4x16 output tiles, channel counts
    from 8 to 64 (one or two 32-channel chunks, 1-4 output fragments), bias + SiLU and the
    fused residual, against the oracle."""
    d = str(tmp_path / "halo")
    modelgen.write_single_conv(d, H, W, Cin, Cout, 3, 1, seed=Cin + Cout, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(Cin).standard_normal((B, H, W, Cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    assert eng.num_ops == len(ops) == 1
    eng.set_op_config(0, yolort.CFG_HALO)
    assert eng.op_config(0) == yolort.CFG_HALO
    eng.write(0, x)
    eng.run_op(0, B)
    got = eng.read(ops[0].out, B).astype(np.float32)
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    ref.run_op(ops[0])
    rel = post.rel_err(got, ref.view(ops[0].out))
    print(f"halo {H}x{W} {Cin}->{Cout} b{B} res={res}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    eng.close()


def test_conv_halo_rejects(tmp_path):
    """The halo config is refused where the kernel does not apply (stride 2, 1x1, over 64
    channels, Cout not a multiple of 16)."""
    for i, (cin, cout, k, s) in enumerate([(32, 32, 3, 2), (32, 32, 1, 1), (96, 32, 3, 1), (32, 24, 3, 1)]):
        d = str(tmp_path / f"r{i}")
        modelgen.write_single_conv(d, 16, 16, cin, cout, k, s, seed=1)
        eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
        with pytest.raises(ValueError):
            eng.set_op_config(0, yolort.CFG_HALO)
        eng.close()


@pytest.mark.parametrize("H,W,Cin,Cout,B,res,act", [
    (80, 80, 64, 64, 2, True, modelgen.ACT_SILU),      # one chunk pair, two 16-ch fragments x 4
    (40, 40, 384, 128, 1, False, modelgen.ACT_SILU),   # 12 chunks: two slices of 64
    (20, 20, 256, 256, 2, True, modelgen.ACT_SILU),    # 8 chunks, two full slices of 128
    (37, 45, 48, 96, 3, False, modelgen.ACT_SILU),     # Cin padded to 64, ragged M = 4995
    (7, 9, 8, 16, 1, False, modelgen.ACT_NONE),        # smallest: one fragment, 63 pixels
    (33, 17, 320, 48, 2, False, modelgen.ACT_SILU),    # Cin 320 in 12 chunks, three fragments
    (20, 20, 192, 144, 1, False, modelgen.ACT_NONE)])  # second slice only partly live
def test_conv_1x1_resident(tmp_path, H, W, Cin, Cout, B, res, act):
    """The weights-resident 1x1 kernel (op config CFG_1X1): input channels from 8 to 384
    (padded to 32-channel chunks), output slices of up to 128 channels with a partly live
    last slice, ragged pixel counts, bias with and without SiLU and the fused residual,
    against the oracle."""
    d = str(tmp_path / "p1")
    modelgen.write_single_conv(d, H, W, Cin, Cout, 1, 1, act=act, seed=Cin + Cout, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(Cin).standard_normal((B, H, W, Cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    assert eng.num_ops == len(ops) == 1
    eng.set_op_config(0, yolort.CFG_1X1)
    assert eng.op_config(0) == yolort.CFG_1X1
    eng.write(0, x)
    eng.run_op(0, B)
    got = eng.read(ops[0].out, B).astype(np.float32)
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    ref.run_op(ops[0])
    rel = post.rel_err(got, ref.view(ops[0].out))
    print(f"1x1 {H}x{W} {Cin}->{Cout} b{B} res={res} act={act}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    # the two-groups-in-flight variant (16-byte stores for even fragment counts) runs the
    # same MFMA chain per output: identical bits
    eng.set_op_config(0, yolort.CFG_1X1S)
    assert eng.op_config(0) == yolort.CFG_1X1S
    eng.write(ops[0].out, np.zeros((B,) + eng.tensor_shape(ops[0].out), np.float16))
    eng.run_op(0, B)
    np.testing.assert_array_equal(eng.read(ops[0].out, B).view(np.uint16), got.astype(np.float16).view(np.uint16))
    eng.close()


def test_conv_1x1_resident_rejects(tmp_path):
    """The resident-1x1 config is refused where the kernel does not apply (3x3, stride 2,
    over 384 input channels, Cout not a multiple of 16)."""
    for i, (cin, cout, k, s) in enumerate([(32, 32, 3, 1), (32, 32, 1, 2), (512, 64, 1, 1), (32, 24, 1, 1)]):
        d = str(tmp_path / f"r{i}")
        modelgen.write_single_conv(d, 16, 16, cin, cout, k, s, seed=1)
        eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
        for cfg in (yolort.CFG_1X1, yolort.CFG_1X1S):
            with pytest.raises(ValueError):
                eng.set_op_config(0, cfg)
        eng.close()


@pytest.mark.parametrize("v", yolort.TAP_3X3)
@pytest.mark.parametrize("H,W,Cin,Cout,B,res", [
    (40, 40, 192, 192, 2, True),     # six 32-channel stages, two or more channel tiles
    (80, 80, 96, 96, 1, False),      # the yolo11x 80x80 bottleneck shape
    (33, 45, 48, 48, 2, True),       # ragged tiles on both axes, a half-live second stage
    (20, 20, 256, 256, 1, False),    # eight stages
    (17, 23, 40, 112, 2, False)])    # Cin 40 (second stage 8 channels), partly live channel tile
def test_conv_tap(tmp_path, v, H, W, Cin, Cout, B, res):
    """The halo-staged 3x3 GEMM (op configs CFG_TAP + v, every tile variant): one LDS stage per
    32-channel block for all 9 taps, tap groups summed through LDS, ragged tiles, channel
    counts that leave part of a stage or a channel tile empty, bias + SiLU and the fused
    residual, against the oracle."""
    d = str(tmp_path / "tap")
    modelgen.write_single_conv(d, H, W, Cin, Cout, 3, 1, seed=Cin + Cout, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(Cin).standard_normal((B, H, W, Cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    assert eng.num_ops == len(ops) == 1
    _check_tap(eng, g, ops, x, v, B, Cout, f"tap v{v} {H}x{W} {Cin}->{Cout} b{B} res={res}")


def _check_tap(eng, g, ops, x, v, B, cout, label):
    try:
        eng.set_op_config(0, yolort.CFG_TAP + v)
    except ValueError:
        # refused only where the variant's channel tile is more than half empty
        assert cout <= yolort.TAP_BN[v] // 2
        eng.close()
        return
    assert eng.op_config(0) == yolort.CFG_TAP + v
    eng.write(0, x)
    eng.run_op(0, B)
    got = eng.read(ops[0].out, B).astype(np.float32)
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    ref.run_op(ops[0])
    rel = post.rel_err(got, ref.view(ops[0].out))
    print(f"{label}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    eng.close()


@pytest.mark.parametrize("v", yolort.TAP_1X1)
@pytest.mark.parametrize("H,W,Cin,Cout,B,res,act", [
    (40, 40, 384, 384, 2, True, modelgen.ACT_SILU),     # 12 stages, one or more channel tiles
    (80, 80, 192, 96, 1, False, modelgen.ACT_SILU),     # channel tile partly live (BN 128..384)
    (33, 45, 96, 144, 2, False, modelgen.ACT_NONE),     # ragged last pixel tile, partly live channel tile
    (20, 20, 1536, 768, 1, False, modelgen.ACT_SILU),   # 48 stages, several channel tiles
    (17, 23, 40, 112, 2, False, modelgen.ACT_SILU)])    # Cin 40: a half-empty second stage
def test_conv_tap_1x1(tmp_path, v, H, W, Cin, Cout, B, res, act):
    """The streaming kernel's 1x1 variants (op configs CFG_TAP + v): the batch's pixels tiled as
    one row, persistent blocks running the stages of all their tiles as one ring sequence, bias
    with and without SiLU and the fused residual, against the oracle."""
    d = str(tmp_path / "tap1")
    modelgen.write_single_conv(d, H, W, Cin, Cout, 1, 1, act=act, seed=Cin + Cout, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(Cin).standard_normal((B, H, W, Cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    assert eng.num_ops == len(ops) == 1
    _check_tap(eng, g, ops, x, v, B, Cout, f"tap1x1 v{v} {H}x{W} {Cin}->{Cout} b{B} res={res}")


@pytest.mark.parametrize("v", range(yolort.NUM_TAPWS_TILES))
@pytest.mark.parametrize("H,W,Cin,Cout,B,res", [
    (40, 40, 192, 192, 2, True),     # six stages, several channel tiles, residual
    (80, 80, 96, 96, 1, False),      # the yolo11x 80x80 bottleneck shape
    (33, 45, 48, 48, 3, True),       # ragged tiles on both axes, a half-live second stage
    (20, 20, 256, 256, 1, False),    # eight stages: every ring slot refilled several times
    (17, 23, 40, 112, 2, False)])    # Cin 40, a partly live channel tile
def test_conv_tapws(tmp_path, v, H, W, Cin, Cout, B, res):
    """The wave-specialised halo-staged 3x3 conv (op configs CFG_TAPWS + v): producer waves
    fill the LDS ring, consumer waves run the MFMAs, slots handed over through LDS counters.
    Against the oracle; no bounded wait expired; a second launch gives the same bits; and
    every image equals its own batch-1 run (results depend on neither timing nor batch)."""
    d = str(tmp_path / "tapws")
    modelgen.write_single_conv(d, H, W, Cin, Cout, 3, 1, seed=Cin + Cout, residual=res)
    g = graphfile.load(d)
    x = np.random.default_rng(Cin).standard_normal((B, H, W, Cin), dtype=np.float32).astype(np.float16)
    eng = yolort.Engine(d, B, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    ops = [graphfile.Op(**vars(o)) for o in graphfile.fuse_adds(g.ops)]
    try:
        eng.set_op_config(0, yolort.CFG_TAPWS + v)
    except ValueError:
        assert Cout <= yolort.TAPWS_BN[v] // 2
        eng.close()
        return
    before = eng.spin_failures()
    eng.write(0, x)
    eng.run_op(0, B)
    got = eng.read(ops[0].out, B)
    eng.run_op(0, B)
    again = eng.read(ops[0].out, B)
    one = []
    for i in range(B):
        eng.write(0, x[i:i + 1])
        eng.run_op(0, 1)
        one.append(eng.read(ops[0].out, 1)[0])
    assert eng.spin_failures() == before == 0
    np.testing.assert_array_equal(again.view(np.uint16), got.view(np.uint16))
    np.testing.assert_array_equal(np.stack(one).view(np.uint16), got.view(np.uint16))
    ref = interp.Interp(g, B)
    ref.set_input(x.astype(np.float32))
    ref.run_op(ops[0])
    rel = post.rel_err(got.astype(np.float32), ref.view(ops[0].out))
    print(f"tapws v{v} {H}x{W} {Cin}->{Cout} b{B} res={res}: rel {rel:.2e}", flush=True)
    assert rel <= TOL
    eng.close()


def test_conv_tapws_rejects(tmp_path):
    """The wave-specialised configs are refused for stride 2, 1x1 convs, Cout not a multiple
    of 16, and past the last variant."""
    for i, (cin, cout, k, s) in enumerate([(32, 32, 3, 2), (32, 32, 1, 1), (32, 24, 3, 1)]):
        d = str(tmp_path / f"r{i}")
        modelgen.write_single_conv(d, 16, 16, cin, cout, k, s, seed=1)
        eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
        for v in range(yolort.NUM_TAPWS_TILES):
            with pytest.raises(ValueError):
                eng.set_op_config(0, yolort.CFG_TAPWS + v)
        eng.close()
    d = str(tmp_path / "ok")
    modelgen.write_single_conv(d, 16, 16, 64, 64, 3, 1, seed=1)
    eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.set_op_config(0, yolort.CFG_TAPWS)
    with pytest.raises(ValueError):
        eng.set_op_config(0, yolort.CFG_TAPWS + yolort.NUM_TAPWS_TILES)
    eng.close()


def test_conv_tap_rejects(tmp_path):
    """The streaming configs are refused where the kernel does not apply (stride 2, the
    other kernel size, Cout not a multiple of 16) and past the last variant."""
    cases = [(32, 32, 3, 2, yolort.TAP_3X3), (32, 32, 1, 1, yolort.TAP_3X3), (32, 24, 3, 1, yolort.TAP_3X3),
             (256, 256, 1, 2, yolort.TAP_1X1), (256, 256, 3, 1, yolort.TAP_1X1), (256, 248, 1, 1, yolort.TAP_1X1)]
    for i, (cin, cout, k, s, variants) in enumerate(cases):
        d = str(tmp_path / f"r{i}")
        modelgen.write_single_conv(d, 16, 16, cin, cout, k, s, seed=1)
        eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
        for v in variants:
            with pytest.raises(ValueError):
                eng.set_op_config(0, yolort.CFG_TAP + v)
        eng.close()
    d = str(tmp_path / "ok")
    modelgen.write_single_conv(d, 16, 16, 64, 64, 3, 1, seed=1)
    eng = yolort.Engine(d, 1, yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH)
    eng.set_op_config(0, yolort.CFG_TAP)
    with pytest.raises(ValueError):
        eng.set_op_config(0, yolort.CFG_TAP + yolort.NUM_TAP_TILES)
    eng.close()


@pytest.mark.parametrize("nmsflag", [0, yolort.YOLO_NMS_BLOCK], ids=["multi", "block"])
@pytest.mark.parametrize("ncls", [1, 12, 20, 80])
def test_nms_paths_crafted_heads(models, ncls, nmsflag):
    """Decode + NMS on crafted head tensors that drive each NMS path: one class (over 2048
    candidates: threshold selection, then one class of 32 chunks whose mask columns are too
    large for LDS), 12 classes (~170 per class), 20 classes (50-120 per class: two chunks)
    and 80 classes (one chunk per class); through the multi-block pipeline (the default)
    and the one-block kernel (YOLO_NMS_BLOCK).  Exact: same raw count, survivors, order and
    classes as the oracle."""
    d = models("yolo11", "n")
    g = graphfile.load(d)
    eng = yolort.Engine(d, 1, yolort.YOLO_NOFUSE | yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH | nmsflag)
    rng = np.random.default_rng(ncls)
    dec = [(k, op) for k, op in enumerate(g.ops) if op.kind == "DECODE"]
    heads = []
    for _, op in dec:
        H, W, C = eng.tensor_shape(op.b)
        cls = np.full((1, H, W, C), -20.0, np.float32)
        pick = rng.integers(0, ncls, (H, W))
        cls[0, np.arange(H)[:, None], np.arange(W)[None, :], pick] = rng.uniform(-2.5, 4.0, (H, W))
        box = rng.normal(0.0, 1.5, (1, H, W, 64)).astype(np.float32)
        box[..., 2::16] += 2.0                 # mass near bin 2: boxes a few strides wide
        eng.write(op.b, cls)
        eng.write(op.a, box)
        heads.append((box[0].astype(np.float16).astype(np.float32),
                      cls[0].astype(np.float16).astype(np.float32), None, op.stride))
    for conf, iou in ((0.25, 0.45), (0.95, 0.3)):
        eng.set_thresholds(conf, iou, 300)
        eng.run_op(dec[-1][0], 1)
        eng.run_post(1)
        want = post.detect(heads, 80, conf, iou)
        got = eng.get(0)
        print(f"{ncls} classes conf {conf}: raw {eng.raw_count(0)} / {want['n_raw']}, kept {len(got)} / "
              f"{len(want['score'])}", flush=True)
        assert eng.raw_count(0) == want["n_raw"]
        assert len(got) == len(want["score"])
        np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
        np.testing.assert_allclose(got[:, 4], want["score"], rtol=0, atol=2e-6)
        np.testing.assert_allclose(got[:, :4], want["box"], rtol=0, atol=2e-3)
    eng.close()


@pytest.mark.parametrize("nmsflag", [0, yolort.YOLO_NMS_BLOCK], ids=["multi", "block"])
def test_nms_tied_scores(models, nmsflag):
    """Every anchor of every level has the same score in one of two classes (8400 candidates,
    4200 per class): the NMS_CAP best are the lowest anchors, so the selection must narrow
    down to the anchor bits of the keys.  Exact against the oracle."""
    d = models("yolo11", "n")
    g = graphfile.load(d)
    eng = yolort.Engine(d, 1, yolort.YOLO_NOFUSE | yolort.YOLO_NOTUNE | yolort.YOLO_NOGRAPH | nmsflag)
    rng = np.random.default_rng(7)
    dec = [(k, op) for k, op in enumerate(g.ops) if op.kind == "DECODE"]
    heads = []
    for _, op in dec:
        H, W, C = eng.tensor_shape(op.b)
        cls = np.full((1, H, W, C), -20.0, np.float32)
        pick = rng.integers(0, 2, (H, W))
        cls[0, np.arange(H)[:, None], np.arange(W)[None, :], pick] = 1.5
        box = rng.normal(0.0, 1.5, (1, H, W, 64)).astype(np.float32)
        box[..., 2::16] += 2.0
        eng.write(op.b, cls)
        eng.write(op.a, box)
        heads.append((box[0].astype(np.float16).astype(np.float32),
                      cls[0].astype(np.float16).astype(np.float32), None, op.stride))
    eng.set_thresholds(0.25, 0.45, 300)
    eng.run_op(dec[-1][0], 1)
    eng.run_post(1)
    want = post.detect(heads, 80, 0.25, 0.45)
    got = eng.get(0)
    print(f"tied scores: raw {eng.raw_count(0)} / {want['n_raw']}, kept {len(got)} / {len(want['score'])}", flush=True)
    assert want["n_raw"] == 8400 and eng.raw_count(0) == want["n_raw"]
    assert len(got) == len(want["score"])
    np.testing.assert_array_equal(got[:, 5].astype(int), want["cls"])
    np.testing.assert_allclose(got[:, 4], want["score"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(got[:, :4], want["box"], rtol=0, atol=2e-3)
    eng.close()
