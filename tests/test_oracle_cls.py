"""Classify path on the CPU: the oracle's geometry, antialiased preprocess, top-k, GAP and
channel softmax pinned against independent definitions, the generator's yolo11-cls topology
against the reference's layer table (docs/specs/cls.md:29-55), and the host loader's
classify rules (engine/engine.cu:180-190)."""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from PIL import Image

import modelgen
import yolort
from oracle import graphfile, interp, post


@pytest.mark.parametrize("S,sh,sw", [(224, 810, 1080), (224, 1080, 1920), (224, 225, 224), (224, 227, 224),
                                     (224, 224, 229), (224, 224, 224), (256, 480, 640), (224, 1000, 333)])
def test_cls_geom(S, sh, sw):
    rh, rw, top, left = post.cls_geom(S, sh, sw)
    assert min(rh, rw) == S
    long_, short = max(sh, sw), min(sh, sw)
    assert max(rh, rw) == S * long_ // short            # int() truncation of the long edge
    assert top == round((rh - S) / 2) and left == round((rw - S) / 2)   # half to even
    assert 0 <= top <= rh - S and 0 <= left <= rw - S


def _triangle_resize_f64(src: np.ndarray, S: int) -> np.ndarray:
    """Antialiased bilinear resize + centre crop written from the filter's definition in
    float64 (separable normalised triangle weights with support max(scale, 1))."""
    sh, sw = src.shape[:2]
    rh, rw, top, left = post.cls_geom(S, sh, sw)

    def weights(n_out, n_in, off):
        f = n_in / (rh if n_in == sh else rw)
        r = max(f, 1.0)
        W = np.zeros((n_out, n_in))
        for o in range(n_out):
            c = (o + off + 0.5) * f
            a, b = max(0, int(c - r + 0.5)), min(n_in, int(c + r + 0.5))
            for i in range(a, b):
                W[o, i] = max(0.0, 1.0 - abs(i + 0.5 - c) / r)
            W[o] /= W[o].sum()
        return W

    Wy, Wx = weights(S, sh, top), weights(S, sw, left)
    t = np.tensordot(Wy, src.astype(np.float64), axes=(1, 0))          # [S, sw, 3]
    x = np.tensordot(t, Wx, axes=(1, 1)).transpose(0, 2, 1) / 255.0      # [S, S, 3]
    return x[..., ::-1]


@pytest.mark.parametrize("hw", [(810, 1080), (300, 224), (224, 500), (233, 241)])
def test_preprocess_cls_vs_float64(hw):
    img = modelgen.synth_frame(hw[0], hw[1], 12, 3)
    got = post.preprocess_cls(img, 224)
    want = _triangle_resize_f64(img, 224)
    assert got.shape == (224, 224, 3)
    # fp32 evaluation + fp16 output: half an fp16 ulp at 1.0 plus fp32 noise
    assert np.abs(got - want).max() <= 6e-4


def test_preprocess_cls_constant_and_identity():
    c = np.full((517, 333, 3), (10, 100, 200), np.uint8)
    got = post.preprocess_cls(c, 224)
    for ch, v in enumerate((200, 100, 10)):   # RGB out of BGR in
        assert np.all(got[..., ch] == np.float16(np.float32(v) / np.float32(255.0)).astype(np.float32))
    img = modelgen.synth_frame(224, 224, 10, 5)
    got = post.preprocess_cls(img, 224)       # scale 1: every pixel is its own source
    want = (img[..., ::-1].astype(np.float32) / np.float32(255.0)).astype(np.float16).astype(np.float32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("hw", [(810, 1080), (480, 640)])
def test_preprocess_cls_vs_pil(hw):
    """PIL's antialiased BILINEAR (its uint8 fixed-point filter) agrees within 1-2 levels."""
    img = modelgen.synth_frame(hw[0], hw[1], 12, 9)
    rh, rw, top, left = post.cls_geom(224, *hw)
    pil = Image.fromarray(img[..., ::-1].copy()).resize((rw, rh), Image.BILINEAR)
    pil = np.asarray(pil)[top:top + 224, left:left + 224].astype(np.float32)
    got = post.preprocess_cls(img, 224) * 255.0
    assert np.abs(got - pil).max() <= 2.0
    assert np.abs(got - pil).mean() <= 0.6


def test_topk_ties_and_order():
    p = np.array([0.1, 0.3, 0.3, 0.05, 0.25, 0.3], np.float32)
    ids, pr = post.topk(p, 4)
    assert ids.tolist() == [1, 2, 5, 4]
    assert pr.tolist() == pytest.approx([0.3, 0.3, 0.3, 0.25])


def test_gap_softmax_vs_torch():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 7, 5, 48), dtype=np.float32)
    want = F.adaptive_avg_pool2d(torch.from_numpy(x).permute(0, 3, 1, 2), 1).permute(0, 2, 3, 1).numpy()
    assert np.abs(interp.gap(x) - want).max() <= 1e-6
    z = (rng.standard_normal((3, 1, 1, 1000), dtype=np.float32) * 4).astype(np.float32)
    s = interp.softmax_ch(z)
    assert np.abs(s - torch.softmax(torch.from_numpy(z), -1).numpy()).max() <= 1e-7
    assert np.allclose(s.sum(-1), 1.0, atol=1e-5)
    assert np.abs(interp.softmax_ch(z + 3.0) - s).max() <= 1e-7   # shift invariance


def test_cls_topology(models):
    """yolo11n-cls: the reference's layer table (docs/specs/cls.md:29-41,47-55) -- layer 8
    out 256, C2PSA c 128 / 2 heads / N = 49 at 224, Classify conv 256 -> 1280, linear
    1280 -> 1000 -- and the parameter count that table implies."""
    d = models("yolo11", "n", "classify", imgsz=224, nc=1000)
    g = graphfile.load(d)
    assert g.task == "classify" and g.nc == 1000 and g.imgsz == 224
    kinds = [o.kind for o in g.ops]
    assert kinds[-3:] == ["GAP", "CONV", "SOFTMAX"]
    attn = [o for o in g.ops if o.kind == "ATTN"]
    assert len(attn) == 1 and attn[0].heads == 2
    qkv_shape = g.shape(attn[0].a)
    assert qkv_shape[:2] == (7, 7)
    head = [o for o in g.ops if o.kind == "CONV"][-2:]
    assert (head[0].Cin, head[0].Cout, head[0].k) == (256, 1280, 1)
    assert (head[1].Cin, head[1].Cout) == (1280, 1000)
    w = np.fromfile(os.path.join(d, "weights.f16"), np.float16)
    assert w.size == 2_800_944
    assert yolort.graph_check(d) == (len(g.ops), "")


def test_cls_loader_rules(models, tmp_path):
    d = models("yolo11", "n", "classify", imgsz=224, nc=1000)
    lines = open(os.path.join(d, "model.graph")).read().splitlines()

    def check(mut):
        dd = tmp_path / f"m{len(os.listdir(tmp_path))}"
        dd.mkdir()
        for f in ("weights.f16", "bias.f32"):
            os.symlink(os.path.join(d, f), dd / f)
        (dd / "model.graph").write_text("\n".join(mut(list(lines))) + "\n")
        return yolort.graph_check(str(dd))

    # nc in the header must match the probs tensor
    n, err = check(lambda L: [L[0], L[1].replace("1000", "999")] + L[2:])
    assert n == -1 and "probs" in err
    # a classify graph needs its SOFTMAX
    n, err = check(lambda L: L[:2] + [" ".join([L[2].split()[0], L[2].split()[1], str(int(L[2].split()[2]) - 1)])]
                   + L[3:-1])
    assert n == -1 and "SOFTMAX" in err
