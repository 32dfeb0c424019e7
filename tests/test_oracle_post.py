"""Pins the pre/post-processing oracle (oracle/post.py) with closed forms, special cases,
reference-held geometry and the greedy-NMS characterisation (hypothesis-driven)."""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import post

F16 = np.float16


# ------------------------------------------------------------------ letterbox
def test_letterbox_geometry_c0():
    """810x1080 -> 640 (the config-0 frame): scale 0.5926, nh 480, top 80, full width."""
    scale, top, left, nh, nw = post.letterbox_geom(640, 640, 810, 1080)
    assert abs(scale - 0.5926) < 1e-4 and (nh, nw, top, left) == (480, 640, 80, 0)
    scale, top, left, nh, nw = post.letterbox_geom(640, 640, 1080, 1920)
    assert (nh, nw, top, left) == (360, 640, 140, 0)


def test_letterbox_identity():
    """Same size: scale 1, every sample lands on a pixel centre -> exact copy /255."""
    img = np.random.default_rng(0).integers(0, 256, (64, 64, 3), dtype=np.uint8)
    out = post.letterbox(img, 64, 64)
    want = (img[..., ::-1].astype(np.float32) / np.float32(255)).astype(F16)
    np.testing.assert_array_equal(out, want)


def test_letterbox_constant_and_pad():
    img = np.full((30, 50, 3), 200, np.uint8)
    out = post.letterbox(img, 64, 64)
    scale, top, left, nh, nw = post.letterbox_geom(64, 64, 30, 50)
    inner = out[top:top + nh, left:left + nw].astype(np.float32)
    np.testing.assert_allclose(inner, np.float32(F16(200 / 255)), atol=0)
    assert (out[:top] == F16(114 / 255)).all() and (out[top + nh:] == F16(114 / 255)).all()


def test_letterbox_vs_float64_bilinear():
    """Textbook half-pixel bilinear with replicate clamp, in float64."""
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (37, 53, 3), dtype=np.uint8)
    S = 48
    out = post.letterbox(img, S, S).astype(np.float64)
    scale, top, left, nh, nw = post.letterbox_geom(S, S, 37, 53)
    s = float(scale)
    for y in range(top, top + nh):
        for x in range(left, left + nw):
            fy, fx = (y - top + 0.5) / s - 0.5, (x - left + 0.5) / s - 0.5
            y0, x0 = int(np.floor(fy)), int(np.floor(fx))
            wy, wx = fy - y0, fx - x0
            ys = [min(max(y0, 0), 36), min(max(y0 + 1, 0), 36)]
            xs = [min(max(x0, 0), 52), min(max(x0 + 1, 0), 52)]
            v = ((1 - wy) * (1 - wx) * img[ys[0], xs[0]] + (1 - wy) * wx * img[ys[0], xs[1]]
                 + wy * (1 - wx) * img[ys[1], xs[0]] + wy * wx * img[ys[1], xs[1]]) / 255.0
            np.testing.assert_allclose(out[y, x], v[::-1], atol=1e-3)


# ------------------------------------------------------------------ decode
def _heads(H, W, nc, ncpad=None):
    ncpad = ncpad or nc
    box = np.zeros((H, W, 64), np.float32)
    cls = np.full((H, W, ncpad), -10.0, np.float32)
    return box, cls


def test_dfl_special_cases():
    one_hot = np.full((3, 4, 16), -30.0, np.float32)
    for s in range(4):
        one_hot[:, s, 3 * s + 1] = 30.0
    d = post.dfl(one_hot)
    np.testing.assert_allclose(d, [[1, 4, 7, 10]] * 3, atol=1e-5)
    np.testing.assert_allclose(post.dfl(np.zeros((2, 4, 16), np.float32)), 7.5, atol=1e-6)
    x = np.random.default_rng(0).standard_normal((5, 4, 16)).astype(np.float32)
    from scipy.special import softmax
    np.testing.assert_allclose(post.dfl(x), (softmax(x.astype(np.float64), -1) * np.arange(16)).sum(-1), rtol=1e-5)


def test_decode_rules():
    from scipy.special import expit
    box, cls = _heads(2, 3, 5, 8)
    cls[0, 0, :5] = [0.3, 2.0, 2.0, -1, 0]     # tie -> first index wins
    cls[0, 1, 5:] = 50.0                        # pad logits never win
    cls[0, 1, 4] = -1.0986123                   # score = 0.25 exactly-ish: kept iff >= conf
    cls[1, 2, 0] = 1.0
    c = post.decode(box, cls, 5, 8, 0.25)
    order = np.argsort(c["anchor"])
    anchors = c["anchor"][order]
    assert list(anchors[:1]) == [0] and c["cls"][order][0] == 1
    np.testing.assert_allclose(c["score"][order][0], expit(2.0), rtol=1e-6)
    assert 5 in anchors and c["cls"][order][list(anchors).index(5)] == 0
    # box: all-zero DFL logits -> d = 7.5 on every side around the anchor centre
    i0 = list(anchors).index(0)
    np.testing.assert_allclose(c["box"][order][i0], [(0.5 - 7.5) * 8, (0.5 - 7.5) * 8, 8 * 8, 8 * 8], atol=1e-4)
    s_edge = np.float32(1) / (np.float32(1) + np.exp(np.float32(1.0986123)))
    assert (1 in anchors) == (s_edge >= np.float32(0.25))


# ------------------------------------------------------------------ NMS
def _greedy_properties(c, keep, thr, cap, max_det):
    order = post.rank_order(c["score"], c["anchor"])[:cap]
    pos = {int(i): r for r, i in enumerate(order)}
    ranks = [pos[int(i)] for i in keep]
    assert ranks == sorted(ranks)                      # output in rank order
    kept = set(int(i) for i in keep)
    for a in range(len(keep)):                         # survivors do not suppress each other
        for b in range(a + 1, len(keep)):
            i, j = keep[a], keep[b]
            if c["cls"][i] == c["cls"][j]:
                inter, ua = post.iou_row(c["box"][i], c["box"][j:j + 1])
                assert not (ua[0] > 0 and inter[0] / ua[0] > np.float32(thr))
    if len(keep) < max_det:                            # every other candidate is explained
        for r, i in enumerate(order):
            if int(i) in kept:
                continue
            ok = False
            for j in keep:
                if pos[int(j)] < r and c["cls"][j] == c["cls"][i]:
                    inter, ua = post.iou_row(c["box"][j], c["box"][i:i + 1])
                    ok |= bool(ua[0] > 0 and inter[0] / ua[0] > np.float32(thr))
            assert ok, r


@settings(max_examples=60, deadline=None)
@given(st.integers(0, 2 ** 31 - 1), st.integers(1, 60), st.integers(1, 4), st.sampled_from([0.3, 0.45, 0.7]))
def test_nms_greedy_characterisation(seed, n, ncls, thr):
    rng = np.random.default_rng(seed)
    xy = rng.uniform(0, 100, (n, 2)).astype(np.float32)
    wh = rng.uniform(1, 40, (n, 2)).astype(np.float32)
    c = {"box": np.concatenate([xy, xy + wh], 1).astype(np.float32),
         "score": rng.choice(np.linspace(0.3, 1.0, 8), n).astype(np.float32),   # many exact ties
         "cls": rng.integers(0, ncls, n), "anchor": rng.permutation(1000)[:n]}
    keep, n_raw = post.nms(c, thr, max_det=300, cap=2048)
    assert n_raw == n
    _greedy_properties(c, keep, thr, 2048, 300)


def test_nms_cap_and_maxdet():
    rng = np.random.default_rng(9)
    n = 500
    xy = rng.uniform(0, 4000, (n, 2)).astype(np.float32)
    c = {"box": np.concatenate([xy, xy + 5], 1).astype(np.float32), "score": rng.uniform(0.3, 1, n).astype(np.float32),
         "cls": np.zeros(n, int), "anchor": np.arange(n)}
    keep, _ = post.nms(c, 0.45, max_det=300, cap=2048)
    assert len(keep) == 300                                   # disjoint boxes: max_det binds
    np.testing.assert_array_equal(keep, post.rank_order(c["score"], c["anchor"])[:300])
    keep2, _ = post.nms(c, 0.45, max_det=300, cap=100)
    assert len(keep2) == 100                                  # only the top `cap` enter NMS


def test_nms_tiny_known():
    c = {"box": np.array([[0, 0, 10, 10], [1, 1, 11, 11], [20, 20, 30, 30], [0, 0, 10, 10]], np.float32),
         "score": np.array([0.9, 0.8, 0.7, 0.95], np.float32), "cls": np.array([0, 0, 0, 1]),
         "anchor": np.arange(4)}
    keep, _ = post.nms(c, 0.45)
    assert list(keep) == [3, 0, 2]       # box 1 overlaps box 0 (IoU 0.68) and is dropped


# ------------------------------------------------------------------ masks
def test_masks_known_case():
    proto = np.zeros((8, 8, 8), np.float32)
    proto[..., 0] = 1.0
    proto[2:5, :, 0] = -1.0
    coef = np.array([[1, 0, 0, 0, 0, 0, 0, 0]], np.float32)
    boxes = np.array([[4.0, 0.0, 20.0, 28.0]], np.float32)   # net 32x32 -> proto scale 1/4
    m = post.masks(proto, coef, boxes, 32, 32)[0]
    want = np.zeros((8, 8), np.uint8)
    want[0:7, 1:5] = 1          # x in [1, 5), y in [0, 7)
    want[2:5] = 0               # negative logits
    np.testing.assert_array_equal(m, want)
