"""Pins the OBB part of the oracle (oracle/post.py: decode_obb, covariance, probiou, nms_obb).

probiou is checked against the Bhattacharyya distance between two Gaussians written
independently in float64 with numpy.linalg, and against its symmetries and clamped limits.
Fast-NMS is checked by brute force, by a chain where it differs from greedy NMS, and by the
>= tie.  The decode is checked against a float64 rotation-matrix restatement of dist2rbox
(docs/specs/obb.md:116-128)."""
import math

import numpy as np

from oracle import post

F32 = np.float32


# ------------------------------------------------------------------ probiou
def _gauss(w, h, th):
    """2x2 covariance of a w x h box rotated by th (float64), R diag(w^2/12, h^2/12) R^T."""
    R = np.array([[math.cos(th), -math.sin(th)], [math.sin(th), math.cos(th)]])
    return R @ np.diag([w * w / 12.0, h * h / 12.0]) @ R.T


def _probiou64(b1, b2):
    """1 - Hellinger distance from the Bhattacharyya distance of N(c1, S1) and N(c2, S2)."""
    S1, S2 = _gauss(*b1[2:]), _gauss(*b2[2:])
    S = (S1 + S2) / 2
    d = np.array(b1[:2]) - np.array(b2[:2])
    bd = d @ np.linalg.inv(S) @ d / 8 + 0.5 * math.log(np.linalg.det(S) / math.sqrt(np.linalg.det(S1) * np.linalg.det(S2)))
    return 1 - math.sqrt(1 - math.exp(-bd))


def _probiou32(b1, b2):
    A1, B1, C1 = post.covariance(b1[2], b1[3], b1[4])
    A2, B2, C2 = post.covariance(b2[2], b2[3], b2[4])
    return float(post.probiou(F32(b1[0]), F32(b1[1]), A1, B1, C1, F32(b2[0]), F32(b2[1]), A2, B2, C2))


def _rand_box(rng, around=None):
    c = rng.uniform(0, 200, 2) if around is None else np.asarray(around[:2]) + rng.normal(0, 8, 2)
    return (float(c[0]), float(c[1]), float(rng.uniform(4, 60)), float(rng.uniform(4, 60)),
            float(rng.uniform(-math.pi / 4, 3 * math.pi / 4)))


def test_probiou_vs_float64_bhattacharyya():
    rng = np.random.default_rng(0)
    worst, n = 0.0, 0
    for _ in range(400):
        b1 = _rand_box(rng)
        b2 = _rand_box(rng, b1)
        want = _probiou64(b1, b2)
        if want > 0.999:          # bd below ~1e-6: fp32 1 - exp(-bd) has no digits left
            continue
        worst = max(worst, abs(_probiou32(b1, b2) - want))
        n += 1
    assert n > 300 and worst < 2e-4, (n, worst)


def test_probiou_cross_term_sign():
    """Two 40x4 sticks at +45 degrees offset along +45 overlap far more than if offset along
    -45: a sign error in the C (cross) term swaps the two."""
    s = math.pi / 4
    along = _probiou32((0, 0, 40, 4, s), (6, 6, 40, 4, s))
    across = _probiou32((0, 0, 40, 4, s), (6, -6, 40, 4, s))
    assert along > 0.5 > across
    assert abs(along - _probiou64((0, 0, 40, 4, s), (6, 6, 40, 4, s))) < 1e-4
    assert abs(across - _probiou64((0, 0, 40, 4, s), (6, -6, 40, 4, s))) < 1e-4


def test_probiou_symmetries():
    rng = np.random.default_rng(1)
    for _ in range(100):
        b1 = _rand_box(rng)
        b2 = _rand_box(rng, b1)
        base = _probiou32(b1, b2)
        assert _probiou32(b2, b1) == base                                 # symmetric, bitwise
        flip = (b1[0], b1[1], b1[2], b1[3], b1[4] + math.pi)
        assert abs(_probiou32(flip, b2) - base) < 2e-5                     # theta ~ theta + pi
        swap = (b1[0], b1[1], b1[3], b1[2], b1[4] + math.pi / 2)
        assert abs(_probiou32(swap, b2) - base) < 2e-5                     # (w,h,t) ~ (h,w,t+pi/2)
        phi = rng.uniform(0, 2 * math.pi)
        c, s = math.cos(phi), math.sin(phi)
        rot = [(c * b[0] - s * b[1], s * b[0] + c * b[1], b[2], b[3], b[4] + phi) for b in (b1, b2)]
        assert abs(_probiou32(*rot) - base) < 2e-4                         # rigid rotation


def test_probiou_clamps():
    """Identical boxes: bd clamps at eps -> 1 - sqrt(1 - exp(-eps) + eps); far boxes: bd
    clamps at 100 -> 1 - sqrt(1 + eps), 0 in fp32, so they never suppress at thr > 0."""
    b = (50.0, 60.0, 20.0, 8.0, 0.3)
    eps = F32(1e-7)
    # in fp32, exp(-eps) = 1 - 2^-24: the clamped value is 0.99960, an unclamped bd of a few
    # 1e-8 would give 0.99968 and a negative one NaN
    clamped = F32(1) - np.sqrt((F32(1) - np.exp(-eps)) + eps)
    assert abs(_probiou32(b, b) - float(clamped)) < 1e-6 and abs(float(clamped) - 0.99960) < 1e-5
    far = _probiou32(b, (5e3, 60.0, 20.0, 8.0, 0.3))
    assert -1e-6 < far <= 0.0
    # zero-size boxes (det = 0): the eps in the t3 sqrt denominator keeps t3 finite
    # (0.5 log(eps) < 0) and only the lower clamp stops bd going negative (NaN iou), so
    # two zero-size boxes at one point suppress each other like identical boxes
    z = (50.0, 60.0, 0.0, 0.0, 0.0)
    assert abs(_probiou32(z, z) - float(clamped)) < 1e-6


# ------------------------------------------------------------------ fast-NMS
def _cands(boxes, scores, cls, anchors=None):
    boxes = np.asarray(boxes, np.float64)
    n = len(scores)
    return {"rbox": boxes[:, :4].astype(F32), "theta": boxes[:, 4].astype(F32),
            "score": np.asarray(scores, F32), "cls": np.asarray(cls, np.int64),
            "anchor": np.arange(n, dtype=np.int64) if anchors is None else np.asarray(anchors, np.int64)}


def _brute_fast_nms(c, thr, max_det, cap):
    order = sorted(range(len(c["score"])), key=lambda i: (-float(c["score"][i]), int(c["anchor"][i])))[:cap]
    keep = []
    for jj, j in enumerate(order):
        bj = tuple(c["rbox"][j]) + (c["theta"][j],)
        hit = False
        for i in order[:jj]:
            if c["cls"][i] != c["cls"][j]:
                continue
            if _probiou32(tuple(c["rbox"][i]) + (c["theta"][i],), bj) >= thr:
                hit = True
                break
        if not hit:
            keep.append(j)
    return keep[:max_det]


def test_nms_obb_brute_force():
    rng = np.random.default_rng(2)
    for trial in range(60):
        n = int(rng.integers(1, 14))
        centre = rng.uniform(0, 60, 2)
        boxes = [(*(centre + rng.normal(0, 6, 2)), rng.uniform(5, 30), rng.uniform(5, 30),
                  rng.uniform(-0.8, 2.4)) for _ in range(n)]
        scores = rng.choice([0.3, 0.5, 0.7, 0.9], n) if trial % 2 else rng.uniform(0.25, 1, n)
        c = _cands(boxes, scores, rng.integers(0, 2, n), rng.permutation(100)[:n])
        thr = float(rng.choice([0.3, 0.45, 0.7]))
        max_det, cap = int(rng.integers(1, 15)), int(rng.integers(1, 15))
        keep, n_raw = post.nms_obb(c, thr, max_det, cap)
        assert n_raw == n
        assert list(keep) == _brute_fast_nms(c, thr, max_det, cap)


def test_nms_obb_fast_not_greedy():
    """A > B > C in score, iou(A,B) and iou(B,C) above thr, iou(A,C) below: greedy NMS keeps
    A and C, fast-NMS keeps A only (the suppressed B still suppresses C)."""
    mk = lambda x: (x, 0.0, 10.0, 10.0, 0.0)
    d = 2.5
    assert _probiou32(mk(0), mk(d)) >= 0.45 and _probiou32(mk(0), mk(2 * d)) < 0.45
    c = _cands([mk(0), mk(d), mk(2 * d)], [0.9, 0.8, 0.7], [0, 0, 0])
    keep, _ = post.nms_obb(c, 0.45)
    assert list(keep) == [0]
    c["cls"] = np.array([0, 1, 0])      # B in another class: it suppresses nothing, and
    keep, _ = post.nms_obb(c, 0.45)     # iou(A, C) < thr keeps C
    assert list(keep) == [0, 1, 2]


def test_nms_obb_threshold_is_inclusive():
    """iou == thr suppresses (>=), one ulp above does not."""
    a, b = (0.0, 0.0, 12.0, 7.0, 0.4), (3.0, 1.0, 9.0, 8.0, 0.1)
    v = np.float32(_probiou32(a, b))
    c = _cands([a, b], [0.9, 0.8], [3, 3])
    assert list(post.nms_obb(c, v)[0]) == [0]
    assert list(post.nms_obb(c, np.nextafter(v, np.float32(2)))[0]) == [0, 1]


def test_nms_obb_rank_cap_and_max_det():
    """Ties in score rank by anchor; max_det keeps the best survivors, cap the best inputs."""
    boxes = [(100.0 * i, 0.0, 10.0, 10.0, 0.0) for i in range(10)]      # disjoint
    scores = [0.5, 0.9, 0.5, 0.7, 0.9, 0.3, 0.5, 0.8, 0.6, 0.4]
    anchors = [9, 8, 7, 6, 5, 4, 3, 2, 1, 0]
    c = _cands(boxes, scores, [0] * 10, anchors)
    keep, n_raw = post.nms_obb(c, 0.45)
    assert n_raw == 10 and list(keep) == [4, 1, 7, 3, 8, 6, 2, 0, 9, 5]
    assert list(post.nms_obb(c, 0.45, max_det=3)[0]) == [4, 1, 7]
    assert list(post.nms_obb(c, 0.45, cap=4)[0]) == [4, 1, 7, 3]


# ------------------------------------------------------------------ decode
def _decode64(box, cls, ang, nc, stride, conf):
    """float64 restatement: DFL expectation, theta = (sigmoid - 1/4) pi, centre = anchor +
    R(theta) ((r - l)/2, (b - t)/2), size (l + r, t + b), all times stride."""
    H, W, _ = box.shape
    out = []
    for y in range(H):
        for x in range(W):
            lg = cls[y, x, :nc].astype(np.float64)
            k = int(np.argmax(lg))
            sc = 1 / (1 + math.exp(-lg[k]))
            if sc < conf:
                continue
            bins = box[y, x].astype(np.float64).reshape(4, 16)
            p = np.exp(bins - bins.max(1, keepdims=True))
            l, t, r, b = (p * np.arange(16)).sum(1) / p.sum(1)
            th = (1 / (1 + math.exp(-float(ang[y, x, 0]))) - 0.25) * math.pi
            R = np.array([[math.cos(th), -math.sin(th)], [math.sin(th), math.cos(th)]])
            cx, cy = np.array([x + 0.5, y + 0.5]) + R @ np.array([(r - l) / 2, (b - t) / 2])
            out.append((y * W + x, cx * stride, cy * stride, (l + r) * stride, (t + b) * stride, th, sc, k))
    return out


def test_decode_obb_vs_float64():
    rng = np.random.default_rng(4)
    H, W, nc, stride = 6, 7, 15, 16
    box = rng.normal(0, 2, (H, W, 64)).astype(np.float16)
    cls = np.concatenate([rng.normal(-1, 1.5, (H, W, nc)), np.zeros((H, W, 1))], 2).astype(np.float16)
    ang = np.concatenate([rng.normal(0, 2, (H, W, 1)), rng.normal(0, 9, (H, W, 7))], 2).astype(np.float16)
    got = post.decode_obb(box, cls, ang, nc, stride, 0.25, anchor_base=100)
    want = _decode64(box, cls, ang, nc, stride, 0.25)
    assert len(want) > 10 and len(got["score"]) == len(want)
    w = np.array([v[1:] for v in want])
    np.testing.assert_array_equal(got["anchor"], [100 + v[0] for v in want])
    np.testing.assert_allclose(got["rbox"], w[:, :4], rtol=0, atol=2e-3)
    np.testing.assert_allclose(got["theta"], w[:, 4], rtol=0, atol=1e-6)
    np.testing.assert_allclose(got["score"], w[:, 5], rtol=0, atol=1e-6)
    np.testing.assert_array_equal(got["cls"], w[:, 6].astype(int))


def test_decode_obb_special_cases():
    """Angle logit 0 -> theta = pi/4; a pad class channel (index >= nc) never wins; with
    theta ~ 0 the rotated box equals the detect decode's box in centre form."""
    H, W, nc = 2, 3, 15
    box = np.zeros((H, W, 64), np.float16)
    box[..., 3] = box[..., 16 + 5] = box[..., 32 + 7] = box[..., 48 + 1] = 20    # l3 t5 r7 b1
    cls = np.full((H, W, 16), -9, np.float16)
    cls[..., 15] = 30                     # pad channel: must be ignored
    cls[0, 1, 4] = 2.0
    ang = np.zeros((H, W, 8), np.float16)
    r = post.decode_obb(box, cls, ang, nc, 8, 0.25)
    assert list(r["anchor"]) == [1] and list(r["cls"]) == [4]
    assert abs(float(r["theta"][0]) - math.pi / 4) < 1e-6
    ang[..., 0] = np.float16(-math.log(3))                                    # sigmoid ~ 1/4
    r = post.decode_obb(box, cls, ang, nc, 8, 0.25)
    d = post.decode(box, cls, nc, 8, 0.25)
    xyxy = d["box"][0]
    ctr = [(xyxy[0] + xyxy[2]) / 2, (xyxy[1] + xyxy[3]) / 2, xyxy[2] - xyxy[0], xyxy[3] - xyxy[1]]
    assert abs(float(r["theta"][0])) < 1e-3
    np.testing.assert_allclose(r["rbox"][0], ctr, rtol=0, atol=0.05)


def test_far_pair_skip_bound():
    """The device NMS skips a same-class pair without evaluating probiou when both boxes are
    "bounded" (covariance determinant >= 1 and >= 1e-4 trace^2, i.e. condition number below
    ~1e4) and |d|^2 > 8 B*(thr) (A1 + B1 + A2 + B2), with B*(thr) = -ln(1 + eps - (1 - thr)^2)
    (for 0.05 <= thr <= 0.95).  Every pair so skipped must have fp32 probiou < thr: checked
    just beyond the skip distance on random pairs and on sticks aligned with their offset
    (where bd / |d|^2 is smallest and the fp32 cross term cancels most)."""
    rng = np.random.default_rng(5)
    checked = 0
    for thr in (0.05, 0.3, 0.45, 0.7, 0.95):
        t = F32(thr)
        K = F32(8) * -np.log(F32(1) + F32(1e-7) - (F32(1) - t) * (F32(1) - t))
        for trial in range(3000):
            stick = trial % 2 == 0
            if stick:
                phi = rng.uniform(-math.pi, math.pi)
                b = []
                for _ in range(2):
                    w = rng.uniform(20, 400)
                    b.append((w, w / rng.uniform(10, 100), phi + rng.normal(0, 0.02)))
                ang = phi
            else:
                b = [(rng.uniform(1, 200), rng.uniform(1, 200), rng.uniform(-1, 3)) for _ in range(2)]
                ang = rng.uniform(-math.pi, math.pi)
            cov = [post.covariance(F32(w), F32(h), F32(th)) for w, h, th in b]
            dets = [max(A * B - C * C, 0) for A, B, C in cov]
            if any(dt < 1 or dt < F32(1e-4) * (A + B) * (A + B) for dt, (A, B, C) in zip(dets, cov)):
                continue
            checked += 1
            tr = (cov[0][0] + cov[1][0]) + (cov[0][1] + cov[1][1])
            r = math.sqrt(float(K * tr) * (1 + rng.uniform(1e-6, 0.02)))
            dx, dy = F32(r * math.cos(ang)), F32(r * math.sin(ang))
            if not dx * dx + dy * dy > K * tr:
                continue
            v = post.probiou(dx, dy, *cov[0], F32(0), F32(0), *cov[1])
            assert v < t, (thr, b, float(v))
    assert checked > 10000
