"""Pre/post-processing oracle (numpy fp32) -- TEST INFRASTRUCTURE, see oracle/__init__.py.

Functions, the reference lines they restate, and what pins them (tests/test_oracle_post.py):

letterbox_geom  host geometry, engine/engine.cu:1704-1710.  Pinned by the C0 numbers
                (810x1080 -> scale 0.5926, nh 480, top 80) and identity at equal size.
letterbox       k_preprocess, engine/engine.cu:966-998 (fp32 bilinear, half-pixel map,
                replicate clamp, pad 114, BGR->RGB, /255, fp16 out).  Pinned by: the
                scale-1 identity (output == src/255 exactly), constant images, and a
                float64 bilinear written from the textbook half-pixel formula.
decode          k_decode<NM>, engine/engine.cu:844-906 (first-max argmax over the real
                classes, sigmoid, keep score >= conf, DFL expectation, xyxy * stride).
                Pinned by one-hot bins -> integer distances, uniform bins -> 7.5, and a
                scipy.special.softmax / expit restatement.
nms             k_nms, engine/engine.cu:1048-1123: greedy, same-class only, suppress when
                inter/union > thr with a union > 0 guard.  Deliberate differences, shared
                with the HIP engine: candidates are ranked by the total order (score desc,
                anchor asc) instead of an unstable bitonic sort over atomic-order slots,
                and the cap keeps the top `cap` by that order instead of the first 1,024 in
                arrival order.  Pinned by the greedy-NMS characterisation (survivors are
                pairwise below thr per class; every suppressed box overlaps a higher-ranked
                survivor above thr) and brute force on tiny sets.
masks           k_mask_assemble, engine/engine.cu:1125-1158 (coef . proto, half-open box
                crop at proto scale, logit > 0).  Pinned by a hand-built case with a known
                answer and by the crop/threshold invariants.
decode_obb      k_decode_obb, engine/engine.cu:908-964 (theta = (sigmoid(t) - 0.25) * pi,
                dist2rbox, record cx, cy, w, h, score, cls, theta).  Pinned by a float64
                restatement of ultralytics dist2rbox as a rotation matrix
                (docs/specs/obb.md:116-128), theta = pi/4 at logit 0, and the axis-aligned
                case reducing to the detect decode.
covariance,     probiou (engine/engine.cu:1160-1176, ultralytics batch_probiou with its eps
probiou         placement).  Pinned by the Bhattacharyya distance between two Gaussians
                computed in float64 with numpy.linalg (det, inv) from R diag(w^2/12, h^2/12)
                R^T, rotation invariance, theta ~ theta + pi, (w, h, theta) ~ (h, w,
                theta + pi/2), identical boxes (bd clamped at eps) and far boxes (clamped
                at 100).
cls_geom        classify host geometry, engine/engine.cu:1036-1046 (torchvision Resize(S):
                short edge -> S, long edge S * long // short; CenterCrop offsets rounded half
                to even).  Pinned by hand cases against Python's round().
preprocess_cls  k_preprocess_cls, engine/engine.cu:1000-1034: PIL-style antialiased bilinear
                (triangle filter whose support widens by the downscale factor), centre crop,
                BGR->RGB, /255.  Evaluated in fp32 in the kernel's operation order, so the
                engine must match it bit for bit.  Pinned by: a float64 separable
                triangle-filter resize written from the filter's definition (agreement to
                fp32 rounding), constant frames (exactly constant output), the scale-1
                identity, and PIL's own antialiased BILINEAR resize (uint8 output, within
                one level).
topk            the reference's top-k insertion (engine/engine.cu:1593-1606): descending,
                lower class id first among equal probabilities.  Pinned vs a stable argsort.
nms_obb         k_nms_obb, engine/engine.cu:1178-1252: ultralytics fast-NMS (a suppressed
                box still suppresses; iou >= thr; same class only).  Ranked and capped by
                the same total order as nms.  Pinned by brute force on tiny sets, a chain
                case where fast-NMS and greedy NMS differ, and the >= tie.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


# ----------------------------------------------------------------------------- classify
def cls_geom(S: int, sh: int, sw: int):
    """(rh, rw, top, left): resize the short edge to S, centre-crop S x S."""
    if sw <= sh:
        rw, rh = S, S * sh // sw
    else:
        rh, rw = S, S * sw // sh
    return rh, rw, int(round((rh - S) / 2)), int(round((rw - S) / 2))


def preprocess_cls(src: np.ndarray, S: int) -> np.ndarray:
    """BGR u8 [sh, sw, 3] -> RGB float32 [S, S, 3] (fp16-rounded): the kernel's fp32
    arithmetic, vectorised over destination pixels, in the kernel's summation order."""
    sh, sw = src.shape[:2]
    rh, rw, top, left = cls_geom(S, sh, sw)
    fy, fx = F32(sh) / F32(rh), F32(sw) / F32(rw)
    ry, rx = max(fy, F32(1.0)), max(fx, F32(1.0))
    oy = np.arange(S)
    cy = ((oy + top).astype(F32) + F32(0.5)) * fy                 # per output row
    cx = ((oy + left).astype(F32) + F32(0.5)) * fx                # per output column
    ya = np.maximum(0, (cy - ry + F32(0.5)).astype(np.int64))
    yb = np.minimum(sh, (cy + ry + F32(0.5)).astype(np.int64))
    xa = np.maximum(0, (cx - rx + F32(0.5)).astype(np.int64))
    xb = np.minimum(sw, (cx + rx + F32(0.5)).astype(np.int64))

    def tri(d, r):
        return np.maximum(F32(0.0), F32(1.0) - np.abs(d).astype(F32) / r).astype(F32)

    ny = np.zeros(S, F32)
    for k in range(int((yb - ya).max())):
        i = ya + k
        ny = np.where(i < yb, ny + tri(i.astype(F32) + F32(0.5) - cy, ry), ny).astype(F32)
    nx = np.zeros(S, F32)
    for k in range(int((xb - xa).max())):
        j = xa + k
        nx = np.where(j < xb, nx + tri(j.astype(F32) + F32(0.5) - cx, rx), nx).astype(F32)
    srcf = src.astype(F32)
    acc = np.zeros((S, S, 3), F32)            # b, g, r sums per destination pixel
    for ki in range(int((yb - ya).max())):
        i = ya + ki                                                       # [S] rows
        wy = tri(i.astype(F32) + F32(0.5) - cy, ry)
        vi = i < yb
        rows = srcf[np.minimum(i, sh - 1)]                                # [S, sw, 3]
        for kj in range(int((xb - xa).max())):
            j = xa + kj                                                   # [S] cols
            wx = tri(j.astype(F32) + F32(0.5) - cx, rx)
            w = (wy[:, None] * wx[None, :]).astype(F32)                   # [S, S]
            px = rows[:, np.minimum(j, sw - 1)]                           # [S, S, 3]
            ok = (vi[:, None] & (j < xb)[None, :])[..., None]
            acc = np.where(ok, acc + (w[..., None] * px).astype(F32), acc).astype(F32)
    inv = F32(1.0) / (ny[:, None] * nx[None, :] * F32(255.0))
    out = (acc * inv[..., None]).astype(F32)[..., ::-1]                  # BGR -> RGB
    return out.astype(np.float16).astype(F32)


def topk(probs: np.ndarray, k: int):
    """(ids, probs) of the k largest, lower id first among equals."""
    order = np.argsort(-probs.astype(np.float64), kind="stable")[:k]
    return order.astype(np.int32), probs[order].astype(F32)


# ----------------------------------------------------------------------------- letterbox
def letterbox_geom(S_h: int, S_w: int, sh: int, sw: int):
    """(scale, top, left, nh, nw) exactly as the engine host computes them in fp32."""
    scale = min(F32(S_h) / F32(sh), F32(S_w) / F32(sw))
    nh = int(math.floor(float(F32(sh) * scale) + 0.5))   # roundf on a positive value
    nw = int(math.floor(float(F32(sw) * scale) + 0.5))
    top, left = (S_h - nh) // 2, (S_w - nw) // 2
    return F32(scale), top, left, nh, nw


def letterbox(src: np.ndarray, S_h: int, S_w: int) -> np.ndarray:
    """src: u8 BGR [sh, sw, 3] -> fp16 RGB [S_h, S_w, 3] in [0, 1] (pad 114)."""
    sh, sw, _ = src.shape
    scale, top, left, nh, nw = letterbox_geom(S_h, S_w, sh, sw)
    y, x = np.mgrid[0:S_h, 0:S_w]
    inside = (y >= top) & (y < top + nh) & (x >= left) & (x < left + nw)
    fy = (F32(0.5) + (y - top).astype(F32)) / scale - F32(0.5)
    fx = (F32(0.5) + (x - left).astype(F32)) / scale - F32(0.5)
    y0 = np.floor(fy).astype(np.int64)
    x0 = np.floor(fx).astype(np.int64)
    wy = (fy - y0.astype(F32)).astype(F32)
    wx = (fx - x0.astype(F32)).astype(F32)
    y1 = np.minimum(y0 + 1, sh - 1)
    x1 = np.minimum(x0 + 1, sw - 1)
    y0 = np.clip(y0, 0, sh - 1)
    x0 = np.clip(x0, 0, sw - 1)
    y1 = np.clip(y1, 0, sh - 1)
    x1 = np.clip(x1, 0, sw - 1)
    one = F32(1.0)
    w00 = (one - wy) * (one - wx)
    w01 = (one - wy) * wx
    w10 = wy * (one - wx)
    w11 = wy * wx
    s = src.astype(F32)
    out = np.empty((S_h, S_w, 3), F32)
    for c_dst, c_src in ((0, 2), (1, 1), (2, 0)):   # RGB out from BGR in
        p00 = s[y0, x0, c_src]
        p01 = s[y0, x1, c_src]
        p10 = s[y1, x0, c_src]
        p11 = s[y1, x1, c_src]
        v = ((p00 * w00 + p01 * w01) + p10 * w10) + p11 * w11
        v = np.where(inside, v, F32(114.0)).astype(F32)
        out[..., c_dst] = v / F32(255.0)
    return out.astype(np.float16)


# ----------------------------------------------------------------------------- decode
def dfl(bins: np.ndarray) -> np.ndarray:
    """bins [..., 4, 16] -> expected distance [..., 4] (softmax over 16 bins, sum p*i)."""
    mx = bins.max(axis=-1, keepdims=True)
    p = np.exp((bins - mx).astype(F32)).astype(F32)
    ssum = np.zeros(bins.shape[:-1], F32)
    esum = np.zeros(bins.shape[:-1], F32)
    for i in range(16):
        ssum = ssum + p[..., i]
        esum = esum + p[..., i] * F32(i)
    return (esum / ssum).astype(F32)


def decode(box: np.ndarray, cls: np.ndarray, nc: int, stride: int, conf: float,
           coef: np.ndarray | None = None, anchor_base: int = 0):
    """One image, one level.  box [H,W,64], cls [H,W,ncpad], coef [H,W,nm] or None.
    Returns a dict of per-candidate arrays in anchor order (anchor index = base + y*W + x)."""
    H, W, _ = box.shape
    logits = cls[..., :nc].astype(F32).reshape(H * W, nc)
    best = logits.max(axis=1)
    bcls = logits.argmax(axis=1)          # first maximum, like the strict '>' scan
    score = (F32(1.0) / (F32(1.0) + np.exp(-best))).astype(F32)
    keep = score >= F32(conf)
    idx = np.nonzero(keep)[0]
    d = dfl(box.astype(F32).reshape(H * W, 4, 16)[idx])
    yy, xx = idx // W, idx % W
    cx = xx.astype(F32) + F32(0.5)
    cy = yy.astype(F32) + F32(0.5)
    st = F32(stride)
    xyxy = np.stack([(cx - d[:, 0]) * st, (cy - d[:, 1]) * st,
                     (cx + d[:, 2]) * st, (cy + d[:, 3]) * st], 1).astype(F32)
    out = {"anchor": (idx + anchor_base).astype(np.int64), "box": xyxy,
           "score": score[idx], "cls": bcls[idx].astype(np.int64)}
    if coef is not None:
        out["coef"] = coef.astype(F32).reshape(H * W, -1)[idx]
    return out


def decode_all(heads, nc: int, conf: float):
    """heads: list of (box, cls, coef|None, stride) for ONE image, levels in op order."""
    parts, base = [], 0
    for box, cls, coef, st in heads:
        parts.append(decode(box, cls, nc, st, conf, coef, base))
        base += box.shape[0] * box.shape[1]
    return {k: np.concatenate([p[k] for p in parts]) for k in parts[0]}


# ----------------------------------------------------------------------------- nms
def iou_row(a: np.ndarray, b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """inter and union of box a [4] against boxes b [n,4], fp32, reference order of ops."""
    xx1 = np.maximum(a[0], b[:, 0])
    yy1 = np.maximum(a[1], b[:, 1])
    xx2 = np.minimum(a[2], b[:, 2])
    yy2 = np.minimum(a[3], b[:, 3])
    w = np.maximum(F32(0.0), xx2 - xx1)
    h = np.maximum(F32(0.0), yy2 - yy1)
    inter = (w * h).astype(F32)
    aarea = (a[2] - a[0]) * (a[3] - a[1])
    ua = ((aarea + (b[:, 2] - b[:, 0]) * (b[:, 3] - b[:, 1])) - inter).astype(F32)
    return inter, ua


def rank_order(score: np.ndarray, anchor: np.ndarray) -> np.ndarray:
    """Indices sorted by (score desc, anchor asc)."""
    return np.lexsort((anchor, -score.astype(np.float64)))


def nms(c: dict, iou_thr: float, max_det: int = 300, cap: int = 2048):
    """Greedy same-class NMS over decoded candidates c (dict from decode_all).
    Returns (indices into c of the survivors in output order, n_raw)."""
    n_raw = len(c["score"])
    order = rank_order(c["score"], c["anchor"])[:cap]
    boxes = c["box"][order]
    cls = c["cls"][order]
    m = len(order)
    dead = np.zeros(m, bool)
    keep = []
    thr = F32(iou_thr)
    for i in range(m):
        if dead[i]:
            continue
        keep.append(order[i])
        if len(keep) == max_det:
            break
        j = np.arange(i + 1, m)
        j = j[(~dead[j]) & (cls[j] == cls[i])]
        if len(j) == 0:
            continue
        inter, ua = iou_row(boxes[i], boxes[j])
        with np.errstate(divide="ignore", invalid="ignore"):
            sup = (ua > 0) & ((inter / np.where(ua > 0, ua, F32(1.0))).astype(F32) > thr)
        dead[j[sup]] = True
    return np.asarray(keep, np.int64), n_raw


def detect(heads, nc: int, conf: float = 0.25, iou: float = 0.45, max_det: int = 300,
           cap: int = 2048):
    """decode + NMS for one image -> dict with arrays in survivor order."""
    c = decode_all(heads, nc, conf)
    keep, n_raw = nms(c, iou, max_det, cap)
    out = {k: v[keep] for k, v in c.items()}
    out["n_raw"] = n_raw
    return out


# ----------------------------------------------------------------------------- OBB
PI32 = F32(3.14159265358979)
EPS = F32(1e-7)


def decode_obb(box: np.ndarray, cls: np.ndarray, ang: np.ndarray, nc: int, stride: int,
               conf: float, anchor_base: int = 0):
    """One image, one level.  box [H,W,64], cls [H,W,ncpad], ang [H,W,>=1] (channel 0 real).
    Returns per-candidate arrays in anchor order; rbox = (cx, cy, w, h) in net pixels."""
    H, W, _ = box.shape
    logits = cls[..., :nc].astype(F32).reshape(H * W, nc)
    best = logits.max(axis=1)
    bcls = logits.argmax(axis=1)
    score = (F32(1.0) / (F32(1.0) + np.exp(-best))).astype(F32)
    idx = np.nonzero(score >= F32(conf))[0]
    d = dfl(box.astype(F32).reshape(H * W, 4, 16)[idx])
    t0 = ang[..., 0].astype(F32).reshape(H * W)[idx]
    th = ((F32(1.0) / (F32(1.0) + np.exp(-t0))).astype(F32) - F32(0.25)) * PI32
    th = th.astype(F32)
    xf = (d[:, 2] - d[:, 0]) * F32(0.5)
    yf = (d[:, 3] - d[:, 1]) * F32(0.5)
    cs, sn = np.cos(th), np.sin(th)
    yy, xx = idx // W, idx % W
    ax = xx.astype(F32) + F32(0.5)
    ay = yy.astype(F32) + F32(0.5)
    st = F32(stride)
    cx = ((ax + xf * cs) - yf * sn) * st
    cy = ((ay + xf * sn) + yf * cs) * st
    rbox = np.stack([cx, cy, (d[:, 0] + d[:, 2]) * st, (d[:, 1] + d[:, 3]) * st], 1).astype(F32)
    return {"anchor": (idx + anchor_base).astype(np.int64), "rbox": rbox, "theta": th,
            "score": score[idx], "cls": bcls[idx].astype(np.int64)}


def decode_obb_all(heads, nc: int, conf: float):
    """heads: list of (box, cls, ang, stride) for ONE image, levels in op order."""
    parts, base = [], 0
    for box, cls, ang, st in heads:
        parts.append(decode_obb(box, cls, ang, nc, st, conf, base))
        base += box.shape[0] * box.shape[1]
    return {k: np.concatenate([p[k] for p in parts]) for k in parts[0]}


def covariance(w: np.ndarray, h: np.ndarray, th: np.ndarray):
    """(A, B, C) of the Gaussian of a w x h box rotated by th; covariance [[A, C], [C, B]]."""
    w, h, th = (np.asarray(v, F32) for v in (w, h, th))
    a = (w * w) * F32(1.0 / 12.0)
    b = (h * h) * F32(1.0 / 12.0)
    cs, sn = np.cos(th), np.sin(th)
    A = ((a * cs) * cs + (b * sn) * sn).astype(F32)
    B = ((a * sn) * sn + (b * cs) * cs).astype(F32)
    C = (((a - b) * cs) * sn).astype(F32)
    return A, B, C


def probiou(x1, y1, A1, B1, C1, x2, y2, A2, B2, C2) -> np.ndarray:
    """probiou of box 1 vs box 2 (broadcasting fp32 arrays), the reference's operation order."""
    dx = (x1 - x2).astype(F32)
    dy = (y1 - y2).astype(F32)
    sA = (A1 + A2).astype(F32)
    sB = (B1 + B2).astype(F32)
    sC = (C1 + C2).astype(F32)
    disc = (sA * sB - sC * sC).astype(F32)
    den = disc + EPS
    t1 = (F32(0.25) * ((sA * dy) * dy + (sB * dx) * dx)) / den
    t2 = (F32(0.5) * ((sC * (-dx)) * dy)) / den
    det1 = np.maximum(A1 * B1 - C1 * C1, F32(0.0)).astype(F32)
    det2 = np.maximum(A2 * B2 - C2 * C2, F32(0.0)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t3 = F32(0.5) * np.log(disc / (F32(4.0) * np.sqrt(det1 * det2) + EPS) + EPS)
    bd = np.minimum(np.maximum((t1 + t2) + t3, EPS), F32(100.0)).astype(F32)
    return (F32(1.0) - np.sqrt((F32(1.0) - np.exp(-bd)) + EPS)).astype(F32)


def nms_obb(c: dict, iou_thr: float, max_det: int = 300, cap: int = 2048):
    """Fast-NMS over decoded OBB candidates c (dict from decode_obb_all): rank j is dropped
    iff a higher rank of its class has probiou >= thr with it.  Returns (indices into c of
    the survivors in output order, n_raw)."""
    n_raw = len(c["score"])
    order = rank_order(c["score"], c["anchor"])[:cap]
    rb, th, cl = c["rbox"][order], c["theta"][order], c["cls"][order]
    A, B, C = covariance(rb[:, 2], rb[:, 3], th)
    thr = F32(iou_thr)
    dead = np.zeros(len(order), bool)
    for k in np.unique(cl):
        mem = np.nonzero(cl == k)[0]               # rank order within the class
        if len(mem) < 2:
            continue
        i, j = mem[:, None], mem[None, :]
        iou = probiou(rb[i, 0], rb[i, 1], A[i], B[i], C[i], rb[j, 0], rb[j, 1], A[j], B[j], C[j])
        hit = np.triu(iou >= thr, 1)               # [earlier, later]
        dead[mem] = hit.any(axis=0)
    keep = order[~dead][:max_det]
    return np.asarray(keep, np.int64), n_raw


def detect_obb(heads, nc: int, conf: float = 0.25, iou: float = 0.45, max_det: int = 300,
               cap: int = 2048):
    """decode_obb + fast-NMS for one image -> dict with arrays in survivor order."""
    c = decode_obb_all(heads, nc, conf)
    keep, n_raw = nms_obb(c, iou, max_det, cap)
    out = {k: v[keep] for k, v in c.items()}
    out["n_raw"] = n_raw
    return out


# ----------------------------------------------------------------------------- masks
def masks(proto: np.ndarray, coef: np.ndarray, boxes: np.ndarray, net_h: int, net_w: int) -> np.ndarray:
    """proto [Ph,Pw,nm], coef [n,nm], boxes [n,4] in net pixels -> u8 [n,Ph,Pw]."""
    Ph, Pw, nm = proto.shape
    rx, ry = F32(Pw) / F32(net_w), F32(Ph) / F32(net_h)
    logit = np.einsum("hwc,nc->nhw", proto.astype(F32), coef.astype(F32)).astype(F32)
    ys = np.arange(Ph, dtype=F32)[None, :, None]
    xs = np.arange(Pw, dtype=F32)[None, None, :]
    bx1 = (boxes[:, 0] * rx)[:, None, None]
    by1 = (boxes[:, 1] * ry)[:, None, None]
    bx2 = (boxes[:, 2] * rx)[:, None, None]
    by2 = (boxes[:, 3] * ry)[:, None, None]
    inside = (xs >= bx1) & (xs < bx2) & (ys >= by1) & (ys < by2)
    return (inside & (logit > 0)).astype(np.uint8)


# ----------------------------------------------------------------------------- matching
def box_iou(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Plain IoU between matched rows of a and b ([n,4] each), float64."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    iw = np.clip(np.minimum(a[:, 2], b[:, 2]) - np.maximum(a[:, 0], b[:, 0]), 0, None)
    ih = np.clip(np.minimum(a[:, 3], b[:, 3]) - np.maximum(a[:, 1], b[:, 1]), 0, None)
    inter = iw * ih
    ua = (a[:, 2] - a[:, 0]) * (a[:, 3] - a[:, 1]) + (b[:, 2] - b[:, 0]) * (b[:, 3] - b[:, 1]) - inter
    return np.where(ua > 0, inter / np.where(ua > 0, ua, 1), 1.0)


def rel_err(gpu: np.ndarray, ref: np.ndarray) -> float:
    """max|gpu - ref| / (max|ref| + 1e-6), the reference's per-op metric (test/compare.py:21-25)."""
    ref = ref.astype(np.float64)
    return float(np.abs(gpu.astype(np.float64) - ref).max() / (np.abs(ref).max() + 1e-6))


def match_e2e(ref: dict, got: dict, ref_masks=None, got_masks=None, score_gate: float = 0.27):
    """The reference's end-to-end matching (test/compare_seg.py:61-100): every reference
    detection, in its survivor order, takes the unused same-class detection of `got` with
    the highest box IoU (first one on ties); IoU <= 0.8 leaves it unmatched, which counts as
    a failure when its score exceeds `score_gate`.  A matched pair fails if |dscore| > 0.02,
    a box corner moved more than 2 px, or (with masks) their mask IoU is below 0.95.
    `ref` / `got`: dicts with "box" [n,4], "score" [n], "cls" [n] (boxes in one coordinate
    system).  Returns a dict of counts and the per-pair |dscore|, corner and mask-IoU lists."""
    rb = np.asarray(ref["box"], np.float64)
    gb = np.asarray(got["box"], np.float64)
    rs, gs = np.asarray(ref["score"], np.float64), np.asarray(got["score"], np.float64)
    rc, gc = np.asarray(ref["cls"]).astype(int), np.asarray(got["cls"]).astype(int)
    used = np.zeros(len(gb), bool)
    out = {"n_ref": len(rb), "n_got": len(gb), "unmatched": 0, "unmatched_gated": 0, "pair_fail": 0,
           "dscore": [], "dbox": [], "mask_iou": []}
    for i in range(len(rb)):
        cand = np.nonzero((gc == rc[i]) & ~used)[0]
        best, bj = 0.0, -1
        if len(cand):
            a, b = rb[i], gb[cand]
            iw = np.clip(np.minimum(a[2], b[:, 2]) - np.maximum(a[0], b[:, 0]), 0, None)
            ih = np.clip(np.minimum(a[3], b[:, 3]) - np.maximum(a[1], b[:, 1]), 0, None)
            inter = iw * ih
            ua = (a[2] - a[0]) * (a[3] - a[1]) + (b[:, 2] - b[:, 0]) * (b[:, 3] - b[:, 1]) - inter
            iou = inter / np.maximum(ua, 1e-9)
            k = int(np.argmax(iou))
            if iou[k] > 0:
                best, bj = float(iou[k]), int(cand[k])
        if bj < 0 or best <= 0.8:
            out["unmatched"] += 1
            out["unmatched_gated"] += int(rs[i] > score_gate)
            continue
        used[bj] = True
        ds = abs(rs[i] - gs[bj])
        db = float(np.abs(rb[i] - gb[bj]).max())
        ok = ds <= 0.02 and db <= 2.0
        out["dscore"].append(ds)
        out["dbox"].append(db)
        if ref_masks is not None and got_masks is not None:
            inter = np.logical_and(ref_masks[i], got_masks[bj]).sum()
            union = np.logical_or(ref_masks[i], got_masks[bj]).sum()
            miou = float(inter) / max(int(union), 1)
            out["mask_iou"].append(miou)
            ok = ok and miou >= 0.95
        out["pair_fail"] += int(not ok)
    out["fails"] = out["unmatched_gated"] + out["pair_fail"]
    return out
