"""Seeded synthetic YOLOv8 / YOLO11 model directories in the reference's on-disk format.

The reference builds its model directory from an ultralytics checkpoint
(`export/export.py:583-729`).  No checkpoint and no ultralytics exist here, so this
module re-derives the same topology from the scale parameters (depth, width,
max_channels) and fills it with seeded random weights, then writes the identical
files the engine loads:

    model.graph   text graph, v2 header   (export/export.py:709-717)
    weights.f16   OHWI fp16 weights        (export/export.py:72-80)
    bias.f32      fp32 biases              (export/export.py:72-80)
    frame.u8/.txt optional raw BGR frame   (the reference's bus_raw.u8/.txt, :569-570)

Topology rules restated (file:line of the reference exporter they follow):
  * conv emission + OHWI packing + pad-to-8          export/export.py:83-145
  * ConvTranspose(k2,s2) -> 1x1 CONV to 4C + PS2     export/export.py:166-181
  * Bottleneck / C3k / C3k2(C2f) / SPPF / C2PSA      export/export.py:222-302
  * zero-copy concat planning, layer walk, heads      export/export.py:317-441
Module construction rules (ultralytics 8.4.x parse_model, restated): channel
c2 = ceil8(min(c2, max_ch) * width); repeats n = max(round(n * depth), 1) when n > 1;
C3k2 uses C3k blocks on scales m/l/x; Detect widths c2 = max(16, ch0 // 4, 64),
c3 = max(ch0, min(nc, 100)); Segment proto width = ceil8(min(256, max_ch) * width).

Weights: conv w ~ N(0, 1/fan_in), BatchNorm folded with gamma ~ U(0.5, 1.5),
beta ~ N(0, 0.1), eps 1e-3 (ultralytics BN eps).  BN running statistics are what BN
running statistics are in a trained model: the per-channel mean and variance of the
conv output, measured here on one seeded calibration frame while the graph is emitted
(with mean 0 / var 1 instead, activations shrink ~0.4x per layer and the head logits
collapse to a constant, so class argmax and NMS order would be decided by rounding
noise).
Head finals (plain Conv2d) use torch's default bias U(+-1/sqrt(fan_in)); the box
final bias is 1.0 (Detect.bias_init) and the class final bias is `cls_bias`
(a fixed prior chosen so random-init weights give tens-to-hundreds of candidates
at conf 0.25 instead of none or all 8,400).
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass, field

import numpy as np

ACT_NONE, ACT_SILU = 0, 1
BN_EPS = 1e-3

# (depth, width, max_channels) per scale
SCALES = {
    "yolo11": {"n": (0.50, 0.25, 1024), "s": (0.50, 0.50, 1024), "m": (0.50, 1.00, 512),
               "l": (1.00, 1.00, 512), "x": (1.00, 1.50, 512)},
    "yolov8": {"n": (0.33, 0.25, 1024), "s": (0.33, 0.50, 1024), "m": (0.67, 0.75, 768),
               "l": (1.00, 1.00, 512), "x": (1.00, 1.25, 512)},
}

# layer tables: (from, repeats, module, args) -- the public yolo11.yaml / yolov8.yaml
LAYERS = {
    "yolo11": [
        (-1, 1, "Conv", [64, 3, 2]), (-1, 1, "Conv", [128, 3, 2]),
        (-1, 2, "C3k2", [256, False, 0.25]), (-1, 1, "Conv", [256, 3, 2]),
        (-1, 2, "C3k2", [512, False, 0.25]), (-1, 1, "Conv", [512, 3, 2]),
        (-1, 2, "C3k2", [512, True]), (-1, 1, "Conv", [1024, 3, 2]),
        (-1, 2, "C3k2", [1024, True]), (-1, 1, "SPPF", [1024, 5]),
        (-1, 2, "C2PSA", [1024]),
        (-1, 1, "Upsample", []), ([-1, 6], 1, "Concat", []), (-1, 2, "C3k2", [512, False]),
        (-1, 1, "Upsample", []), ([-1, 4], 1, "Concat", []), (-1, 2, "C3k2", [256, False]),
        (-1, 1, "Conv", [256, 3, 2]), ([-1, 13], 1, "Concat", []), (-1, 2, "C3k2", [512, False]),
        (-1, 1, "Conv", [512, 3, 2]), ([-1, 10], 1, "Concat", []), (-1, 2, "C3k2", [1024, True]),
    ],
    "yolov8": [
        (-1, 1, "Conv", [64, 3, 2]), (-1, 1, "Conv", [128, 3, 2]),
        (-1, 3, "C2f", [128, True]), (-1, 1, "Conv", [256, 3, 2]),
        (-1, 6, "C2f", [256, True]), (-1, 1, "Conv", [512, 3, 2]),
        (-1, 6, "C2f", [512, True]), (-1, 1, "Conv", [1024, 3, 2]),
        (-1, 3, "C2f", [1024, True]), (-1, 1, "SPPF", [1024, 5]),
        (-1, 1, "Upsample", []), ([-1, 6], 1, "Concat", []), (-1, 3, "C2f", [512]),
        (-1, 1, "Upsample", []), ([-1, 4], 1, "Concat", []), (-1, 3, "C2f", [256]),
        (-1, 1, "Conv", [256, 3, 2]), ([-1, 12], 1, "Concat", []), (-1, 3, "C2f", [512]),
        (-1, 1, "Conv", [512, 3, 2]), ([-1, 9], 1, "Concat", []), (-1, 3, "C2f", [1024]),
    ],
}
HEAD_FROM = {"yolo11": [16, 19, 22], "yolov8": [15, 18, 21]}


def ceil8(x: float) -> int:
    return int(math.ceil(x / 8) * 8)


def autopad(k: int) -> int:
    return k // 2


@dataclass
class ConvSpec:
    """One convolution of the module tree: c1 -> c2, k x k, stride s, groups g."""
    c1: int
    c2: int
    k: int = 1
    s: int = 1
    g: int = 1
    act: int = ACT_SILU
    bn: bool = True             # ultralytics Conv (BN folded) vs plain nn.Conv2d
    bias: float | None = None   # constant bias override (Detect.bias_init)
    name: str = ""              # module path in an ultralytics state_dict ("model.2.m.0.cv1")


def fold_bn(w: np.ndarray, gamma: np.ndarray, beta: np.ndarray, mean: np.ndarray, var: np.ndarray):
    """BatchNorm folded into the preceding conv (eval mode, eps BN_EPS): w [O, ...], -> (w', b')."""
    scale = gamma / np.sqrt(var + np.float32(BN_EPS))
    return (w * scale.reshape((-1,) + (1,) * (w.ndim - 1))).astype(np.float32), (beta - mean * scale).astype(np.float32)


def _conv_nhwc(x: np.ndarray, w: np.ndarray, s: int, p: int, g: int) -> np.ndarray:
    """Calibration-pass convolution: x [N,H,W,Cin] fp32, w [O, Cin/g, k, k] -> [N,Ho,Wo,O], no bias."""
    N, H, W, Cin = x.shape
    O, ig, k, _ = w.shape
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    xp = np.pad(x, ((0, 0), (p, p), (p, p), (0, 0))) if p else x
    if g == 1:
        taps = [xp[:, ky:ky + s * (Ho - 1) + 1:s, kx:kx + s * (Wo - 1) + 1:s, :]
                for ky in range(k) for kx in range(k)]
        cols = np.concatenate(taps, axis=3).reshape(N * Ho * Wo, k * k * Cin)
        return (cols @ w.transpose(0, 2, 3, 1).reshape(O, -1).T).reshape(N, Ho, Wo, O)
    y = np.zeros((N, Ho, Wo, O), np.float32)
    for ky in range(k):
        for kx in range(k):
            y += xp[:, ky:ky + s * (Ho - 1) + 1:s, kx:kx + s * (Wo - 1) + 1:s, :] * w[:, 0, ky, kx]
    return y


def _silu(y):
    return y / (np.float32(1.0) + np.exp(-y))


class ModelGraph:
    """Graph under construction: buffers [H,W,C], channel-slice tensors, ops, weights.

    With a calibration frame, every emitted op is also evaluated (fp32, batch 1) so each
    BatchNorm can be folded with the running statistics of its own conv output."""

    def __init__(self, seed: int, calib: np.ndarray | None = None, source=None, record: dict | None = None):
        # source: parameters come from a checkpoint (convert.StateDictSource) instead of the
        # seeded generator; record: the generator's unfolded parameters are stored into this
        # dict under ultralytics state_dict names (the inverse of a checkpoint import)
        self.source = source
        self.record = record
        self.rng = np.random.default_rng(seed)
        self.bufs: list[tuple[int, int, int]] = []
        self.tens: list[tuple[int, int, int]] = []
        self.ops: list[tuple] = []
        self.w16: list[np.ndarray] = []
        self.b32: list[np.ndarray] = []
        self.woff = 0
        self.boff = 0
        self.cal = calib is not None
        self.bv: list[np.ndarray] = []       # calibration values per buffer
        self._calib0 = calib

    # -- storage ------------------------------------------------------------------
    def buf(self, H, W, C):
        self.bufs.append((H, W, C))
        if self.cal:
            self.bv.append(np.zeros((self._calib0.shape[0], H, W, C), np.float32))
        return len(self.bufs) - 1

    def ten(self, b, coff, C):
        assert coff + C <= self.bufs[b][2]
        self.tens.append((b, coff, C))
        return len(self.tens) - 1

    def newt(self, H, W, C):
        t = self.ten(self.buf(H, W, C), 0, C)
        if self.cal and t == 0:
            self.val(0)[...] = self._calib0
        return t

    def shape(self, t):
        b, _, C = self.tens[t]
        H, W, _ = self.bufs[b]
        return H, W, C

    def val(self, t) -> np.ndarray:
        b, coff, C = self.tens[t]
        return self.bv[b][..., coff:coff + C]

    def add_weight(self, w_ohwi: np.ndarray, b: np.ndarray):
        w = np.ascontiguousarray(w_ohwi, dtype=np.float16).ravel()
        b = np.ascontiguousarray(b, dtype=np.float32).ravel()
        woff, boff = self.woff, self.boff
        self.w16.append(w)
        self.b32.append(b)
        self.woff += w.size
        self.boff += b.size
        return woff, boff

    # -- random parameters ----------------------------------------------------------
    def _conv_params(self, sp: ConvSpec, x_val: np.ndarray | None):
        """Returns torch-layout weight [O, I/g, k, k] (fp32, BN folded) and bias [O]."""
        if self.source is not None:
            return self.source.conv(sp)
        ig = sp.c1 // sp.g
        fan_in = ig * sp.k * sp.k
        w = self.rng.standard_normal((sp.c2, ig, sp.k, sp.k), dtype=np.float32) / np.float32(math.sqrt(fan_in))
        if sp.bn:
            gamma = self.rng.uniform(0.5, 1.5, sp.c2).astype(np.float32)
            beta = (self.rng.standard_normal(sp.c2, dtype=np.float32) * np.float32(0.1))
            mean = np.zeros(sp.c2, np.float32)
            var = np.ones(sp.c2, np.float32)
            if x_val is not None:
                z = _conv_nhwc(x_val[..., :sp.c1], w, sp.s, autopad(sp.k), sp.g)
                mean = z.mean(axis=(0, 1, 2)).astype(np.float32)
                var = z.var(axis=(0, 1, 2)).astype(np.float32)
            if self.record is not None:
                self.record.update({f"{sp.name}.conv.weight": w.copy(), f"{sp.name}.bn.weight": gamma,
                                    f"{sp.name}.bn.bias": beta, f"{sp.name}.bn.running_mean": mean,
                                    f"{sp.name}.bn.running_var": var})
            w, b = fold_bn(w, gamma, beta, mean, var)
        else:
            bound = 1.0 / math.sqrt(fan_in)
            b = self.rng.uniform(-bound, bound, sp.c2).astype(np.float32)
        if sp.bias is not None:
            b = np.full(sp.c2, sp.bias, np.float32)
        if self.record is not None and not sp.bn:
            self.record.update({f"{sp.name}.weight": w.copy(), f"{sp.name}.bias": b.copy()})
        return w.astype(np.float32), b.astype(np.float32)

    def _eval_conv(self, x, w, b, sp: ConvSpec, out):
        """Calibration value of a conv output (fp32 weights, unpadded channels)."""
        if not self.cal:
            return
        y = _conv_nhwc(self.val(x)[..., :sp.c1], w, sp.s, autopad(sp.k), sp.g) + b
        if sp.act == ACT_SILU:
            y = _silu(y)
        o = self.val(out)
        o[...] = 0.0
        o[..., :sp.c2] = y

    # -- op emitters (export/export.py:83-220) ---------------------------------------
    def conv(self, x, sp: ConvSpec, out=None):
        H, W, Cin = self.shape(x)
        assert sp.c1 == Cin, (sp, Cin)
        assert sp.g == 1 or (sp.g == Cin and sp.c2 == Cin)
        p = autopad(sp.k)
        Ho, Wo = (H + 2 * p - sp.k) // sp.s + 1, (W + 2 * p - sp.k) // sp.s + 1
        if out is None:
            out = self.newt(Ho, Wo, sp.c2)
        assert self.shape(out) == (Ho, Wo, sp.c2), (self.shape(out), (Ho, Wo, sp.c2))
        w, b = self._conv_params(sp, self.val(x) if self.cal else None)
        woff, boff = self.add_weight(w.transpose(0, 2, 3, 1), b)   # OHWI
        self.ops.append(("CONV", x, out, sp.k, sp.s, p, sp.g, sp.act, Cin, sp.c2, woff, boff))
        self._eval_conv(x, w, b, sp, out)
        return out

    def conv_pad(self, x, sp: ConvSpec, cpad=None):
        """Conv whose output channels are zero-padded to a multiple of 8 (zero weight rows,
        zero bias), and whose input may carry extra zero channels (zero weight columns)."""
        if cpad is None:
            cpad = ceil8(sp.c2)
        H, W, Cin = self.shape(x)
        dw = sp.g > 1
        if sp.c2 == cpad and sp.c1 == Cin:
            return self.conv(x, sp)
        p = autopad(sp.k)
        Ho, Wo = (H + 2 * p - sp.k) // sp.s + 1, (W + 2 * p - sp.k) // sp.s + 1
        out = self.newt(Ho, Wo, cpad)
        w0, b0 = self._conv_params(sp, self.val(x) if self.cal else None)
        self._eval_conv(x, w0, b0, sp, out)
        w, b = w0.transpose(0, 2, 3, 1), b0
        if not dw and sp.c1 < Cin:
            w = np.concatenate([w, np.zeros(w.shape[:3] + (Cin - sp.c1,), w.dtype)], 3)
        w = np.concatenate([w, np.zeros((cpad - sp.c2,) + w.shape[1:], w.dtype)], 0)
        b = np.concatenate([b, np.zeros(cpad - sp.c2, np.float32)])
        woff, boff = self.add_weight(w, b)
        self.ops.append(("CONV", x, out, sp.k, sp.s, p, cpad if dw else 1, sp.act,
                         cpad if dw else Cin, cpad, woff, boff))
        return out

    def add(self, a, b, out):
        assert self.shape(a) == self.shape(b) == self.shape(out)
        self.ops.append(("ADD", a, b, out))
        if self.cal:
            self.val(out)[...] = self.val(a) + self.val(b)
        return out

    def maxpool5(self, x, out):
        self.ops.append(("MAXPOOL5", x, out))
        if self.cal:
            v = self.val(x)
            _, H, W, _ = v.shape
            vp = np.pad(v, ((0, 0), (2, 2), (2, 2), (0, 0)), constant_values=-np.inf)
            m = np.full(v.shape, -np.inf, np.float32)
            for dy in range(5):
                for dx in range(5):
                    m = np.maximum(m, vp[:, dy:dy + H, dx:dx + W])
            self.val(out)[...] = m
        return out

    def upsample2(self, x, out):
        H, W, C = self.shape(x)
        assert self.shape(out) == (2 * H, 2 * W, C)
        self.ops.append(("UPSAMPLE2", x, out))
        if self.cal:
            self.val(out)[...] = self.val(x).repeat(2, 1).repeat(2, 2)
        return out

    def copyc(self, x, out):
        assert self.shape(x) == self.shape(out)
        self.ops.append(("COPYC", x, out))
        if self.cal:
            self.val(out)[...] = self.val(x)
        return out

    def conv_transpose2(self, x, c_out: int, out=None, name: str = ""):
        """ConvTranspose2d(Cin -> C, k=2, s=2) emitted as a 1x1 CONV to 4C (quadrant-major
        rows q*C + o, q = 2*di + dj) followed by PS2 (export/export.py:166-181)."""
        H, W, Cin = self.shape(x)
        C = c_out
        if self.source is not None:
            wt, bt = self.source.conv_transpose(name, Cin, C)
        else:
            wt = self.rng.standard_normal((Cin, C, 2, 2), dtype=np.float32) / np.float32(math.sqrt(Cin))
            bound = 1.0 / math.sqrt(Cin)
            bt = self.rng.uniform(-bound, bound, C).astype(np.float32)
            if self.record is not None:
                self.record.update({f"{name}.weight": wt.copy(), f"{name}.bias": bt.copy()})
        self.last_convt = (wt.copy(), bt.copy())
        w = wt.transpose(2, 3, 1, 0).reshape(4 * C, 1, 1, Cin)
        b = np.tile(bt, 4)
        woff, boff = self.add_weight(w, b)
        up4 = self.newt(H, W, 4 * C)
        self.ops.append(("CONV", x, up4, 1, 1, 0, 1, ACT_NONE, Cin, 4 * C, woff, boff))
        if out is None:
            out = self.newt(2 * H, 2 * W, C)
        self.ops.append(("PS2", up4, out))
        if self.cal:
            u = self.val(x) @ w.reshape(4 * C, Cin).T + b
            o = self.val(out)
            for di in range(2):
                for dj in range(2):
                    q = 2 * di + dj
                    o[:, di::2, dj::2, :] = u[..., q * C:(q + 1) * C]
        return out

    def gap(self, x, out):
        """Global average pool [H,W,C] -> [1,1,C] (export/export.py:199-202)."""
        H, W, C = self.shape(x)
        assert self.shape(out) == (1, 1, C)
        self.ops.append(("GAP", x, out))
        if self.cal:
            self.val(out)[...] = self.val(x).mean(axis=(1, 2), keepdims=True)
        return out

    def linear(self, x, O: int, name: str = ""):
        """nn.Linear(I, O) on a [1,1,I] tensor as a 1x1 CONV (export/export.py:208-217):
        weights N(0, 1/I), bias U(+-1/sqrt(I)) (torch's default bias range), no activation."""
        H, W, I = self.shape(x)
        assert (H, W) == (1, 1)
        out = self.newt(1, 1, O)
        if self.source is not None:
            w, b = self.source.linear(name, I, O)
            w = w.reshape(O, 1, 1, I)
        else:
            w = self.rng.standard_normal((O, 1, 1, I), dtype=np.float32) / np.float32(math.sqrt(I))
            bound = 1.0 / math.sqrt(I)
            b = self.rng.uniform(-bound, bound, O).astype(np.float32)
            if self.record is not None:
                self.record.update({f"{name}.weight": w.reshape(O, I).copy(), f"{name}.bias": b.copy()})
        woff, boff = self.add_weight(w, b)
        self.ops.append(("CONV", x, out, 1, 1, 0, 1, ACT_NONE, I, O, woff, boff))
        if self.cal:
            self.val(out)[...] = self.val(x) @ w.reshape(O, I).T + b
        return out

    def softmax(self, x, out):
        """Channel softmax of a [1,1,C] tensor (export/export.py:204-206)."""
        assert self.shape(x) == self.shape(out)
        self.ops.append(("SOFTMAX", x, out))
        if self.cal:
            v = self.val(x)
            e = np.exp(v - v.max(axis=-1, keepdims=True))
            self.val(out)[...] = e / e.sum(axis=-1, keepdims=True)
        return out

    # -- serialisation (export/export.py:709-719) -------------------------------------
    def write(self, path: str, task: str, nc: int, imgsz: int):
        os.makedirs(path, exist_ok=True)
        with open(os.path.join(path, "model.graph"), "w") as f:
            f.write("YOLO11GRAPH 2\n")
            f.write(f"TASK {task} {nc} {imgsz}\n")
            f.write(f"{len(self.bufs)} {len(self.tens)} {len(self.ops)}\n")
            for (H, W, C) in self.bufs:
                f.write(f"B {H} {W} {C}\n")
            for (b, coff, C) in self.tens:
                f.write(f"T {b} {coff} {C}\n")
            for op in self.ops:
                f.write(" ".join(str(v) for v in op) + "\n")
        np.concatenate(self.w16).astype(np.float16).tofile(os.path.join(path, "weights.f16"))
        np.concatenate(self.b32).astype(np.float32).tofile(os.path.join(path, "bias.f32"))


# ---------------------------------------------------------------------------------------
# module decomposition (export/export.py:222-302)

def _bottleneck(g, x, c1, c2, shortcut, e, out, name=""):
    c_ = int(c2 * e)
    t = g.conv(x, ConvSpec(c1, c_, 3, name=f"{name}.cv1"))
    g.conv(t, ConvSpec(c_, c2, 3, name=f"{name}.cv2"), out=out)
    if shortcut and c1 == c2:
        g.add(out, x, out)
    return out


def _c3k(g, x, c1, c2, n, shortcut, out, name=""):
    H, W, _ = g.shape(x)
    c_ = int(c2 * 0.5)
    cat = g.buf(H, W, 2 * c_)
    cur = g.conv(x, ConvSpec(c1, c_, 1, name=f"{name}.cv1"))
    for j in range(n):
        dst = g.ten(cat, 0, c_) if j == n - 1 else g.newt(H, W, c_)
        _bottleneck(g, cur, c_, c_, shortcut, 1.0, dst, f"{name}.m.{j}")
        cur = dst
    g.conv(x, ConvSpec(c1, c_, 1, name=f"{name}.cv2"), out=g.ten(cat, c_, c_))
    g.conv(g.ten(cat, 0, 2 * c_), ConvSpec(2 * c_, c2, 1, name=f"{name}.cv3"), out=out)
    return out


def _c2f(g, x, c1, c2, n, c3k, e, shortcut, v11, out, name=""):
    """C3k2 (v11) / C2f (v8): cv1 -> split -> n blocks chained -> concat -> cv2."""
    H, W, _ = g.shape(x)
    c = int(c2 * e)
    cat = g.buf(H, W, (2 + n) * c)
    g.conv(x, ConvSpec(c1, 2 * c, 1, name=f"{name}.cv1"), out=g.ten(cat, 0, 2 * c))
    prev = g.ten(cat, c, c)
    for j in range(n):
        dst = g.ten(cat, (2 + j) * c, c)
        if c3k:
            _c3k(g, prev, c, c, 2, shortcut, dst, f"{name}.m.{j}")
        else:
            # C3k2's Bottleneck keeps e=0.5; C2f's uses e=1.0
            _bottleneck(g, prev, c, c, shortcut, 0.5 if v11 else 1.0, dst, f"{name}.m.{j}")
        prev = dst
    return g.conv(g.ten(cat, 0, (2 + n) * c), ConvSpec((2 + n) * c, c2, 1, name=f"{name}.cv2"), out=out)


def _sppf(g, x, c1, c2, out, name=""):
    H, W, _ = g.shape(x)
    c_ = c1 // 2
    cat = g.buf(H, W, 4 * c_)
    g.conv(x, ConvSpec(c1, c_, 1, name=f"{name}.cv1"), out=g.ten(cat, 0, c_))
    for j in range(3):
        g.maxpool5(g.ten(cat, j * c_, c_), g.ten(cat, (j + 1) * c_, c_))
    return g.conv(g.ten(cat, 0, 4 * c_), ConvSpec(4 * c_, c2, 1, name=f"{name}.cv2"), out=out)


def _psablock(g, xio, c, name=""):
    """x = x + attn(x); x = x + ffn(x), in place on view xio (export/export.py:269-290)."""
    H, W, C = g.shape(xio)
    heads = c // 64
    hd = c // heads
    kd = int(hd * 0.5)
    per = 2 * kd + hd
    qkv = g.conv(xio, ConvSpec(c, c + 2 * kd * heads, 1, act=ACT_NONE, name=f"{name}.attn.qkv"))
    qb = g.tens[qkv][0]
    vbuf = g.buf(H, W, C)
    for h in range(heads):
        g.copyc(g.ten(qb, h * per + 2 * kd, hd), g.ten(vbuf, h * hd, hd))
    vt = g.ten(vbuf, 0, C)
    ao = g.newt(H, W, C)
    g.ops.append(("ATTN", qkv, ao, heads, kd, hd))
    if g.cal:
        nb = g.val(qkv).shape[0]
        t = g.val(qkv).reshape(nb, H * W, heads, per)
        o = np.empty((nb, H * W, heads * hd), np.float32)
        for i in range(nb):
            for h in range(heads):
                q, k, v = t[i, :, h, :kd], t[i, :, h, kd:2 * kd], t[i, :, h, 2 * kd:]
                sc = (q @ k.T) * np.float32(kd ** -0.5)
                e = np.exp(sc - sc.max(1, keepdims=True))
                o[i, :, h * hd:(h + 1) * hd] = (e / e.sum(1, keepdims=True)) @ v
        g.val(ao)[...] = o.reshape(nb, H, W, heads * hd)
    pe = g.conv(vt, ConvSpec(c, c, 3, g=c, act=ACT_NONE, name=f"{name}.attn.pe"))
    g.add(ao, pe, ao)
    pr = g.conv(ao, ConvSpec(c, c, 1, act=ACT_NONE, name=f"{name}.attn.proj"))
    g.add(xio, pr, xio)
    f1 = g.conv(xio, ConvSpec(c, 2 * c, 1, name=f"{name}.ffn.0"))
    f2 = g.conv(f1, ConvSpec(2 * c, c, 1, act=ACT_NONE, name=f"{name}.ffn.1"))
    g.add(xio, f2, xio)
    return xio


def _c2psa(g, x, c1, c2, n, out, name=""):
    H, W, _ = g.shape(x)
    c = int(c1 * 0.5)
    cat = g.buf(H, W, 2 * c)
    g.conv(x, ConvSpec(c1, 2 * c, 1, name=f"{name}.cv1"), out=g.ten(cat, 0, 2 * c))
    b = g.ten(cat, c, c)
    for j in range(n):
        _psablock(g, b, c, f"{name}.m.{j}")
    return g.conv(g.ten(cat, 0, 2 * c), ConvSpec(2 * c, c1, 1, name=f"{name}.cv2"), out=out)


# ---------------------------------------------------------------------------------------

@dataclass
class ModelInfo:
    arch: str
    scale: str
    task: str
    nc: int
    imgsz: int
    graph: ModelGraph = field(repr=False)
    seed: int = 0
    cls_bias: float = 0.0


def build_model(arch: str = "yolo11", scale: str = "n", task: str = "detect", nc: int = 80,
                imgsz: int = 640, seed: int = 0, cls_bias: float = -3.0, nm: int = 32,
                calibrate: bool = True, source=None, record: dict | None = None) -> ModelInfo:
    """Builds the flat op graph of a seeded random-init YOLO model (export/export.py:317-441)."""
    assert arch in SCALES and scale in SCALES[arch], (arch, scale)
    assert task in ("detect", "segment", "obb", "classify"), task
    cls_task = task == "classify"
    assert not cls_task or arch == "yolo11", "classify models: yolo11 only"

    assert imgsz % 32 == 0
    depth, width, max_ch = SCALES[arch][scale]
    v11 = arch == "yolo11"
    S = imgsz
    calib = calibration_frames(S, seed) if calibrate and source is None else None
    g = ModelGraph(seed, calib, source, record)
    x0 = g.newt(S, S, 3)

    # resolve module args (parse_model rules)
    layers = []
    ch, hw = {-1: 3}, {-1: S}
    # yolo11-cls: the detect backbone's layers 0-8, then C2PSA (no SPPF, no neck), then
    # the Classify head (docs/specs/cls.md:29-41)
    table = LAYERS[arch][:9] + [(-1, 2, "C2PSA", [1024])] if cls_task else LAYERS[arch]
    for i, (f, n, m, args) in enumerate(table):
        srcs = [(i - 1 if j == -1 else j) for j in ([f] if isinstance(f, int) else f)]
        n_ = max(round(n * depth), 1) if n > 1 else n
        c1 = ch[srcs[0]]
        ih = hw[srcs[0]]
        spec = {"m": m, "srcs": srcs}
        if m in ("Conv", "C3k2", "C2f", "SPPF", "C2PSA"):
            c2 = ceil8(min(args[0], max_ch) * width)
            spec.update(c1=c1, c2=c2, n=n_)
            if m == "Conv":
                spec.update(k=args[1], s=args[2])
                hw[i] = (ih + 2 * autopad(args[1]) - args[1]) // args[2] + 1
            else:
                hw[i] = ih
            if m == "C3k2":
                spec.update(c3k=bool(args[1]) or scale in "mlx",
                            e=args[2] if len(args) > 2 else 0.5)
            if m == "C2f":
                spec.update(shortcut=bool(args[1]) if len(args) > 1 else False)
            ch[i] = c2
        elif m == "Upsample":
            ch[i], hw[i] = c1, ih * 2
        elif m == "Concat":
            ch[i], hw[i] = sum(ch[s] for s in srcs), ih
        layers.append(spec)
    n_body = len(layers)

    # concat planning: producers write straight into their cat-buffer slice
    catbuf, feed, feed_copy = {}, {}, {}
    for i, sp in enumerate(layers):
        if sp["m"] != "Concat":
            continue
        catbuf[i] = g.buf(hw[i], hw[i], ch[i])
        off = 0
        for s in sp["srcs"]:
            if s in feed or s < 0 or layers[s]["m"] == "Concat":
                feed_copy.setdefault(i, []).append((s, off))
            else:
                feed[s] = (catbuf[i], off, ch[s])
            off += ch[s]

    outs = {-1: x0}
    for i, sp in enumerate(layers):
        m = sp["m"]
        xin = outs[sp["srcs"][0]]
        dst = g.ten(*feed[i]) if i in feed else None
        mn = f"model.{i}"
        if m == "Conv":
            y = g.conv(xin, ConvSpec(sp["c1"], sp["c2"], sp["k"], sp["s"], name=mn), out=dst)
        elif m == "C2PSA":
            y = _c2psa(g, xin, sp["c1"], sp["c2"], sp["n"], dst, mn)
        elif m == "SPPF":
            y = _sppf(g, xin, sp["c1"], sp["c2"], dst, mn)
        elif m == "C3k2":
            y = _c2f(g, xin, sp["c1"], sp["c2"], sp["n"], sp["c3k"], sp["e"], True, True, dst, mn)
        elif m == "C2f":
            y = _c2f(g, xin, sp["c1"], sp["c2"], sp["n"], False, 0.5, sp["shortcut"], False, dst, mn)
        elif m == "Upsample":
            y = g.upsample2(xin, dst if dst is not None else g.newt(hw[i], hw[i], ch[i]))
        else:
            for s, off in feed_copy.get(i, []):
                g.copyc(outs[s], g.ten(catbuf[i], off, ch[s]))
            y = g.ten(catbuf[i], 0, ch[i])
        outs[i] = y

    if cls_task:
        # Classify (export/export.py:391-398): Conv(c1, 1280, 1) -> GAP -> Linear(1280, nc)
        # -> softmax; the head width 1280 is fixed (docs/specs/cls.md:53-54)
        hn = f"model.{n_body}"
        h = g.conv(outs[n_body - 1], ConvSpec(ch[n_body - 1], 1280, 1, name=f"{hn}.conv"))
        gp = g.gap(h, g.newt(1, 1, 1280))
        logits = g.linear(gp, nc, f"{hn}.linear")
        g.softmax(logits, g.newt(1, 1, nc))
        return ModelInfo(arch, scale, task, nc, imgsz, g, seed, cls_bias)

    # Detect / Segment / OBB head (export/export.py:400-438)
    feats_idx = HEAD_FROM[arch]
    feats = [outs[j] for j in feats_idx]
    chs = [ch[j] for j in feats_idx]
    strides = [8, 16, 32]
    reg_max = 16
    c2h = max(16, chs[0] // 4, reg_max * 4)
    c3h = max(chs[0], min(nc, 100))
    ncpad = ceil8(nc)
    seg = task == "segment"
    obb = task == "obb"
    c4o = max(chs[0] // 4, 1)            # OBB angle branch width, ne = 1 (docs/specs/obb.md:60-61)
    hn = f"model.{n_body}"
    if seg:
        npr = ceil8(min(256, max_ch) * width)
        t = g.conv(feats[0], ConvSpec(chs[0], npr, 3, name=f"{hn}.proto.cv1"))
        t = g.conv_transpose2(t, npr, name=f"{hn}.proto.upsample")
        t = g.conv(t, ConvSpec(npr, npr, 3, name=f"{hn}.proto.cv2"))
        t_proto = g.conv(t, ConvSpec(npr, nm, 1, name=f"{hn}.proto.cv3"))
        c4 = max(chs[0] // 4, nm)
    for i, (f, cx, st) in enumerate(zip(feats, chs, strides)):
        bn_, cn_, an_ = f"{hn}.cv2.{i}", f"{hn}.cv3.{i}", f"{hn}.cv4.{i}"
        b = g.conv(f, ConvSpec(cx, c2h, 3, name=f"{bn_}.0"))
        b = g.conv(b, ConvSpec(c2h, c2h, 3, name=f"{bn_}.1"))
        b = g.conv(b, ConvSpec(c2h, 4 * reg_max, 1, act=ACT_NONE, bn=False, bias=1.0, name=f"{bn_}.2"))
        if v11:
            c = g.conv_pad(f, ConvSpec(cx, cx, 3, g=cx, name=f"{cn_}.0.0"))
            c = g.conv_pad(c, ConvSpec(cx, c3h, 1, name=f"{cn_}.0.1"))
            c = g.conv_pad(c, ConvSpec(c3h, c3h, 3, g=c3h, name=f"{cn_}.1.0"))
            c = g.conv_pad(c, ConvSpec(c3h, c3h, 1, name=f"{cn_}.1.1"))
        else:
            c = g.conv_pad(f, ConvSpec(cx, c3h, 3, name=f"{cn_}.0"))
            c = g.conv_pad(c, ConvSpec(c3h, c3h, 3, name=f"{cn_}.1"))
        c = g.conv_pad(c, ConvSpec(c3h, nc, 1, act=ACT_NONE, bn=False, bias=cls_bias, name=f"{cn_}.2"), ncpad)
        if seg:
            mc = g.conv(f, ConvSpec(cx, c4, 3, name=f"{an_}.0"))
            mc = g.conv(mc, ConvSpec(c4, c4, 3, name=f"{an_}.1"))
            mc = g.conv(mc, ConvSpec(c4, nm, 1, act=ACT_NONE, bn=False, name=f"{an_}.2"))
            g.ops.append(("DECODESEG", b, c, mc, st))
        elif obb:
            a = g.conv(f, ConvSpec(cx, c4o, 3, name=f"{an_}.0"))
            a = g.conv(a, ConvSpec(c4o, c4o, 3, name=f"{an_}.1"))
            a = g.conv_pad(a, ConvSpec(c4o, 1, 1, act=ACT_NONE, bn=False, name=f"{an_}.2"), 8)
            g.ops.append(("DECODEOBB", b, c, a, st))
        else:
            g.ops.append(("DECODE", b, c, st))
    if seg:
        g.ops.append(("MASKS", t_proto))
    return ModelInfo(arch, scale, task, nc, imgsz, g, seed, cls_bias)


def calibration_frames(S: int, seed: int) -> np.ndarray:
    """Two RGB [0,1] frames for the BN statistics: a full S x S frame and a letterbox-shaped
    one (content 3/4 of the height between two 114-gray bands), so the statistics cover
    both padded and unpadded inputs."""
    full = synth_frame(S, S, 50, seed + 1000)
    nh = (3 * S // 4) // 2 * 2
    boxed = np.full((S, S, 3), 114, np.uint8)
    top = (S - nh) // 2
    boxed[top:top + nh] = synth_frame(nh, S, 20, seed + 1001)
    x = np.stack([full, boxed])[..., ::-1].astype(np.float32) / np.float32(255.0)
    return np.ascontiguousarray(x)


def write_model(path: str, arch="yolo11", scale="n", task="detect", nc=80, imgsz=640, seed=0,
                cls_bias=-3.0) -> ModelInfo:
    info = build_model(arch, scale, task, nc, imgsz, seed, cls_bias)
    info.graph.write(path, task, nc, imgsz)
    with open(os.path.join(path, "gen.txt"), "w") as f:
        f.write(f"{arch} {scale} {task} nc={nc} imgsz={imgsz} seed={seed} cls_bias={cls_bias}\n")
    return info


def write_single_conv(path: str, H: int, W: int, Cin: int, Cout: int, k: int, s: int,
                      act: int = ACT_SILU, seed: int = 0, dw: bool = False, residual: bool = False):
    """A one-op graph (input -> CONV [-> ADD residual]) used by the isolated conv sweep."""
    g = ModelGraph(seed)
    x = g.newt(H, W, Cin)
    sp = ConvSpec(Cin, Cout, k, s, g=Cin if dw else 1, act=act)
    y = g.conv(x, sp)
    if residual:
        g.add(y, x, y)
    g.write(path, "detect", 80, H if H == W else 0)
    return g


def write_copy(path: str, H: int, W: int, C: int):
    """A one-op graph: [H,W,C] -> COPYC -> [H,W,C] (a plain copy of known size)."""
    g = ModelGraph(0)
    x = g.newt(H, W, C)
    g.copyc(x, g.newt(H, W, C))
    g.add_weight(np.zeros((8, 1, 1, 1), np.float32), np.zeros(8, np.float32))
    g.write(path, "detect", 80, H if H == W else 0)
    return g


def write_attention(path: str, H: int, W: int, heads: int, kd: int = 32, hd: int = 64):
    """A one-op graph: qkv input [H,W,heads*(2kd+hd)] -> ATTN -> [H,W,heads*hd]."""
    g = ModelGraph(0)
    qkv = g.newt(H, W, heads * (2 * kd + hd))
    out = g.newt(H, W, heads * hd)
    g.ops.append(("ATTN", qkv, out, heads, kd, hd))
    g.add_weight(np.zeros((8, 1, 1, 1), np.float32), np.zeros(8, np.float32))
    g.write(path, "detect", 80, H if H == W else 0)
    return g


# ---------------------------------------------------------------------------------------
# synthetic frames: u8 BGR HWC

def synth_frame(h: int, w: int, n_rects: int, seed: int) -> np.ndarray:
    """Uniform noise plus `n_rects` seeded solid rectangles."""
    rng = np.random.default_rng(seed)
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    for _ in range(n_rects):
        x0, x1 = np.sort(rng.integers(0, w, 2))
        y0, y1 = np.sort(rng.integers(0, h, 2))
        img[y0:y1 + 1, x0:x1 + 1] = rng.integers(0, 256, 3, dtype=np.uint8)
    return img


def synth_polygons(h: int, w: int, n_polys: int, seed: int) -> np.ndarray:
    """Uniform noise plus `n_polys` seeded filled polygons (even-odd rule)."""
    rng = np.random.default_rng(seed)
    img = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    for _ in range(n_polys):
        nv = int(rng.integers(3, 8))
        cx, cy = rng.uniform(0, w), rng.uniform(0, h)
        rad = rng.uniform(0.03, 0.2) * min(h, w)
        ang = np.sort(rng.uniform(0, 2 * np.pi, nv))
        r = rad * rng.uniform(0.5, 1.0, nv)
        px, py = cx + r * np.cos(ang), cy + r * np.sin(ang)
        x0, x1 = int(max(0, px.min())), int(min(w - 1, px.max()))
        y0, y1 = int(max(0, py.min())), int(min(h - 1, py.max()))
        if x1 < x0 or y1 < y0:
            continue
        yy, xx = np.mgrid[y0:y1 + 1, x0:x1 + 1].astype(np.float32) + 0.5
        inside = np.zeros(yy.shape, bool)
        for a in range(nv):
            b = (a + 1) % nv
            xa, ya, xb, yb = px[a], py[a], px[b], py[b]
            cond = (ya > yy) != (yb > yy)
            xint = (xb - xa) * (yy - ya) / ((yb - ya) if yb != ya else 1e-9) + xa
            inside ^= cond & (xx < xint)
        img[y0:y1 + 1, x0:x1 + 1][inside] = rng.integers(0, 256, 3, dtype=np.uint8)
    return img


def write_frame(path: str, img: np.ndarray):
    """Raw BGR frame in the reference's bus_raw.u8 / bus_raw.txt layout."""
    img.tofile(os.path.join(path, "frame.u8"))
    with open(os.path.join(path, "frame.txt"), "w") as f:
        f.write(f"{img.shape[0]} {img.shape[1]}")


def count_ops(info_or_graph) -> dict:
    g = info_or_graph.graph if isinstance(info_or_graph, ModelInfo) else info_or_graph
    out: dict = {}
    for op in g.ops:
        out[op[0]] = out.get(op[0], 0) + 1
    out["total"] = len(g.ops)
    return out
