"""fp32 per-op graph interpreter (numpy) -- TEST INFRASTRUCTURE, see oracle/__init__.py.

Restates the reference's CPU per-op path `run_reference` (export/export.py:446-526) over
NHWC buffers instead of CHW ones.  Every buffer is float32 [B, H, W, C]; a tensor is a
channel slice of a buffer, exactly as in the engine (engine/engine.cu:31-78).  With
`round_fp16=True` each op's output is rounded through fp16 on write, which is the
reference's isolated-kernel baseline mode (export/export.py:451-460).

Per-op semantics (reference line they restate) and what pins each one:
  CONV      F.conv2d + SiLU, OHWI fp16 weights     export/export.py:467-474
            pinned vs torch.nn.functional.conv2d (library routine) and a brute-force
            loop on tiny shapes (tests/test_oracle_ops.py)
  ADD       elementwise                              export/export.py:475-476
  MAXPOOL5  max_pool2d(5, 1, 2)                      :477-478   pinned vs F.max_pool2d
  UPSAMPLE2 nearest x2                               :479-480   pinned vs F.interpolate
  PS2       quadrant pixel shuffle                   :481-489   pinned: 1x1 CONV + PS2
            equals F.conv_transpose2d(k2, s2) on the generator's own weights
  COPYC     channel copy                             :490-491
  ATTN      softmax(q^T k * kd^-1/2), v @ att^T      :492-500   pinned vs
            F.scaled_dot_product_attention and row-sum / permutation invariants
  GAP       mean over H, W                           :501-502   pinned vs
            F.adaptive_avg_pool2d(1)
  SOFTMAX   softmax over channels                    :503-504   pinned vs torch.softmax
            and the sum-to-one / shift-invariance properties
Epilogue order for a fused residual is act then +res (engine/engine.cu:471-478); the
unfused graph expresses the same thing as CONV followed by ADD.
"""
from __future__ import annotations

import numpy as np
from numpy.lib.stride_tricks import sliding_window_view

from .graphfile import Graph, Op

F32 = np.float32


def silu(y: np.ndarray) -> np.ndarray:
    return (y / (F32(1.0) + np.exp(-y))).astype(F32)


def conv_weights(g: Graph, op: Op) -> tuple[np.ndarray, np.ndarray]:
    """Weight [O, k, k, Cin/g] (fp16 values as fp32) and bias [O] of a CONV op."""
    ig = op.Cin // op.g
    n = op.Cout * op.k * op.k * ig
    w = g.weights[op.woff:op.woff + n].astype(F32).reshape(op.Cout, op.k, op.k, ig)
    b = g.bias[op.boff:op.boff + op.Cout].astype(F32)
    return w, b


def conv2d_nhwc(x: np.ndarray, w: np.ndarray, b: np.ndarray, s: int, p: int, groups: int,
                acc=F32, kperm: np.random.Generator | None = None) -> np.ndarray:
    """x [B,H,W,Cin] fp32, w [O,k,k,Cin/g] -> [B,Ho,Wo,O] fp32 (im2col over (ky,kx,ci)).
    `acc` is the arithmetic type of the products and sums (float32, or float64 to measure
    what fp32 accumulation alone changes); the result is float32 either way.  `kperm`
    (dense convs): the K terms are summed in an order drawn from this generator, the same
    sum in another valid fp32 order."""
    if acc is not F32:
        x, w, b = x.astype(acc), w.astype(acc), b.astype(acc)
    B, H, W, Cin = x.shape
    O, k, _, ig = w.shape
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    xp = np.pad(x, ((0, 0), (p, p), (p, p), (0, 0))) if p else x
    if groups == 1:
        if k == 1 and s == 1:
            cols = xp.reshape(-1, Cin)
        else:
            v = sliding_window_view(xp, (k, k), axis=(1, 2))[:, ::s, ::s][:, :Ho, :Wo]
            cols = np.ascontiguousarray(v.transpose(0, 1, 2, 4, 5, 3)).reshape(B * Ho * Wo, k * k * Cin)
        wk = w.reshape(O, -1)
        if kperm is not None:
            perm = kperm.permutation(wk.shape[1])
            cols, wk = cols[:, perm], wk[:, perm]
        y = cols @ wk.T
        y += b
        return y.reshape(B, Ho, Wo, O).astype(F32, copy=False)
    assert groups == Cin == O and ig == 1
    y = np.broadcast_to(b, (B, Ho, Wo, O)).astype(acc)
    for ky in range(k):
        for kx in range(k):
            y = y + xp[:, ky:ky + s * (Ho - 1) + 1:s, kx:kx + s * (Wo - 1) + 1:s, :] * w[:, ky, kx, 0]
    return y.astype(F32, copy=False)


def maxpool5(x: np.ndarray) -> np.ndarray:
    B, H, W, C = x.shape
    xp = np.pad(x, ((0, 0), (2, 2), (2, 2), (0, 0)), constant_values=-np.inf)
    return sliding_window_view(xp, (5, 5), axis=(1, 2)).max(axis=(-1, -2)).astype(F32)


def upsample2(x: np.ndarray) -> np.ndarray:
    return x.repeat(2, axis=1).repeat(2, axis=2)


def ps2(x: np.ndarray) -> np.ndarray:
    """[B,H,W,4C] with quadrant-major channel blocks q = 2*di + dj -> [B,2H,2W,C]."""
    B, H, W, C4 = x.shape
    C = C4 // 4
    y = np.empty((B, 2 * H, 2 * W, C), F32)
    for di in range(2):
        for dj in range(2):
            q = 2 * di + dj
            y[:, di::2, dj::2, :] = x[..., q * C:(q + 1) * C]
    return y


def gap(x: np.ndarray) -> np.ndarray:
    """[B, H, W, C] -> [B, 1, 1, C] mean over H and W (fp32)."""
    return x.mean(axis=(1, 2), keepdims=True, dtype=np.float64).astype(F32)


def softmax_ch(x: np.ndarray) -> np.ndarray:
    """Softmax over the channel axis of [B, 1, 1, C] (fp32 math, max-shifted)."""
    e = np.exp((x - x.max(axis=-1, keepdims=True)).astype(F32))
    return (e / e.sum(axis=-1, keepdims=True, dtype=F32)).astype(F32)


def attention(qkv: np.ndarray, heads: int, kd: int, hd: int, acc=F32) -> np.ndarray:
    """qkv [B,H,W,heads*(2kd+hd)] (per-head [q kd | k kd | v hd]) -> [B,H,W,heads*hd]
    (arithmetic in `acc`, result float32)."""
    B, H, W, _ = qkv.shape
    N = H * W
    per = 2 * kd + hd
    t = qkv.astype(acc).reshape(B, N, heads, per)
    out = np.empty((B, N, heads * hd), F32)
    scale = acc(kd ** -0.5)
    for b in range(B):
        for h in range(heads):
            q = t[b, :, h, :kd]
            k = t[b, :, h, kd:2 * kd]
            v = t[b, :, h, 2 * kd:]
            s = (q @ k.T) * scale
            s = s - s.max(axis=1, keepdims=True)
            e = np.exp(s)
            p = e / e.sum(axis=1, keepdims=True)
            out[b, :, h * hd:(h + 1) * hd] = p @ v
    return out.reshape(B, H, W, heads * hd)


class Interp:
    """Executes a parsed graph for a batch of B images.  `acc64`: conv and attention
    arithmetic in float64 (outputs still stored as float32, and through fp16 with
    `round_fp16`); `order_seed`: conv sums in another fp32 order.  Both measure how much a
    whole frame depends on the rounding of its fp32 accumulations."""

    def __init__(self, g: Graph, B: int = 1, round_fp16: bool = False, acc64: bool = False,
                 order_seed: int | None = None):
        self.g, self.B, self.round_fp16 = g, B, round_fp16
        self.acc = np.float64 if acc64 else F32
        # order_seed: every dense conv sums its K terms in a seeded random order
        self.kperm = None if order_seed is None else np.random.default_rng(order_seed)
        self.bufs = [np.zeros((B, H, W, C), F32) for (H, W, C) in g.bufs]
        self.heads_in: list = []   # DECODE / DECODESEG / DECODEOBB inputs, in op order

    def view(self, t: int) -> np.ndarray:
        b, coff, C = self.g.tens[t]
        return self.bufs[b][..., coff:coff + C]

    def write(self, t: int, val: np.ndarray):
        if self.round_fp16:
            val = val.astype(np.float16).astype(F32)
        self.view(t)[...] = val

    def set_input(self, x: np.ndarray):
        """x: [B, S, S, 3] (any float dtype; stored through fp16 like the engine input)."""
        self.view(0)[...] = np.asarray(x, F32).astype(np.float16).astype(F32)

    def run_op(self, op: Op) -> int | None:
        """Runs one op; returns the output tensor id (None for decode/mask ops)."""
        g = self.g
        if op.kind == "CONV":
            w, b = conv_weights(g, op)
            y = conv2d_nhwc(self.view(op.a), w, b, op.s, op.p, op.g, self.acc, self.kperm)
            if op.act == 1:
                y = silu(y)
            if op.b >= 0:    # fused residual: act then +res
                y = y + self.view(op.b)
            self.write(op.out, y)
            return op.out
        if op.kind == "ADD":
            self.write(op.out, self.view(op.a) + self.view(op.b))
            return op.out
        if op.kind == "MAXPOOL5":
            self.write(op.out, maxpool5(self.view(op.a)))
            return op.out
        if op.kind == "UPSAMPLE2":
            self.write(op.out, upsample2(self.view(op.a)))
            return op.out
        if op.kind == "PS2":
            self.write(op.out, ps2(self.view(op.a)))
            return op.out
        if op.kind == "COPYC":
            self.write(op.out, self.view(op.a).copy())
            return op.out
        if op.kind == "ATTN":
            self.write(op.out, attention(self.view(op.a), op.heads, op.kd, op.hd, self.acc))
            return op.out
        if op.kind == "GAP":     # export/export.py:501-502: mean over H, W
            self.write(op.out, gap(self.view(op.a)))
            return op.out
        if op.kind == "SOFTMAX":  # export/export.py:503-504: softmax over channels
            self.write(op.out, softmax_ch(self.view(op.a)))
            return op.out
        if op.kind in ("DECODE", "DECODESEG", "DECODEOBB"):
            # DECODESEG: coef = mask coefficients; DECODEOBB: coef = angle view
            coef = self.view(op.out).copy() if op.kind != "DECODE" else None
            self.heads_in.append((self.view(op.a).copy(), self.view(op.b).copy(), coef, op.stride))
            return None
        if op.kind == "MASKS":
            return None
        raise NotImplementedError(op.kind)

    def run(self, ops=None, on_op=None):
        self.heads_in = []
        for k, op in enumerate(ops if ops is not None else self.g.ops):
            t = self.run_op(op)
            if on_op is not None and t is not None:
                on_op(k, op, t)
        return self
