"""PyTorch fp32 per-op CPU path -- TEST INFRASTRUCTURE and bench.py's CPU baseline.

The reference checks its engine against a torch fp32 interpreter of the exported graph,
`run_reference` (export/export.py:446-526): channel-first buffers, one torch call per op,
fp16 weights read as fp32.  This module is this build's own form of that CPU path: the
whole batch at once in NCHW buffers, each conv's weight tensor prepared once at load (so a
timed frame measures only the per-op compute), and the frame's CPU pre/post from
`oracle.post` (letterbox, decode, NMS).

Per-op semantics (reference line, torch routine):
  CONV       F.conv2d (+ F.silu, + residual after the activation)   export/export.py:467-474
  ADD        a + b                                                   :475-476
  MAXPOOL5   F.max_pool2d(5, 1, 2)                                   :477-478
  UPSAMPLE2  nearest x2                                              :479-480
  PS2        quadrant pixel shuffle                                  :481-489
  COPYC      copy                                                    :490-491
  ATTN       softmax(q^T k * kd^-1/2), v att^T per head              :492-500
  GAP, SOFTMAX  mean over H, W; softmax over channels                :501-504
Pinned by tests/test_oracle_torch.py against the numpy interpreter (oracle.interp, itself
pinned against torch library routines and brute force): every op output of yolo11n, -seg
and -cls agrees to fp32 rounding, and the detections are identical.

Run as a script it times the yolo11n batch-1 frame of BASELINE config 0 on this host's
cores and prints one JSON line (bench.py runs it in a separate process, so the GPU
library is never loaded next to it):
    python oracle/torchref.py --seconds 15
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

if __package__ in (None, ""):
    _ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, _ROOT)
    from oracle import graphfile, post          # noqa: E402
else:
    from . import graphfile, post


class TorchRef:
    """Executes a parsed graph (oracle.graphfile.Graph) for a batch of B images."""

    def __init__(self, g: graphfile.Graph, B: int = 1):
        self.g, self.B = g, B
        self.bufs = [torch.zeros(B, C, H, W) for (H, W, C) in g.bufs]
        self.conv = {}
        for k, op in enumerate(g.ops):
            if op.kind != "CONV":
                continue
            ig = op.Cin // op.g
            n = op.Cout * op.k * op.k * ig
            w = g.weights[op.woff:op.woff + n].astype(np.float32).reshape(op.Cout, op.k, op.k, ig)
            w = torch.from_numpy(np.ascontiguousarray(w.transpose(0, 3, 1, 2)))
            b = torch.from_numpy(g.bias[op.boff:op.boff + op.Cout].astype(np.float32).copy())
            self.conv[k] = (w, b)
        self.heads: list = []

    def view(self, t: int) -> torch.Tensor:
        b, coff, C = self.g.tens[t]
        return self.bufs[b][:, coff:coff + C]

    def set_input(self, x_nhwc: np.ndarray):
        """x: [B, S, S, 3] float (stored through fp16, like the engine's input tensor)."""
        x = torch.from_numpy(np.asarray(x_nhwc, np.float32)).half().float().permute(0, 3, 1, 2)
        self.view(0).copy_(x)

    def run_op(self, k: int):
        op = self.g.ops[k]
        v = self.view
        kind = op.kind
        if kind == "CONV":
            w, b = self.conv[k]
            y = F.conv2d(v(op.a), w, b, stride=op.s, padding=op.p, groups=op.g)
            if op.act == 1:
                y = F.silu(y)
            if op.b >= 0:
                y = y + v(op.b)
            v(op.out).copy_(y)
        elif kind == "ADD":
            v(op.out).copy_(v(op.a) + v(op.b))
        elif kind == "MAXPOOL5":
            v(op.out).copy_(F.max_pool2d(v(op.a), 5, 1, 2))
        elif kind == "UPSAMPLE2":
            v(op.out).copy_(F.interpolate(v(op.a), scale_factor=2, mode="nearest"))
        elif kind == "PS2":
            x = v(op.a)
            C = x.shape[1] // 4
            o = v(op.out)
            for di in range(2):
                for dj in range(2):
                    q = 2 * di + dj
                    o[:, :, di::2, dj::2] = x[:, q * C:(q + 1) * C]
        elif kind == "COPYC":
            v(op.out).copy_(v(op.a))
        elif kind == "ATTN":
            x = v(op.a)
            B, _, H, W = x.shape
            N = H * W
            t = x.reshape(B, op.heads, 2 * op.kd + op.hd, N)
            q, kk, vv = t.split([op.kd, op.kd, op.hd], dim=2)
            att = torch.softmax((q.transpose(-2, -1) @ kk) * (op.kd ** -0.5), dim=-1)
            v(op.out).copy_((vv @ att.transpose(-2, -1)).reshape(B, op.heads * op.hd, H, W))
        elif kind == "GAP":
            v(op.out).copy_(v(op.a).mean(dim=(2, 3), keepdim=True))
        elif kind == "SOFTMAX":
            v(op.out).copy_(torch.softmax(v(op.a), dim=1))
        elif kind in ("DECODE", "DECODESEG", "DECODEOBB"):
            coef = v(op.out).clone() if kind != "DECODE" else None
            self.heads.append((v(op.a).clone(), v(op.b).clone(), coef, op.stride))
        elif kind == "MASKS":
            pass
        else:
            raise NotImplementedError(kind)

    @torch.no_grad()
    def run(self):
        self.heads = []
        for k in range(len(self.g.ops)):
            self.run_op(k)
        return self

    def heads_nhwc(self, img: int = 0):
        """Decode inputs of one image as numpy NHWC arrays (oracle.post layout)."""
        cv = lambda t: None if t is None else t[img].permute(1, 2, 0).numpy()
        return [(cv(b), cv(c), cv(m), s) for b, c, m, s in self.heads]


def frame(ref: TorchRef, img: np.ndarray, S: int, nc: int, conf=0.25, iou=0.45):
    """One batch-1 frame: letterbox -> every op -> decode + NMS (all on the CPU)."""
    ref.set_input(post.letterbox(img, S, S)[None])
    ref.run()
    return post.detect(ref.heads_nhwc(0), nc, conf, iou)


def _bench(seconds: float, max_frames: int):
    import json
    import tempfile
    import time
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "yolo11.cu_amd"))
    import modelgen
    ncpu = os.cpu_count() or 1
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else ncpu
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    # every core this process may use: the affinity set, capped by OMP_NUM_THREADS when the
    # host sets it (the GPU pool gives a process a share of the machine's cores)
    threads = min(ncpu, aff, omp) if omp > 0 else min(ncpu, aff)
    torch.set_num_threads(threads)
    with tempfile.TemporaryDirectory() as d:
        modelgen.write_model(d, "yolo11", "n", cls_bias=-8.0)
        g = graphfile.load(d)
        img = modelgen.synth_frame(810, 1080, 20, 1)
        ref = TorchRef(g, 1)
        det = frame(ref, img, 640, 80)       # warm-up (allocator, oneDNN primitives)
        times = []
        t_start = time.perf_counter()
        while len(times) < max_frames and (time.perf_counter() - t_start < seconds or len(times) < 10):
            t0 = time.perf_counter()
            det = frame(ref, img, 640, 80)
            times.append(time.perf_counter() - t0)
    ms = float(np.median(times)) * 1e3
    print(json.dumps({"ms": ms, "frames": len(times), "threads": torch.get_num_threads(), "cpu_count": ncpu,
                      "affinity": aff, "omp_num_threads": omp, "kept": int(len(det["score"]))}), flush=True)


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser()
    ap.add_argument("--seconds", type=float, default=15.0)
    ap.add_argument("--max-frames", type=int, default=200)
    a = ap.parse_args()
    _bench(a.seconds, a.max_frames)
