"""Model-dir reader for the oracle (test infrastructure; see oracle/__init__.py).

Restates the reference's `loadGraph` grammar (engine/engine.cu:88-141) and fuse pass
(`fuseAdds`, engine/engine.cu:1484-1501) in Python so tests can walk the same op list the
engine executes.  Pinned by: round-tripping every graph the generator writes, and by the
op-count / op-arity checks in tests/test_modelgen.py against the reference-held counts
(README.md:191: 109 dumped ops for yolo11n, 141 for yolo11m).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np

ARITY = {"CONV": 11, "ADD": 3, "MAXPOOL5": 2, "UPSAMPLE2": 2, "COPYC": 2, "ATTN": 5,
         "DECODE": 3, "DECODEOBB": 4, "PS2": 2, "DECODESEG": 4, "MASKS": 1, "GAP": 2,
         "SOFTMAX": 2}


@dataclass
class Op:
    kind: str
    a: int = -1
    b: int = -1
    out: int = -1
    k: int = 0
    s: int = 0
    p: int = 0
    g: int = 0
    act: int = 0
    Cin: int = 0
    Cout: int = 0
    woff: int = 0
    boff: int = 0
    heads: int = 0
    kd: int = 0
    hd: int = 0
    stride: int = 0


@dataclass
class Graph:
    task: str
    nc: int
    imgsz: int
    bufs: list = field(default_factory=list)   # (H, W, C)
    tens: list = field(default_factory=list)   # (buf, coff, C)
    ops: list = field(default_factory=list)
    weights: np.ndarray | None = None           # fp16
    bias: np.ndarray | None = None              # fp32

    def shape(self, t):
        b, _, C = self.tens[t]
        H, W, _ = self.bufs[b]
        return H, W, C


def parse_op(tag: str, v: list[int]) -> Op:
    if tag not in ARITY or len(v) != ARITY[tag]:
        raise ValueError(f"bad op {tag} {v}")
    if tag == "CONV":
        return Op("CONV", a=v[0], out=v[1], k=v[2], s=v[3], p=v[4], g=v[5], act=v[6],
                  Cin=v[7], Cout=v[8], woff=v[9], boff=v[10])
    if tag == "ADD":
        return Op("ADD", a=v[0], b=v[1], out=v[2])
    if tag == "ATTN":
        return Op("ATTN", a=v[0], out=v[1], heads=v[2], kd=v[3], hd=v[4])
    if tag == "DECODE":
        return Op("DECODE", a=v[0], b=v[1], stride=v[2])
    if tag in ("DECODEOBB", "DECODESEG"):
        return Op(tag, a=v[0], b=v[1], out=v[2], stride=v[3])
    if tag == "MASKS":
        return Op("MASKS", a=v[0])
    return Op(tag, a=v[0], out=v[1])


def load(path: str, with_weights: bool = True) -> Graph:
    with open(os.path.join(path, "model.graph")) as f:
        toks = f.read().split()
    pos = 0

    def nxt():
        nonlocal pos
        t = toks[pos]
        pos += 1
        return t

    magic, ver = nxt(), int(nxt())
    task, nc, imgsz = "detect", 80, 0
    if ver >= 2:
        if nxt() != "TASK":
            raise ValueError("bad TASK header")
        task, nc, imgsz = nxt(), int(nxt()), int(nxt())
    nb, nt, no = int(nxt()), int(nxt()), int(nxt())
    g = Graph(task, nc, imgsz)
    for _ in range(nb):
        nxt()
        g.bufs.append((int(nxt()), int(nxt()), int(nxt())))
    for _ in range(nt):
        nxt()
        g.tens.append((int(nxt()), int(nxt()), int(nxt())))
    for _ in range(no):
        tag = nxt()
        n = ARITY.get(tag)
        if n is None:
            raise ValueError(f"bad op {tag}")
        g.ops.append(parse_op(tag, [int(nxt()) for _ in range(n)]))
    if with_weights:
        g.weights = np.fromfile(os.path.join(path, "weights.f16"), np.float16)
        g.bias = np.fromfile(os.path.join(path, "bias.f32"), np.float32)
    return g


def fuse_adds(ops: list[Op]) -> list[Op]:
    """A CONV immediately followed by an ADD consuming its output becomes a CONV with a
    residual (b) whose out is the ADD's out (engine/engine.cu:1484-1501)."""
    out, i = [], 0
    while i < len(ops):
        op = Op(**vars(ops[i]))
        if op.kind == "CONV" and op.b < 0 and i + 1 < len(ops):
            nx = ops[i + 1]
            if nx.kind == "ADD" and (nx.a == op.out or nx.b == op.out):
                op.b = nx.b if nx.a == op.out else nx.a
                op.out = nx.out
                i += 1
        out.append(op)
        i += 1
    return out
