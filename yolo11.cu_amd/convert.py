"""Real-checkpoint import: an ultralytics YOLOv8 / YOLO11 state_dict -> the model-dir format.

    python yolo11.cu_amd/convert.py yolo11n.safetensors build/yolo11n [--imgsz 640]
    python yolo11.cu_amd/convert.py yolo11n_state_dict.pt build/yolo11n

The reference exporter walks a live ultralytics model (export/export.py:83-145 conv packing,
:166-181 ConvTranspose rewrite, :222-302 module decomposition, :319-441 layer walk,
:709-719 file writer).  ultralytics is not a dependency here, so the checkpoint is read as
plain tensors: a `state_dict` saved with torch.save (loaded with weights_only=True, so
nothing in the file is executed), or a safetensors file.  A pickled ultralytics `.pt`
(the whole model object) is not loadable that way; save `model.state_dict()` from it first.

The topology is the generator's (modelgen.build_model, the same emission order as the
exporter); only the parameter source changes: every conv takes its tensors from the
state_dict under its ultralytics module path (`model.<layer>.<attr>...`):
  * Conv modules: `.conv.weight` and either BatchNorm `.bn.{weight,bias,running_mean,
    running_var}` (folded here with eps 1e-3, ultralytics' BatchNorm eps) or, for an
    already fused model, `.conv.bias`;
  * the head's plain Conv2d finals: `.weight`, `.bias`;
  * Segment's ConvTranspose2d `proto.upsample` and Classify's `linear`.
The architecture, scale, task and class count are read off the tensors (first conv width,
block count of layer 2, C2PSA / proto / cv4 / linear keys, final class conv rows); every
tensor must be consumed exactly once, with the shape the topology expects, and the DFL conv
must hold arange(16).  Parity against ultralytics itself is unpinned offline (no ultralytics
and no checkpoint in this environment).
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

import modelgen

# (first conv width, blocks in layer 2) -> scale, per architecture
_SCALE_KEYS = {
    "yolo11": {(16, 1): "n", (32, 1): "s", (64, 1): "m", (64, 2): "l", (96, 2): "x"},
    "yolov8": {(16, 1): "n", (32, 1): "s", (48, 2): "m", (64, 3): "l", (80, 3): "x"},
}
_IGNORED_SUFFIXES = (".num_batches_tracked",)


class StateDictSource:
    """Conv parameters from an ultralytics state_dict (numpy float32 arrays by key)."""

    def __init__(self, sd: dict):
        self.sd = {k: np.asarray(v, dtype=np.float32) for k, v in sd.items()}
        self.used: set[str] = set()

    def take(self, key: str, shape=None) -> np.ndarray:
        if key not in self.sd:
            raise KeyError(f"checkpoint has no tensor {key!r}")
        v = self.sd[key]
        if shape is not None and tuple(v.shape) != tuple(shape):
            raise ValueError(f"{key}: shape {tuple(v.shape)}, the topology expects {tuple(shape)}")
        if key in self.used:
            raise ValueError(f"{key} used twice")
        self.used.add(key)
        return v

    def conv(self, sp: modelgen.ConvSpec):
        """torch-layout weight [O, I/g, k, k] and bias [O], BatchNorm folded."""
        shape = (sp.c2, sp.c1 // sp.g, sp.k, sp.k)
        if not sp.bn:
            w = self.take(f"{sp.name}.weight", shape)
            key = f"{sp.name}.bias"
            b = self.take(key, (sp.c2,)) if key in self.sd else np.zeros(sp.c2, np.float32)
            return w, b
        w = self.take(f"{sp.name}.conv.weight", shape)
        if f"{sp.name}.bn.weight" in self.sd:
            gamma, beta, mean, var = (self.take(f"{sp.name}.bn.{f}", (sp.c2,))
                                      for f in ("weight", "bias", "running_mean", "running_var"))
            return modelgen.fold_bn(w, gamma, beta, mean, var)
        return w, self.take(f"{sp.name}.conv.bias", (sp.c2,))

    def conv_transpose(self, name: str, cin: int, cout: int):
        w = self.take(f"{name}.weight", (cin, cout, 2, 2))
        return w, self.take(f"{name}.bias", (cout,))

    def linear(self, name: str, i: int, o: int):
        return self.take(f"{name}.weight", (o, i)), self.take(f"{name}.bias", (o,))

    def unused(self) -> list[str]:
        return sorted(k for k in self.sd if k not in self.used and not k.endswith(_IGNORED_SUFFIXES))


def load_state_dict(path: str) -> dict:
    """Tensors of a checkpoint file as numpy arrays (never executes code from the file)."""
    if path.endswith(".safetensors"):
        from safetensors.numpy import load_file
        return dict(load_file(path))
    if path.endswith(".npz"):
        with np.load(path, allow_pickle=False) as z:
            return {k: z[k] for k in z.files}
    import torch
    obj = torch.load(path, map_location="cpu", weights_only=True)
    for k in ("model", "state_dict", "ema"):   # common wrappers around a state_dict
        if isinstance(obj, dict) and isinstance(obj.get(k), dict):
            obj = obj[k]
    if not isinstance(obj, dict) or not all(hasattr(v, "shape") for v in obj.values()):
        raise ValueError(f"{path}: not a state_dict of tensors (save model.state_dict() from the checkpoint)")
    return {k: v.detach().float().numpy() for k, v in obj.items()}


def infer(sd: dict) -> dict:
    """arch, scale, task and nc of a state_dict, from its keys and tensor shapes."""
    keys = sd.keys()
    arch = "yolo11" if any(".attn.qkv." in k for k in keys) else "yolov8"
    w0 = sd["model.0.conv.weight"].shape[0]
    n2 = len({k.split(".")[3] for k in keys if k.startswith("model.2.m.")})
    scale = _SCALE_KEYS[arch].get((w0, n2))
    if scale is None:
        raise ValueError(f"unknown {arch} scale: first conv width {w0}, {n2} blocks in layer 2")
    if any(k.endswith(".linear.weight") for k in keys):
        head = max(int(k.split(".")[1]) for k in keys if k.endswith(".linear.weight"))
        return dict(arch=arch, scale=scale, task="classify", nc=sd[f"model.{head}.linear.weight"].shape[0])
    head = max(int(k.split(".")[1]) for k in keys if k.startswith("model."))
    task = ("segment" if f"model.{head}.proto.cv1.conv.weight" in sd
            else "obb" if f"model.{head}.cv4.0.0.conv.weight" in sd else "detect")
    return dict(arch=arch, scale=scale, task=task, nc=sd[f"model.{head}.cv3.0.2.weight"].shape[0])


def convert(sd: dict, out_dir: str, imgsz: int | None = None, **override) -> modelgen.ModelInfo:
    """Writes model.graph / weights.f16 / bias.f32 for a state_dict; returns the model info."""
    meta = infer(sd)
    meta.update({k: v for k, v in override.items() if v is not None})
    if imgsz is None:
        imgsz = 224 if meta["task"] == "classify" else 640
    src = StateDictSource(sd)
    info = modelgen.build_model(meta["arch"], meta["scale"], meta["task"], meta["nc"], imgsz, source=src)
    if meta["task"] != "classify":
        head = max(int(k.split(".")[1]) for k in sd if k.startswith("model."))
        key = f"model.{head}.dfl.conv.weight"
        if key in sd:
            if not np.array_equal(src.take(key, (1, 16, 1, 1)).ravel(), np.arange(16, dtype=np.float32)):
                raise ValueError(f"{key} is not arange(16): the decode assumes the fixed DFL projection")
    left = src.unused()
    if left:
        raise ValueError(f"{len(left)} checkpoint tensors have no place in the {meta['arch']}{meta['scale']}-"
                         f"{meta['task']} topology: {left[:8]}{' ...' if len(left) > 8 else ''}")
    info.graph.write(out_dir, meta["task"], meta["nc"], imgsz)
    with open(os.path.join(out_dir, "gen.txt"), "w") as f:
        f.write(f"{meta['arch']} {meta['scale']} {meta['task']} nc={meta['nc']} imgsz={imgsz} converted\n")
    return info


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="convert", description=__doc__.split("\n\n")[0])
    ap.add_argument("checkpoint", help="state_dict (.pt via torch.save), .safetensors or .npz")
    ap.add_argument("out_dir")
    ap.add_argument("--imgsz", type=int, default=None, help="network input size (default 640, classify 224)")
    ap.add_argument("--arch", choices=["yolo11", "yolov8"], default=None)
    ap.add_argument("--scale", choices=list("nsmlx"), default=None)
    ap.add_argument("--task", choices=["detect", "segment", "obb", "classify"], default=None)
    ap.add_argument("--nc", type=int, default=None)
    a = ap.parse_args(argv)
    info = convert(load_state_dict(a.checkpoint), a.out_dir, a.imgsz, arch=a.arch, scale=a.scale, task=a.task,
                   nc=a.nc)
    n = modelgen.count_ops(info)
    print(f"{a.out_dir}: {info.arch}{info.scale}-{info.task} nc={info.nc} imgsz={info.imgsz}, {n['total']} ops")
    return 0


if __name__ == "__main__":
    sys.exit(main())
