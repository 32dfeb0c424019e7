"""Real-checkpoint import (yolo11.cu_amd/convert.py) on the CPU.

* The ultralytics state_dict layout is pinned independently of this build's code by the
  public parameter counts of the ultralytics model summaries (every trainable tensor:
  conv weights, BatchNorm gamma/beta, head biases, the 16-weight DFL conv): a layout with a
  wrong or missing module, a transposed shape or a wrong width misses these totals.
* Conversion round trip: a seeded model's unfolded parameters, written under ultralytics
  names as a torch state_dict (.pt, loaded weights-only) or safetensors, convert back to the
  byte-identical model dir (graph, fp16 weights, biases), for every task and both archs.
* BatchNorm folding against its closed form, fused checkpoints, and the refusals (missing
  tensor, wrong shape, leftover tensors, a DFL conv that is not arange(16)).
* The converted dir loads through the C ABI's host-only loader with the generator's op
  counts.  Parity against ultralytics itself stays unpinned offline.
"""
import filecmp
import os

import numpy as np
import pytest
import torch

import convert
import modelgen
import yolort

# ultralytics model summaries (unfused): total trainable parameters
PUBLIC_PARAMS = {("yolo11", "n", "detect"): 2_624_080, ("yolo11", "s", "detect"): 9_458_752,
                 ("yolo11", "m", "detect"): 20_114_688, ("yolo11", "l", "detect"): 25_372_160,
                 ("yolo11", "x", "detect"): 56_966_176, ("yolov8", "n", "detect"): 3_157_200,
                 ("yolo11", "n", "segment"): 2_876_848, ("yolo11", "n", "classify"): 2_812_104}

CASES = [("yolo11", "n", "detect", 80, 640), ("yolo11", "n", "segment", 80, 640), ("yolo11", "n", "obb", 15, 640),
         ("yolo11", "n", "classify", 1000, 224), ("yolov8", "n", "detect", 80, 640), ("yolo11", "m", "detect", 80, 640)]


def _state_dict(arch, scale, task, nc, imgsz, seed=0):
    """A seeded model's parameters under ultralytics names (+ the fixed DFL conv and the
    BatchNorm step counters a real state_dict carries)."""
    rec = {}
    info = modelgen.build_model(arch, scale, task, nc, imgsz, seed, cls_bias=-8.0, record=rec)
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in rec.items()}
    if task != "classify":
        head = max(int(k.split(".")[1]) for k in sd)
        sd[f"model.{head}.dfl.conv.weight"] = torch.arange(16, dtype=torch.float32).view(1, 16, 1, 1)
    for k in list(sd):
        if k.endswith(".bn.running_var"):
            sd[k[:-len("running_var")] + "num_batches_tracked"] = torch.tensor(0)
    return info, sd


@pytest.mark.parametrize("key,params", list(PUBLIC_PARAMS.items()))
def test_state_dict_layout_matches_public_param_counts(key, params):
    arch, scale, task = key
    nc, imgsz = (1000, 224) if task == "classify" else (80, 640)
    rec = {}
    modelgen.build_model(arch, scale, task, nc, imgsz, calibrate=False, record=rec)
    n = sum(v.size for k, v in rec.items() if not k.endswith(("running_mean", "running_var")))
    assert n + (16 if task != "classify" else 0) == params


@pytest.mark.parametrize("arch,scale,task,nc,imgsz", CASES)
def test_round_trip_byte_identical(tmp_path, arch, scale, task, nc, imgsz):
    info, sd = _state_dict(arch, scale, task, nc, imgsz)
    want = tmp_path / "gen"
    info.graph.write(str(want), task, nc, imgsz)
    assert convert.infer({k: v.numpy() for k, v in sd.items()}) == dict(arch=arch, scale=scale, task=task, nc=nc)
    p = tmp_path / "ckpt.pt"
    torch.save(sd, p)
    got = tmp_path / "conv"
    convert.main([str(p), str(got), "--imgsz", str(imgsz)])
    for f in ("model.graph", "weights.f16", "bias.f32"):
        assert filecmp.cmp(want / f, got / f, shallow=False), f
    n, err = yolort.graph_check(str(got))
    assert n == modelgen.count_ops(info)["total"], err


def test_safetensors_and_wrapped_checkpoints(tmp_path):
    from safetensors.torch import save_file
    info, sd = _state_dict("yolo11", "n", "detect", 80, 640)
    want = tmp_path / "gen"
    info.graph.write(str(want), "detect", 80, 640)
    save_file({k: v.contiguous() for k, v in sd.items() if v.dtype == torch.float32}, str(tmp_path / "m.safetensors"))
    torch.save({"model": sd, "epoch": 3}, tmp_path / "wrapped.pt")
    for src in ("m.safetensors", "wrapped.pt"):
        out = tmp_path / src.replace(".", "_")
        convert.main([str(tmp_path / src), str(out)])
        assert filecmp.cmp(want / "weights.f16", out / "weights.f16", shallow=False)


def test_bn_folding_closed_form_and_fused_checkpoint(tmp_path):
    info, sd = _state_dict("yolo11", "n", "detect", 80, 640)
    sdn = {k: v.numpy() for k, v in sd.items()}
    src = convert.StateDictSource(sdn)
    sp = modelgen.ConvSpec(3, 16, 3, 2, name="model.0")
    w, b = src.conv(sp)
    g, be, mu, var = (sdn[f"model.0.bn.{f}"].astype(np.float64) for f in ("weight", "bias", "running_mean", "running_var"))
    s = g / np.sqrt(var + 1e-3)
    np.testing.assert_allclose(w, sdn["model.0.conv.weight"] * s[:, None, None, None], rtol=1e-6)
    np.testing.assert_allclose(b, be - mu * s, rtol=1e-6, atol=1e-6)
    # the same model fused (BatchNorm folded into conv.weight / conv.bias, no bn.* tensors)
    fused = {}
    for k, v in sdn.items():
        if k.endswith(".bn.weight"):
            m = k[:-len(".bn.weight")]
            fw, fb = modelgen.fold_bn(sdn[f"{m}.conv.weight"], v, sdn[f"{m}.bn.bias"], sdn[f"{m}.bn.running_mean"],
                                      sdn[f"{m}.bn.running_var"])
            fused[f"{m}.conv.weight"], fused[f"{m}.conv.bias"] = fw, fb
        elif ".bn." not in k and not (k.endswith(".conv.weight") and k[:-len(".conv.weight")] + ".bn.weight" in sdn):
            fused[k] = v
    convert.convert(fused, str(tmp_path / "fused"))
    want = tmp_path / "gen"
    info.graph.write(str(want), "detect", 80, 640)
    assert filecmp.cmp(want / "weights.f16", tmp_path / "fused" / "weights.f16", shallow=False)


def test_refusals(tmp_path):
    _, sd = _state_dict("yolo11", "n", "detect", 80, 640)
    base = {k: v.numpy() for k, v in sd.items()}
    bad = dict(base)
    del bad["model.4.m.0.cv2.conv.weight"]
    with pytest.raises(KeyError, match="model.4.m.0.cv2.conv.weight"):
        convert.convert(bad, str(tmp_path / "a"))
    bad = dict(base)
    bad["model.9.cv1.conv.weight"] = np.zeros((128, 256, 3, 3), np.float32)
    with pytest.raises(ValueError, match="model.9.cv1.conv.weight: shape"):
        convert.convert(bad, str(tmp_path / "b"))
    bad = dict(base)
    bad["model.23.extra.weight"] = np.zeros(3, np.float32)
    with pytest.raises(ValueError, match="no place"):
        convert.convert(bad, str(tmp_path / "c"))
    bad = dict(base)
    bad["model.23.dfl.conv.weight"] = np.ones((1, 16, 1, 1), np.float32)
    with pytest.raises(ValueError, match="arange"):
        convert.convert(bad, str(tmp_path / "d"))
    assert not os.path.exists(tmp_path / "a" / "model.graph")
