"""Algorithmic work of the ops a frame runs, and the launch units they run in.

Used by the benchmark (per-unit time attribution, roofline entries) and by the HBM traffic
tool (profiling.py), so both count work the same way:

    conv   2*B*Ho*Wo*Cout*k^2*Cin/g FLOPs; input + weights + output (+ residual) in fp16
           plus the fp32 bias
    attn   2*B*heads*N^2*(kd + hd) FLOPs; Q, K, V read once and the output written once
           (the N x N scores never leave the chip)
    other  (upsample, copy, add, pool, pixel shuffle, GAP, softmax) the bytes of their
           inputs and outputs
"""
from __future__ import annotations

KIND_KERNEL = {"ATTN": "k_attention", "MAXPOOL5": "k_sppf_pool / k_maxpool5", "UPSAMPLE2": "k_upsample2",
               "COPYC": "k_copyc", "ADD": "k_add", "PS2": "k_ps2", "GAP": "k_gap", "SOFTMAX": "k_softmax_ch"}


def conv_kernel_name(cfg: int, tail: int = -1) -> str:
    """The kernel an op config selects (yolo_set_op_config's numbering), with its tail retile."""
    if cfg == 1000:
        return "k_conv3x3_halo"
    if cfg == 1001:
        return "k_conv1x1_resident"
    if cfg == 1002:
        return "k_conv1x1_stream"
    if cfg >= 1200:
        return f"k_conv_tapws variant {cfg - 1200}"
    if cfg >= 1100:
        return f"k_conv_tap variant {cfg - 1100}"
    if tail >= 0:
        return f"k_conv_gemm cfg {cfg}, last-wave rows under cfg {tail} (two dispatches)"
    return f"k_conv_gemm cfg {cfg}"


def op_work(eng, k: int, B: int) -> tuple[float, float]:
    """(FLOPs, HBM bytes) of op k at batch B, by the rules above."""
    info = eng.op_info(k)
    kind = info["kind"]
    if kind in ("DECODE", "DECODESEG", "DECODEOBB", "MASKS"):
        return 0.0, 0.0
    Ho, Wo, Co = eng.tensor_shape(info["out"])
    Hi, Wi, Ci = eng.tensor_shape(info["a"])
    if kind == "CONV":
        g = max(info["g"], 1)
        kk = info["k"] * info["k"]
        flops = 2.0 * B * Ho * Wo * info["Cout"] * kk * info["Cin"] / g
        out_px = B * Ho * Wo * info["Cout"]
        nbytes = 2.0 * (B * Hi * Wi * info["Cin"] + info["Cout"] * kk * info["Cin"] / g + out_px
                        + (out_px if info["b"] >= 0 else 0)) + 4.0 * info["Cout"]
        return flops, nbytes
    if kind == "ATTN":
        # qkv width heads * (2 kd + hd), output heads * hd, kd = 32 (the loader's rule)
        heads = (Ci - Co) // 64
        hd = Co // heads
        n = Hi * Wi
        return 2.0 * B * heads * n * n * (32 + hd), 2.0 * B * n * (Ci + Co)
    nin = 2 if kind == "ADD" else 1
    return 0.0, 2.0 * B * (nin * Hi * Wi * Ci + Ho * Wo * Co)


def unit_kernel(eng, k: int) -> tuple[str, str]:
    """Kernel name and shape class of the launch unit whose first op is k."""
    info = eng.op_info(k)
    if info["kind"] != "CONV":
        return KIND_KERNEL.get(info["kind"], info["kind"]), ""
    if info["Cin"] == 3:
        return "k_conv_first", "stem 3x3 s2"
    if info["g"] > 1:
        return "k_dwconv", "depthwise 3x3"
    cls = "1x1" if info["k"] == 1 else f"{info['k']}x{info['k']} s{info['s']}"
    return conv_kernel_name(eng.op_config(k), eng.op_tail(k)), cls


def units(eng, B: int) -> list[dict]:
    """Launch units in launch order: index, member ops, first op, kernel, class, FLOPs and
    algorithmic bytes of the members."""
    unit = [eng.op_unit(k) for k in range(eng.num_ops)]
    out: dict[int, dict] = {}
    for k, u in enumerate(unit):
        if u < 0:
            continue
        if u not in out:
            name, cls = unit_kernel(eng, k)
            out[u] = {"unit": u, "first": k, "ops": [], "kernel": name, "class": cls, "flops": 0.0, "bytes": 0.0}
        if eng.op_info(k)["kind"] == "ATTN" and k != out[u]["first"]:
            out[u]["kernel"] = "k_attention"   # an attention launch carrying channel copies
        f, b = op_work(eng, k, B)
        out[u]["ops"].append(k)
        out[u]["flops"] += f
        out[u]["bytes"] += b
    return [out[u] for u in sorted(out)]


def unit_table(eng, B: int, per_unit_ms) -> list[dict]:
    """Per-unit kernel time (reported on each unit's first op) grouped by kernel and shape
    class, with the FLOPs and bytes of the ops the units launch; most time first."""
    groups: dict = {}
    for u in units(eng, B):
        g = groups.setdefault((u["kernel"], u["class"]), {"kernel": u["kernel"], "class": u["class"], "launches": 0,
                                                          "ms": 0.0, "flops": 0.0, "bytes": 0.0, "ops": [],
                                                          "firsts": []})
        g["launches"] += 1
        g["ms"] += float(per_unit_ms[u["first"]])
        g["flops"] += u["flops"]
        g["bytes"] += u["bytes"]
        g["ops"] += u["ops"]
        g["firsts"].append(u["first"])
    return sorted(groups.values(), key=lambda g: -g["ms"])
