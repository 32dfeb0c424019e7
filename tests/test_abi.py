"""C-ABI library checks that need no GPU: it loads, exports every symbol include/yolo.h
declares, and its host-only loader (yolo_graph_check) accepts the generated model dirs and
rejects malformed ones with the reference loader's rules (engine/engine.cu:88-191)."""
import os
import shutil

import pytest

import modelgen
import yolort


def test_exports_every_header_symbol():
    lib = yolort.load()
    syms = yolort.header_symbols()
    assert len(syms) >= 40
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # the ctypes signature table covers the whole header, nothing more
    assert sorted(yolort._SIGS) == syms


def test_tile_table():
    tiles = yolort.tile_configs()
    assert len(tiles) >= 8
    for BM, BN, WM, WN, BK, NS in tiles:
        assert BK in (32, 64, 128)
        assert (BM // WM) % 16 == 0 and (BN // WN) % 16 == 0
        assert 64 * WM * WN <= 1024 and (WM * WN) % 4 == 0
        assert 2 <= NS <= 8
        # the LDS ring fits the 160 KiB of a CU
        assert NS * (BM + BN) * BK * 2 <= 160 * 1024
        # every wave issues the same number of 64-chunk DMA groups for both operands
        assert (BM * BK // 8 // 64) % (WM * WN) == 0 and (BN * BK // 8 // 64) % (WM * WN) == 0


@pytest.mark.parametrize("arch,scale,task,nops", [("yolo11", "n", "detect", 112), ("yolo11", "m", "detect", 144),
                                                  ("yolo11", "n", "segment", 127), ("yolov8", "n", "detect", 77)])
def test_graph_check_accepts(models, arch, scale, task, nops):
    d = models(arch, scale, task)
    n, err = yolort.graph_check(d)
    assert n == nops, err


def _mutate(src, dst, fn):
    shutil.copytree(src, dst)
    p = os.path.join(dst, "model.graph")
    lines = open(p).read().splitlines()
    open(p, "w").write("\n".join(fn(lines)) + "\n")
    return dst


@pytest.mark.parametrize("name,fn,msg", [
    ("badtask", lambda L: [L[0], "TASK classify 1000 640"] + L[2:], "classify"),
    ("badop", lambda L: L[:-1] + ["FOO 1 2"], "bad op"),
    ("short", lambda L: L[:-1] + [" ".join(L[-1].split()[:2])], "short op line"),
    ("imgsz", lambda L: [L[0], "TASK detect 80 320"] + L[2:], "imgsz"),
    ("ncpad", lambda L: [L[0], "TASK detect 81 640"] + L[2:], "8-aligned cls view"),
    ("tensor", lambda L: [l if not l.startswith("T 0 ") else "T 999 0 3" for l in L], "missing buffer"),
])
def test_graph_check_rejects(models, tmp_path, name, fn, msg):
    d = _mutate(models("yolo11", "n"), str(tmp_path / name), fn)
    n, err = yolort.graph_check(d)
    assert n == -1 and msg in err, err


def test_graph_check_obb(models, tmp_path):
    """yolo11n-obb at 1024: 118 ops + 3 DECODEOBB; DECODEOBB outside an obb graph and a
    DECODE inside one are rejected."""
    d = models("yolo11", "n", "obb", -6.25, 1024, 0, 15)
    n, err = yolort.graph_check(d)
    assert n == 121, err
    bad = _mutate(d, str(tmp_path / "obbtask"), lambda L: [L[0], "TASK detect 15 1024"] + L[2:])
    n, err = yolort.graph_check(bad)
    assert n == -1 and "DECODEOBB needs task=obb" in err, err
    bad = _mutate(d, str(tmp_path / "obbdec"), lambda L: [
        " ".join(["DECODE"] + l.split()[1:3] + l.split()[4:]) if l.startswith("DECODEOBB") else l for l in L])
    n, err = yolort.graph_check(bad)
    assert n == -1 and "obb graphs decode with DECODEOBB" in err, err


def test_graph_check_missing_dir(tmp_path):
    n, err = yolort.graph_check(str(tmp_path / "nope"))
    assert n == -1 and "model.graph" in err
