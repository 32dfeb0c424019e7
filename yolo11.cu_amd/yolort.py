"""ctypes binding of libyolo11_amd.so (the C ABI in include/yolo.h).

This is the Python face of the engine for tests and benchmarks; it talks to the library
only through the C ABI, uses numpy for host arrays and the library's own allocation
helpers for device memory (no torch in the process, so exactly one HIP runtime is
loaded).  There is no CPU fallback: if the library is missing, `load()` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libyolo11_amd.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "yolo.h")

YOLO_NOFUSE, YOLO_NOTUNE, YOLO_NOGRAPH, YOLO_BRANCHES, YOLO_DAGGRAPH, YOLO_NOGROUP = 1, 2, 4, 8, 16, 32
YOLO_NMS_BLOCK = 64
PIXEL_BGR, PIXEL_RGBX = 0, 1   # frame layouts of yolo_stage_frames (B,G,R / R,G,B,X bytes)
JPEG_STAGED, JPEG_UNSUPPORTED, JPEG_INVALID = 0, 1, 2   # yolo_stage_jpeg per-stream status
CFG_HALO = 1000   # op config of the LDS-halo 3x3 kernel (small-channel stride-1 convs)
CFG_1X1 = 1001    # op config of the weights-resident 1x1 kernel (stride 1, Cin <= 384)
CFG_1X1S = 1002   # the same with two pixel groups in flight per wave and 16-byte stores
CFG_TAP = 1100    # op configs 1100 .. 1100 + NUM_TAP_TILES - 1: streaming-conv tile variants
NUM_TAP_TILES = 13
TAP_3X3 = range(0, 8)    # variants for 3x3 stride-1 convs (halo-staged)
TAP_1X1 = range(8, 13)   # variants for 1x1 stride-1 convs
TAP_BN = (64, 96, 64, 64, 96, 64, 96, 48, 384, 192, 192, 128, 256)   # output channels per block
CFG_TAPWS = 1200  # op configs 1200 .. 1200 + NUM_TAPWS_TILES - 1: wave-specialised 3x3 variants
NUM_TAPWS_TILES = 4
TAPWS_BN = (64, 48, 64, 96)
OP_KINDS = ["CONV", "ADD", "MAXPOOL5", "UPSAMPLE2", "COPYC", "ATTN", "DECODE", "GAP", "SOFTMAX",
            "DECODEOBB", "PS2", "DECODESEG", "MASKS"]
MAX_OUT = 300


class YoloDet(C.Structure):
    _fields_ = [("x1", C.c_float), ("y1", C.c_float), ("x2", C.c_float), ("y2", C.c_float),
                ("score", C.c_float), ("cls", C.c_int)]


class YoloObbDet(C.Structure):
    _fields_ = [("x", C.c_float), ("y", C.c_float), ("w", C.c_float), ("h", C.c_float),
                ("angle", C.c_float), ("score", C.c_float), ("cls", C.c_int)]


class YoloHeadLevel(C.Structure):
    _fields_ = [("box", C.c_void_p), ("cls", C.c_void_p), ("H", C.c_int), ("W", C.c_int),
                ("stride", C.c_int), ("box_stride", C.c_int), ("box_off", C.c_int),
                ("cls_stride", C.c_int), ("cls_off", C.c_int)]


class YoloBatchResult(C.Structure):
    _fields_ = [("tag", C.c_longlong), ("status", C.c_int), ("model", C.c_int), ("task", C.c_int),
                ("batch", C.c_int), ("queue_ms", C.c_float), ("infer_ms", C.c_float), ("n", C.c_int),
                ("stride", C.c_int), ("rows", C.POINTER(C.c_float)), ("rle", C.POINTER(C.c_uint)),
                ("rle_len", C.POINTER(C.c_int)), ("mask_h", C.c_int), ("mask_w", C.c_int),
                ("lb_scale", C.c_float), ("lb_top", C.c_int), ("lb_left", C.c_int), ("host", C.c_void_p),
                ("owner", C.c_void_p)]


_SIGS = {
    "yolo_create": (C.c_void_p, [C.c_char_p, C.c_int]),
    "yolo_task": (C.c_int, [C.c_void_p]),
    "yolo_exec_ms": (C.c_float, [C.c_void_p, C.c_int]),
    "yolo_stream": (C.c_void_p, [C.c_void_p]),
    "yolo_preprocess": (None, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "yolo_run": (None, [C.c_void_p, C.c_int]),
    "yolo_run_async": (None, [C.c_void_p, C.c_int]),
    "yolo_sync": (None, [C.c_void_p]),
    "yolo_get": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(YoloDet), C.c_int]),
    "yolo_stage_frames": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p), C.POINTER(C.c_int),
                                    C.POINTER(C.c_int), C.c_int, C.c_int]),
    "yolo_stage_jpeg": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t), C.c_int,
                                  C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_decode_jpeg": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t), C.c_int,
                                   C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_letterbox_decoded": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "yolo_jpeg_submit": (C.c_void_p, [C.c_char_p, C.c_size_t]),
    "yolo_decode_tickets": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p), C.c_int, C.POINTER(C.c_int),
                                      C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_jpeg_release": (None, [C.c_void_p]),
    "yolo_decoder_threads": (C.c_int, []),
    "yolo_jpeg_max_pixels": (C.c_longlong, [C.c_longlong]),
    "yolo_op_unit": (C.c_int, [C.c_void_p, C.c_int]),
    "yolo_num_units": (C.c_int, [C.c_void_p]),
    "yolo_run_unit": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "yolo_marker": (C.c_int, [C.c_void_p]),
    "yolo_get_masks": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "yolo_batcher_create": (C.c_void_p, [C.POINTER(C.c_void_p), C.POINTER(C.c_int), C.c_int, C.c_double]),
    "yolo_batcher_submit_jpeg": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t, C.c_longlong]),
    "yolo_batcher_submit_frame": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_longlong]),
    "yolo_batcher_wait": (C.c_int, [C.c_void_p, C.POINTER(YoloBatchResult), C.c_int, C.c_int]),
    "yolo_batcher_release": (None, [C.POINTER(YoloBatchResult), C.c_int]),
    "yolo_batcher_stage_ms": (C.c_double, [C.c_void_p]),
    "yolo_batcher_stop": (None, [C.c_void_p]),
    "yolo_batcher_destroy": (None, [C.c_void_p]),
    "yolo_jpeg_probe": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_jpeg_coefficients": (C.c_longlong, [C.c_char_p, C.c_size_t, C.c_void_p, C.c_size_t]),
    "yolo_get_batch": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(YoloDet), C.c_int, C.POINTER(C.c_int)]),
    "yolo_get_obb_batch": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(YoloObbDet), C.c_int, C.POINTER(C.c_int)]),
    "yolo_preprocess_cls": (None, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "yolo_get_cls": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_float), C.c_int]),
    "yolo_slot_geom": (None, [C.c_void_p, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_get_obb": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(YoloObbDet), C.c_int]),
    "yolo_mask_dim": (None, [C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_get_mask": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "yolo_create_ex": (C.c_void_p, [C.c_char_p, C.c_int, C.c_int, C.c_char_p, C.c_int]),
    "yolo_destroy": (None, [C.c_void_p]),
    "yolo_graph_check": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int]),
    "yolo_set_thresholds": (C.c_int, [C.c_void_p, C.c_float, C.c_float, C.c_int]),
    "yolo_raw_count": (C.c_int, [C.c_void_p, C.c_int]),
    "yolo_num_ops": (C.c_int, [C.c_void_p]),
    "yolo_op_info": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int)]),
    "yolo_num_tensors": (C.c_int, [C.c_void_p]),
    "yolo_tensor_shape": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_int)]),
    "yolo_read_tensor": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "yolo_write_tensor": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "yolo_read_tensor_slots": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "yolo_write_tensor_slots": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "yolo_run_op": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "yolo_run_post": (C.c_int, [C.c_void_p, C.c_int]),
    "yolo_op_config": (C.c_int, [C.c_void_p, C.c_int]),
    "yolo_set_op_config": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "yolo_op_split": (C.c_int, [C.c_void_p, C.c_int]),
    "yolo_set_op_split": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "yolo_op_tail": (C.c_int, [C.c_void_p, C.c_int]),
    "yolo_set_op_tail": (C.c_int, [C.c_void_p, C.c_int, C.c_int]),
    "yolo_num_tile_configs": (C.c_int, []),
    "yolo_tile_config": (C.c_int, [C.c_int, C.POINTER(C.c_int)]),
    "yolo_frame_graph": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                   C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "yolo_frame_run": (C.c_int, [C.c_void_p]),
    "yolo_frame_launch": (C.c_int, [C.c_void_p]),
    "yolo_time_graph": (C.c_float, [C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "yolo_profile_ops": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "yolo_profile_stages": (C.c_int, [C.c_void_p, C.c_int, C.POINTER(C.c_float)]),
    "yolo_profile_units": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "yolo_spin_failures": (C.c_int, [C.c_void_p]),
    "yolo_dev_alloc": (C.c_void_p, [C.c_size_t]),
    "yolo_dev_free": (None, [C.c_void_p]),
    "yolo_host_alloc": (C.c_void_p, [C.c_size_t]),
    "yolo_host_free": (None, [C.c_void_p]),
    "yolo_copy_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "yolo_copy_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    "yolo_detect_static": (C.c_int, [C.POINTER(YoloHeadLevel), C.c_int, C.c_int, C.c_int, C.c_float,
                                     C.c_float, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/yolo.h."""
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(yolo_[a-z0-9_]+)\s*\(", txt)))


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def tile_configs() -> list[tuple[int, int, int, int, int, int]]:
    """(BM, BN, WM, WN, BK, stages) of every compiled GEMM tile configuration."""
    lib = load()
    out = []
    for i in range(lib.yolo_num_tile_configs()):
        v = (C.c_int * 6)()
        lib.yolo_tile_config(i, v)
        out.append(tuple(v))
    return out


class DeviceBuffer:
    """Device memory from the engine's allocator."""

    def __init__(self, nbytes: int):
        self.lib = load()
        self.nbytes = nbytes
        self.ptr = self.lib.yolo_dev_alloc(max(nbytes, 16))
        if not self.ptr:
            raise MemoryError(f"yolo_dev_alloc({nbytes}) failed")

    def free(self):
        if self.ptr:
            self.lib.yolo_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def decoder_threads() -> int:
    """Threads (the caller included) the library's JPEG entropy decoding runs on."""
    return load().yolo_decoder_threads()


def jpeg_probe(data: bytes) -> tuple[int, int, int]:
    """(1 if yolo_stage_jpeg decodes it / 0 if a JPEG outside that set / -1 if not a JPEG,
    height, width) from the stream's headers."""
    h, w = C.c_int(0), C.c_int(0)
    r = load().yolo_jpeg_probe(data, len(data), C.byref(h), C.byref(w))
    return r, h.value, w.value


def jpeg_max_pixels(n: int = 0) -> int:
    """The largest frame (pixels) the engine decodes; n > 0 sets it (process-wide)."""
    return load().yolo_jpeg_max_pixels(n)


def jpeg_submit(data: bytes):
    """Starts entropy-decoding a JPEG stream on the library's decoder threads; a ticket for
    Engine.decode_tickets, or None if the engine does not decode this stream."""
    return load().yolo_jpeg_submit(data, len(data)) or None


def jpeg_release(ticket) -> None:
    """Frees a ticket that will not be decoded."""
    if ticket:
        load().yolo_jpeg_release(ticket)


def jpeg_coefficients(data: bytes) -> np.ndarray | None:
    """The library's entropy decode (host code): int16 quantised coefficients, natural order,
    plane after plane; None if unsupported, raises on a corrupt stream."""
    lib = load()
    n = lib.yolo_jpeg_coefficients(data, len(data), None, 0)
    if n < 0:
        return None
    out = np.empty(n, np.int16)
    r = lib.yolo_jpeg_coefficients(data, len(data), out.ctypes.data, n)
    if r == -2:
        raise ValueError("corrupt JPEG stream")
    return out


BATCH_OK, BATCH_DECODE_FAILED, BATCH_STOPPED, BATCH_FAILED = 0, 1, 2, 3   # YoloBatchResult.status


class Batcher:
    """The native batch worker (yolo_batcher_*): a deadline-aware batcher and the per-batch
    loop on a library thread.  The engines belong to it while it runs."""

    def __init__(self, engines: list, max_batch: list[int], target_ms: float = 50.0):
        self.lib = load()
        n = len(engines)
        hs = (C.c_void_p * n)(*[e.h for e in engines])
        mb = (C.c_int * n)(*max_batch)
        self.h = self.lib.yolo_batcher_create(hs, mb, n, float(target_ms))
        if not self.h:
            raise RuntimeError("yolo_batcher_create failed")
        self._buf = (YoloBatchResult * 64)()

    def submit_jpeg(self, model: int, data: bytes, tag: int) -> int:
        """0 queued, 1 not a stream the engine decodes, -1 stopped."""
        return self.lib.yolo_batcher_submit_jpeg(self.h, model, data, len(data), tag)

    def submit_frame(self, model: int, ptr: int, height: int, width: int, tag: int) -> int:
        return self.lib.yolo_batcher_submit_frame(self.h, model, ptr, height, width, tag)

    def wait(self, timeout_ms: int = 100):
        """Finished requests as dicts (rows copied out of the library), [] on timeout, None
        once the batcher has stopped and answered everything.  One caller thread only."""
        n = self.lib.yolo_batcher_wait(self.h, self._buf, len(self._buf), timeout_ms)
        if n < 0:
            return None
        out = []
        for i in range(n):
            r = self._buf[i]
            rows = np.ctypeslib.as_array(r.rows, (r.n * r.stride,)).reshape(r.n, r.stride).copy() \
                if r.n > 0 else np.zeros((0, max(r.stride, 1)), np.float32)
            rec = dict(tag=r.tag, status=r.status, model=r.model, task=r.task, batch=r.batch,
                       queue_ms=r.queue_ms, infer_ms=r.infer_ms, rows=rows, host=r.host or 0)
            if r.task == 3 and r.status == 0:
                lens = np.ctypeslib.as_array(r.rle_len, (r.n,)).copy() if r.n > 0 else np.zeros(0, np.int32)
                runs = np.ctypeslib.as_array(r.rle, (int(lens.sum()),)).copy() if r.n > 0 else np.zeros(0, np.uint32)
                rec.update(rle_len=lens, rle=runs, mask_hw=(r.mask_h, r.mask_w),
                           geom=(r.lb_scale, r.lb_top, r.lb_left))
            out.append(rec)
        if n:
            self.lib.yolo_batcher_release(self._buf, n)
        return out

    def stage_ms(self) -> float:
        return self.lib.yolo_batcher_stage_ms(self.h)

    def stop(self):
        if self.h:
            self.lib.yolo_batcher_stop(self.h)

    def destroy(self):
        if self.h:
            self.lib.yolo_batcher_destroy(self.h)
            self.h = None


class PinnedBuffer:
    """Pinned host memory viewed as a numpy array."""

    def __init__(self, shape, dtype=np.uint8):
        self.lib = load()
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        self.ptr = self.lib.yolo_host_alloc(max(n, 16))
        if not self.ptr:
            raise MemoryError("yolo_host_alloc failed")
        self.array = np.ctypeslib.as_array((C.c_uint8 * n).from_address(self.ptr)).view(dt).reshape(shape)

    def free(self):
        if self.ptr:
            self.array = None
            self.lib.yolo_host_free(self.ptr)
            self.ptr = None


class Engine:
    def __init__(self, model_dir: str, max_batch: int = 1, flags: int = 0):
        self.lib = load()
        err = C.create_string_buffer(1024)
        self.h = self.lib.yolo_create_ex(model_dir.encode(), max_batch, flags, err, 1024)
        if not self.h:
            raise RuntimeError(f"yolo_create_ex failed: {err.value.decode()}")
        self.max_batch = max_batch
        self._getbuf = {}

    def close(self):
        if self.h:
            self.lib.yolo_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- graph introspection
    @property
    def num_ops(self) -> int:
        return self.lib.yolo_num_ops(self.h)

    def op_info(self, k: int) -> dict:
        v = (C.c_int * 9)()
        if self.lib.yolo_op_info(self.h, k, v) != 0:
            raise IndexError(k)
        kind, a, b, out, kk, s, g, cin, cout = v
        return dict(kind=OP_KINDS[kind], a=a, b=b, out=out, k=kk, s=s, g=g, Cin=cin, Cout=cout)

    def tensor_shape(self, t: int) -> tuple[int, int, int]:
        v = (C.c_int * 3)()
        if self.lib.yolo_tensor_shape(self.h, t, v) != 0:
            raise IndexError(t)
        return tuple(v)

    def read(self, t: int, B: int = 1) -> np.ndarray:
        H, W, Cc = self.tensor_shape(t)
        out = np.empty((B, H, W, Cc), np.float16)
        if self.lib.yolo_read_tensor(self.h, t, B, out.ctypes.data) != 0:
            raise RuntimeError("yolo_read_tensor failed")
        return out

    def write(self, t: int, arr: np.ndarray):
        arr = np.ascontiguousarray(arr, dtype=np.float16)
        H, W, Cc = self.tensor_shape(t)
        assert arr.shape[1:] == (H, W, Cc), (arr.shape, (H, W, Cc))
        if self.lib.yolo_write_tensor(self.h, t, arr.shape[0], arr.ctypes.data) != 0:
            raise RuntimeError("yolo_write_tensor failed")

    def read_slots(self, t: int, first: int, n: int = 1) -> np.ndarray:
        """Tensor t of images first .. first+n-1 as [n, H, W, C] fp16."""
        H, W, Cc = self.tensor_shape(t)
        out = np.empty((n, H, W, Cc), np.float16)
        if self.lib.yolo_read_tensor_slots(self.h, t, first, n, out.ctypes.data) != 0:
            raise RuntimeError("yolo_read_tensor_slots failed")
        return out

    def write_slots(self, t: int, first: int, arr: np.ndarray):
        arr = np.ascontiguousarray(arr, dtype=np.float16)
        H, W, Cc = self.tensor_shape(t)
        assert arr.shape[1:] == (H, W, Cc), (arr.shape, (H, W, Cc))
        if self.lib.yolo_write_tensor_slots(self.h, t, first, arr.shape[0], arr.ctypes.data) != 0:
            raise RuntimeError("yolo_write_tensor_slots failed")

    def run_op(self, k: int, B: int = 1):
        if self.lib.yolo_run_op(self.h, k, B) != 0:
            raise RuntimeError(f"yolo_run_op({k}) failed")

    def run_post(self, B: int = 1):
        if self.lib.yolo_run_post(self.h, B) != 0:
            raise RuntimeError("yolo_run_post failed")

    def op_config(self, k: int) -> int:
        return self.lib.yolo_op_config(self.h, k)

    def set_op_config(self, k: int, cfg: int):
        if self.lib.yolo_set_op_config(self.h, k, cfg) != 0:
            raise ValueError((k, cfg))

    def op_split(self, k: int) -> int:
        return self.lib.yolo_op_split(self.h, k)

    def set_op_split(self, k: int, splits: int):
        if self.lib.yolo_set_op_split(self.h, k, splits) != 0:
            raise ValueError((k, splits))

    def op_tail(self, k: int) -> int:
        return self.lib.yolo_op_tail(self.h, k)

    def set_op_tail(self, k: int, tail: int):
        if self.lib.yolo_set_op_tail(self.h, k, tail) != 0:
            raise ValueError((k, tail))

    # -- frame API
    def set_thresholds(self, conf=0.25, iou=0.45, max_det=300):
        if self.lib.yolo_set_thresholds(self.h, conf, iou, max_det) != 0:
            raise ValueError((conf, iou, max_det))

    def preprocess(self, dev_ptr: int, h: int, w: int, slot: int = 0):
        self.lib.yolo_preprocess(self.h, dev_ptr, h, w, slot)

    def run(self, B: int = 1):
        self.lib.yolo_run(self.h, B)

    def run_async(self, B: int = 1):
        """Launches the batch-B graph on the engine stream and returns; `sync` waits."""
        self.lib.yolo_run_async(self.h, B)

    def sync(self):
        self.lib.yolo_sync(self.h)

    def _records(self, fn, struct, nf: int, slot: int, cap: int) -> np.ndarray:
        # the C structs are nf-1 floats then an int: read them through one reused float32
        # buffer (a per-record Python loop costs more than the frame's NMS)
        key = (struct, cap)
        buf = self._getbuf.get(key)
        if buf is None:
            buf = self._getbuf[key] = np.empty((cap, nf), np.float32)
        n = fn(self.h, slot, buf.ctypes.data_as(C.POINTER(struct)), cap)
        out = buf[:n].astype(np.float64)
        out[:, nf - 1] = buf[:n].view(np.int32)[:, nf - 1]
        return out

    def get(self, slot: int = 0, cap: int = MAX_OUT) -> np.ndarray:
        """Survivors as rows (x1, y1, x2, y2, score, cls) in original-image coords."""
        return self._records(self.lib.yolo_get, YoloDet, 6, slot, cap)

    def _records_batch(self, fn, struct, nf: int, B: int, cap: int) -> list[np.ndarray]:
        key = (struct, cap * B)
        buf = self._getbuf.get(key)
        if buf is None:
            buf = self._getbuf[key] = np.empty((B * cap, nf), np.float32)
        counts = np.zeros(B, np.int32)
        fn(self.h, B, buf.ctypes.data_as(C.POINTER(struct)), cap, counts.ctypes.data_as(C.POINTER(C.c_int)))
        allr = buf.astype(np.float64)
        allr[:, nf - 1] = buf.view(np.int32)[:, nf - 1]
        return [allr[s * cap:s * cap + int(counts[s])] for s in range(B)]

    def get_batch(self, B: int, cap: int = MAX_OUT) -> list[np.ndarray]:
        """`get` of slots 0..B-1 in one call."""
        return self._records_batch(self.lib.yolo_get_batch, YoloDet, 6, B, cap)

    def get_obb_batch(self, B: int, cap: int = MAX_OUT) -> list[np.ndarray]:
        """`get_obb` of slots 0..B-1 in one call."""
        return self._records_batch(self.lib.yolo_get_obb_batch, YoloObbDet, 7, B, cap)

    def stage_frames(self, host_ptrs, heights, widths, fmt: int = PIXEL_BGR, first_slot: int = 0):
        """Copies raw frames of pixel layout `fmt` (PIXEL_BGR, PIXEL_RGBX) from host memory
        (pinned: asynchronous) into the handle's staging buffers and letterboxes them into
        slots first_slot.. (async on the stream)."""
        n = len(host_ptrs)
        p = (C.c_void_p * n)(*host_ptrs)
        hh = (C.c_int * n)(*heights)
        ww = (C.c_int * n)(*widths)
        if self.lib.yolo_stage_frames(self.h, n, p, hh, ww, fmt, first_slot) != 0:
            raise RuntimeError("yolo_stage_frames failed")

    def _jpeg(self, fn, streams, first_slot):
        n = len(streams)
        data = (C.c_char_p * n)(*streams)
        sizes = (C.c_size_t * n)(*[len(b) for b in streams])
        hh, ww, st = (C.c_int * n)(), (C.c_int * n)(), (C.c_int * n)()
        if fn(self.h, n, data, sizes, first_slot, hh, ww, st) < 0:
            raise RuntimeError(f"{fn.__name__} failed")
        return [(st[i], hh[i], ww[i]) for i in range(n)]

    def stage_jpeg(self, streams: list[bytes], first_slot: int = 0):
        """Decodes JPEG streams on the engine (entropy decoding on the library's threads, the
        rest on the GPU) and letterboxes them into slots first_slot..; returns per-stream
        (status, height, width), status JPEG_STAGED / JPEG_UNSUPPORTED / JPEG_INVALID."""
        return self._jpeg(self.lib.yolo_stage_jpeg, streams, first_slot)

    def decode_jpeg(self, streams: list[bytes], first_slot: int = 0):
        """The decode half of stage_jpeg: the slots' staging frames only (no letterbox, slot
        geometry unchanged); letterbox_decoded finishes the staging."""
        return self._jpeg(self.lib.yolo_decode_jpeg, streams, first_slot)

    def decode_tickets(self, tickets: list, first_slot: int = 0):
        """decode_jpeg for tickets from jpeg_submit (consumed, whatever the outcome): the
        entropy decoding already ran at submission."""
        n = len(tickets)
        tk = (C.c_void_p * n)(*tickets)
        hh, ww, st = (C.c_int * n)(), (C.c_int * n)(), (C.c_int * n)()
        if self.lib.yolo_decode_tickets(self.h, n, tk, first_slot, hh, ww, st) < 0:
            raise RuntimeError("yolo_decode_tickets failed")
        return [(st[i], hh[i], ww[i]) for i in range(n)]

    def letterbox_decoded(self, n: int, first_slot: int = 0) -> int:
        r = self.lib.yolo_letterbox_decoded(self.h, n, first_slot)
        if r < 0:
            raise RuntimeError("yolo_letterbox_decoded failed")
        return r

    def get_obb(self, slot: int = 0, cap: int = MAX_OUT) -> np.ndarray:
        """OBB survivors as rows (cx, cy, w, h, theta, score, cls) in original-image coords."""
        return self._records(self.lib.yolo_get_obb, YoloObbDet, 7, slot, cap)

    def preprocess_cls(self, dev_ptr: int, h: int, w: int, slot: int = 0):
        self.lib.yolo_preprocess_cls(self.h, dev_ptr, h, w, slot)

    def get_cls(self, slot: int = 0, k: int = 5) -> tuple[np.ndarray, np.ndarray]:
        """Top-k (class ids, probabilities) of a classify handle's slot."""
        ids = np.empty(k, np.int32)
        probs = np.empty(k, np.float32)
        n = self.lib.yolo_get_cls(self.h, slot, ids.ctypes.data_as(C.POINTER(C.c_int)),
                                  probs.ctypes.data_as(C.POINTER(C.c_float)), k)
        return ids[:n].copy(), probs[:n].copy()

    def raw_count(self, slot: int = 0) -> int:
        return self.lib.yolo_raw_count(self.h, slot)

    def slot_geom(self, slot: int = 0):
        s, t, l = C.c_float(), C.c_int(), C.c_int()
        self.lib.yolo_slot_geom(self.h, slot, C.byref(s), C.byref(t), C.byref(l))
        return s.value, t.value, l.value

    def mask_dim(self):
        ph, pw = C.c_int(), C.c_int()
        self.lib.yolo_mask_dim(self.h, C.byref(ph), C.byref(pw))
        return ph.value, pw.value

    def get_mask(self, slot: int, det: int) -> np.ndarray | None:
        ph, pw = self.mask_dim()
        out = np.empty((ph, pw), np.uint8)
        if self.lib.yolo_get_mask(self.h, slot, det, out.ctypes.data) != 0:
            return None
        return out

    def exec_ms(self, B: int = 1) -> float:
        return self.lib.yolo_exec_ms(self.h, B)

    def task(self) -> int:
        return self.lib.yolo_task(self.h)

    def frame_graph(self, dev_ptrs, heights, widths, host_ptrs=None):
        B = len(dev_ptrs)
        dv = (C.c_void_p * B)(*dev_ptrs)
        hv = (C.c_void_p * B)(*host_ptrs) if host_ptrs is not None else None
        hs = (C.c_int * B)(*heights)
        ws = (C.c_int * B)(*widths)
        if self.lib.yolo_frame_graph(self.h, B, dv, hv, hs, ws) != 0:
            raise RuntimeError("yolo_frame_graph failed")

    def frame_run(self):
        if self.lib.yolo_frame_run(self.h) != 0:
            raise RuntimeError("yolo_frame_run failed")

    def time_graph(self, which: int, B: int, iters: int) -> float:
        ms = self.lib.yolo_time_graph(self.h, which, B, iters)
        if ms < 0:
            raise RuntimeError("yolo_time_graph failed")
        return ms

    def profile_ops(self, B: int, iters: int) -> np.ndarray:
        n = self.num_ops
        out = (C.c_float * n)()
        if self.lib.yolo_profile_ops(self.h, B, iters, out) != 0:
            raise RuntimeError("yolo_profile_ops failed")
        return np.array(out, np.float64)

    def profile_units(self, B: int, iters: int, reps: int) -> np.ndarray:
        """Kernel ms per launch unit (reported on its first op), units repeated back to back."""
        n = self.num_ops
        out = (C.c_float * n)()
        if self.lib.yolo_profile_units(self.h, B, iters, reps, out) != 0:
            raise RuntimeError("yolo_profile_units failed")
        return np.array(out, np.float64)

    def num_units(self) -> int:
        return self.lib.yolo_num_units(self.h)

    def run_unit(self, u: int, B: int):
        if self.lib.yolo_run_unit(self.h, u, B) != 0:
            raise RuntimeError(f"yolo_run_unit({u}) failed")

    def spin_failures(self) -> int:
        """Bounded waits that expired in wave-specialised kernels on this device (0 when every
        launch was sound)."""
        return self.lib.yolo_spin_failures(self.h)

    def marker(self):
        if self.lib.yolo_marker(self.h) != 0:
            raise RuntimeError("yolo_marker failed")

    def op_unit(self, k: int) -> int:
        """Launch unit of op k (ops of one unit share a launch), -1 if no unit launches it."""
        return self.lib.yolo_op_unit(self.h, k)

    def profile_stages(self, iters: int) -> dict:
        """ms of the frame graph's letterbox, decode, NMS and mask stages (stream-ordered)."""
        out = (C.c_float * 4)()
        if self.lib.yolo_profile_stages(self.h, iters, out) != 0:
            raise RuntimeError("yolo_profile_stages failed")
        return dict(letterbox=out[0], decode=out[1], nms=out[2], masks=out[3])

    def upload(self, buf: DeviceBuffer, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= buf.nbytes
        if self.lib.yolo_copy_h2d(self.h, buf.ptr, arr.ctypes.data, arr.nbytes) != 0:
            raise RuntimeError("yolo_copy_h2d failed")


def detect_static(levels, B: int, nc: int, conf: float, iou: float, max_det: int, dets_ptr: int,
                  counts_ptr: int, raw_ptr: int | None = None, stream: int | None = None) -> int:
    """yolo_detect_static: decode + NMS of device head tensors with no allocation.
    `levels`: (box_ptr, cls_ptr, H, W, stride, box_stride, box_off, cls_stride, cls_off) per
    level.  Returns the entry point's status (0 or -1)."""
    lib = load()
    arr = (YoloHeadLevel * len(levels))(*[YoloHeadLevel(*lv) for lv in levels])
    return lib.yolo_detect_static(arr, len(levels), B, nc, conf, iou, max_det, dets_ptr, counts_ptr,
                                  raw_ptr, stream)


def graph_check(model_dir: str) -> tuple[int, str]:
    lib = load()
    err = C.create_string_buffer(1024)
    n = lib.yolo_graph_check(model_dir.encode(), err, 1024)
    return n, err.value.decode()
