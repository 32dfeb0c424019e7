"""JPEG decode on the CPU: the oracle's restatement (oracle/jpeg.py) pixel for pixel against
PIL / libjpeg-turbo over a corpus of sizes, qualities, chroma subsamplings, Huffman tables,
restart intervals and grayscale; the zigzag and IDCT pinned by their closed forms; and the
library's native entropy decoder (yolo_jpeg_coefficients, host code only) coefficient for
coefficient against the oracle's."""
import io

import numpy as np
import pytest
from PIL import Image

import modelgen
from oracle import jpeg


def _encode(rgb, mode="RGB", **kw):
    buf = io.BytesIO()
    im = Image.fromarray(rgb)
    if mode == "L":
        im = im.convert("L")
    im.save(buf, "JPEG", **kw)
    return buf.getvalue()


def _pil_rgb(data):
    with Image.open(io.BytesIO(data)) as im:
        return np.asarray(im.convert("RGB"))


def _frame(h, w, seed):
    """Natural-looking content (smooth fields and edges) plus noise, so every coefficient
    band and both signs occur."""
    rng = np.random.default_rng(seed)
    img = modelgen.synth_frame(h, w, max(1, (h * w) // 900), seed)[..., ::-1]
    noise = rng.integers(-20, 21, img.shape)
    return np.clip(img.astype(np.int32) + noise, 0, 255).astype(np.uint8)


CORPUS = [
    # (h, w, encoder options)
    (48, 64, dict(quality=90, subsampling=2)),
    (37, 53, dict(quality=90, subsampling=2)),
    (37, 53, dict(quality=75, subsampling=1)),
    (37, 53, dict(quality=95, subsampling=0)),
    (41, 30, dict(quality=100, subsampling=2)),
    (41, 30, dict(quality=20, subsampling=2)),
    (33, 70, dict(quality=85, subsampling=2, optimize=True)),
    (40, 56, dict(quality=90, subsampling=2, restart_marker_blocks=3)),
    (40, 56, dict(quality=90, subsampling=0, restart_marker_rows=1)),
    (17, 9, dict(quality=90, subsampling=0)),
    (9, 17, dict(quality=50, subsampling=1)),
    (64, 80, dict(quality=90, mode="L")),
    (23, 31, dict(quality=60, mode="L", restart_marker_blocks=2)),
]


@pytest.mark.parametrize("case", range(len(CORPUS)))
def test_oracle_matches_pil(case):
    h, w, kw = CORPUS[case]
    kw = dict(kw)
    mode = kw.pop("mode", "RGB")
    data = _encode(_frame(h, w, 40 + case), mode, **kw)
    got = jpeg.decode(data)
    want = _pil_rgb(data)
    assert got.shape == want.shape == (h, w, 3)
    assert np.array_equal(got, want), f"{int((got != want).sum())} samples differ, max {np.abs(got.astype(int) - want).max()}"


def test_oracle_440_matches_pil():
    """4:4:0 (chroma halved vertically only; PIL's encoder does not write it): a 4:2:2 stream
    with each component's H and V sampling factors swapped and the frame's width and height
    swapped is a valid 4:4:0 stream (of the transposed block layout); both decoders must
    agree on it."""
    rgb = _frame(36, 50, 7)
    data = _encode(np.ascontiguousarray(rgb), quality=90, subsampling=1)     # 4:2:2 = h2v1
    assert np.array_equal(jpeg.decode(data), _pil_rgb(data))
    hdr = jpeg.parse(data)
    sof = data.index(b"\xff\xc0")
    b = bytearray(data)
    nc = b[sof + 9]
    for i in range(nc):
        f = b[sof + 11 + 3 * i]
        b[sof + 11 + 3 * i] = (f & 15) << 4 | f >> 4
    h, w = hdr["frame"]["H"], hdr["frame"]["W"]
    b[sof + 5:sof + 7], b[sof + 7:sof + 9] = w.to_bytes(2, "big"), h.to_bytes(2, "big")
    data2 = bytes(b)
    got, want = jpeg.decode(data2), _pil_rgb(data2)
    assert got.shape == want.shape and np.array_equal(got, want)


def test_unsupported_streams():
    rgb = _frame(24, 24, 3)
    with pytest.raises(jpeg.Unsupported):
        jpeg.layout(jpeg.parse(_encode(rgb, quality=90, progressive=True)))
    with pytest.raises(ValueError):
        jpeg.parse(b"\x89PNG\r\n\x1a\n")


def test_zigzag_and_idct_closed_forms():
    # zigzag: a permutation whose k-th entry lies on anti-diagonal r + c nondecreasing in k
    zz = jpeg.ZZ
    assert sorted(zz.tolist()) == list(range(64))
    diag = (zz // 8) + (zz % 8)
    assert np.all(np.diff(diag) >= 0)
    assert zz[:6].tolist() == [0, 1, 8, 16, 9, 2]
    # IDCT: a DC-only block is flat at round(dc * q / 8) + 128; a single AC term follows the
    # cosine basis to within the fixed-point rounding (one level)
    q = np.ones(64, np.int32)
    c = np.zeros((1, 1, 64), np.int32)
    c[0, 0, 0] = 80
    assert np.all(jpeg.idct_plane(c, q) == 138)
    for k in (1, 8, 9, 27, 63):
        c = np.zeros((1, 1, 64), np.int32)
        c[0, 0, k] = 64
        u, v = k // 8, k % 8
        x = np.arange(8)
        cu = np.cos((2 * x + 1) * u * np.pi / 16) * (np.sqrt(0.5) if u == 0 else 1.0)
        cv = np.cos((2 * x + 1) * v * np.pi / 16) * (np.sqrt(0.5) if v == 0 else 1.0)
        ref = 0.25 * 64 * np.outer(cu, cv) + 128
        got = jpeg.idct_plane(c, q).astype(np.float64)
        assert np.abs(got - ref).max() <= 1.0, k
    # range limit: clamp over the valid span, wrap outside it
    v = np.array([-129, -128, -1, 0, 127, 128, 383, 511, 512, 895, 896])
    assert jpeg.range_limit(v).tolist() == [0, 0, 127, 128, 255, 255, 255, 255, 0, 0, 0]


def test_colour_tables_match_formula():
    """Each table entry is the BT.601 term rounded to an integer, within the 2^-16 error of its
    fixed-point constant times |x| <= 128 (a wrong constant or sign is off by far more)."""
    crr, cbb, crg, cbg = jpeg.ycc_tables()
    x = np.arange(256) - 128
    tol = 0.5 + 128 * 2.0 ** -16 * 2
    assert np.abs(crr - 1.402 * x).max() <= tol
    assert np.abs(cbb - 1.772 * x).max() <= tol
    g = (cbg[:, None] + crg[None, :]) >> 16
    ref = -0.34414 * x[:, None] - 0.71414 * x[None, :]
    assert np.abs(g - ref).max() <= tol


# ------------------------------------------------------------------ the library's entropy decoder
def _lib_coefs(data):
    import yolort
    return yolort.jpeg_coefficients(data)


def _oracle_coefs(data):
    return np.concatenate([c.reshape(-1) for c in jpeg.coefficients(data)]).astype(np.int16)


@pytest.mark.parametrize("case", range(len(CORPUS)))
def test_native_entropy_decode_matches_oracle(case):
    import yolort
    h, w, kw = CORPUS[case]
    kw = dict(kw)
    mode = kw.pop("mode", "RGB")
    data = _encode(_frame(h, w, 40 + case), mode, **kw)
    assert yolort.jpeg_probe(data) == (1, h, w)
    got = _lib_coefs(data)
    want = _oracle_coefs(data)
    assert got is not None and got.shape == want.shape
    assert np.array_equal(got, want)


def test_native_entropy_decode_large_and_extremes():
    """A 640x480 photo-like frame at quality 100 (long codes, large coefficients) and a
    flat frame (EOB-only blocks) decode to the oracle's coefficients."""
    import yolort
    for rgb, q in ((_frame(480, 640, 9), 100), (np.full((16, 24, 3), 77, np.uint8), 90)):
        data = _encode(rgb, quality=q, subsampling=2)
        assert np.array_equal(_lib_coefs(data), _oracle_coefs(data))


def test_native_probe_and_failures():
    import yolort
    rgb = _frame(24, 40, 1)
    assert yolort.jpeg_probe(_encode(rgb, quality=90, progressive=True))[0] == 0
    assert yolort.jpeg_probe(b"\x89PNG\r\n\x1a\n" + bytes(64))[0] == -1
    assert yolort.jpeg_probe(b"")[0] == -1
    assert _lib_coefs(_encode(rgb, quality=90, progressive=True)) is None
    data = _encode(rgb, quality=90)
    # truncated inside the entropy-coded data: corrupt (PIL refuses it as well)
    with pytest.raises(ValueError):
        _lib_coefs(data[:len(data) - 200])
    # headers cut short
    assert yolort.jpeg_probe(data[:100])[0] == -1
    # garbage entropy data decodes deterministically or is rejected, never crashes
    rng = np.random.default_rng(3)
    hdr = jpeg.parse(data)
    for _ in range(20):
        junk = bytes(rng.integers(0, 256, 300, dtype=np.uint8).tolist())
        try:
            _lib_coefs(data[:hdr["offset"]] + junk + b"\xff\xd9")
        except ValueError:
            pass


def test_host_only_jpeg_library():
    """libyolo11_jpeg.so (what server front-end processes load) needs no HIP runtime and reads
    every stream's headers as the engine library does."""
    import shutil
    import subprocess
    import yolort
    import yoloserve
    path = yolort.LIB_PATH.replace("libyolo11_amd.so", "libyolo11_jpeg.so")
    if shutil.which("readelf"):
        needed = subprocess.run(["readelf", "-d", path], capture_output=True, text=True, check=True).stdout
        assert "NEEDED" in needed and "amdhip" not in needed and "hsa" not in needed
    streams = [_encode(_frame(h, w, 40 + i), **{k: v for k, v in kw.items() if k != "mode"})
               for i, (h, w, kw) in enumerate(CORPUS[:6])]
    streams += [_encode(_frame(24, 40, 1), quality=90, progressive=True), b"\x89PNG\r\n\x1a\n" + bytes(40), b""]
    for s in streams:
        r, h, w = yolort.jpeg_probe(s)
        assert yoloserve.jpeg_dims(s) == ((h, w) if r == 1 else None)


def _declare_size(data: bytes, h: int, w: int) -> bytes:
    """The stream with its SOF0 frame header rewritten to declare h x w pixels (the entropy
    data is left as it is, far too short for such a frame)."""
    i = data.index(b"\xff\xc0")
    b = bytearray(data)
    b[i + 5:i + 7] = h.to_bytes(2, "big")
    b[i + 7:i + 9] = w.to_bytes(2, "big")
    return bytes(b)


def test_huge_declared_frame_is_refused():
    """A few hundred bytes declaring a 16384 x 16384 4:4:4 frame (1.5 GB of coefficients if
    accepted) is outside the engine's set: probe 0, no coefficients, no ticket, so the
    server hands it to PIL, whose decompression-bomb check refuses it for that request only.
    The cap is the library's maximum frame size, PIL's MAX_IMAGE_PIXELS by default."""
    import yolort
    data = _encode(_frame(16, 16, 2), quality=90, subsampling=0)
    assert yolort.jpeg_probe(data) == (1, 16, 16)
    cap = yolort.jpeg_max_pixels()
    assert cap == Image.MAX_IMAGE_PIXELS == 89478485
    huge = _declare_size(data, 16384, 16384)
    assert len(huge) < 2048
    assert yolort.jpeg_probe(huge)[0] == 0
    assert _lib_coefs(huge) is None
    assert yolort.jpeg_submit(huge) is None
    # the cap is inclusive, and configurable
    side = int(np.sqrt(cap))
    assert yolort.jpeg_probe(_declare_size(data, side, side)) == (1, side, side)
    assert yolort.jpeg_probe(_declare_size(data, side + 1, side + 1))[0] == 0
    try:
        assert yolort.jpeg_max_pixels(1 << 30) == 1 << 30
        assert yolort.jpeg_probe(huge) == (1, 16384, 16384)
        assert yolort.jpeg_max_pixels(255) == 255
        assert yolort.jpeg_probe(data)[0] == 0
        assert yolort.jpeg_max_pixels(0) == 255           # 0 reads without setting
    finally:
        yolort.jpeg_max_pixels(cap)
    assert yolort.jpeg_probe(data) == (1, 16, 16)
