"""CPU restatement of the JPEG decode the engine's GPU path performs (test infrastructure only:
imported by tests/, never by the product).

The reference server decodes JPEG requests with nvJPEG -- entropy decoding on CPU threads, the
rest on the GPU -- and everything else with stb_image (server/serve.cpp:71-131).  nvJPEG is
closed and absent here; the pixel contract this build holds is that of the decoder its own
server falls back to, PIL 12.2 over libjpeg-turbo (bundled with Pillow, API 6.2), whose
algorithms are published:

* ITU-T T.81 (JPEG) baseline / extended-sequential Huffman decoding: canonical code
  construction (Annex C), DC differences and AC run/size pairs with EXTEND (F.2.2), restart
  intervals (F.2.2.5), interleaved MCUs of Hi x Vi blocks per component (A.2.3);
* the IJG "islow" integer IDCT (Loeffler-Ligtenberg-Moschytz, 13-bit constants, 2 extra bits
  after the column pass, rounding shifts) and its range-limit table, which maps the IDCT
  output v to clamp(v + 128) for v in [-128, 511] and wraps beyond that (v & 1023);
* IJG "fancy" chroma upsampling: triangle filters 3/4 + 1/4, with the rounding biases that
  alternate between the two output samples, edge samples special-cased, vertical context rows
  replicated at the component's top and bottom;
* JFIF YCbCr -> RGB with 16-bit fixed-point tables (ITU-R BT.601 full range).

Pinned by tests/test_jpeg.py: every pixel equals PIL's decode over a corpus of sizes,
qualities, chroma subsamplings (4:4:4, 4:2:2, 4:2:0, 4:4:0), optimized Huffman tables,
restart intervals and grayscale, so a wrong constant, bias or edge rule fails there.
The entropy decoder is pure Python (small images only); IDCT, upsampling and colour are numpy.
"""
from __future__ import annotations

import numpy as np


class Unsupported(Exception):
    """A valid JPEG outside the GPU path (progressive, arithmetic, 12-bit, CMYK, ...)."""


def zigzag() -> np.ndarray:
    """zz[k] = natural (row-major) index of the k-th coefficient in zigzag order (T.81 A.3.6)."""
    order = []
    for s in range(15):
        cells = [(i, s - i) for i in range(8) if 0 <= s - i < 8]
        if s % 2 == 0:
            cells.reverse()                  # even diagonals run bottom-left to top-right
        order += [r * 8 + c for r, c in cells]
    return np.array(order, np.int32)


ZZ = zigzag()


# ------------------------------------------------------------------ headers
def parse(data: bytes) -> dict:
    """Markers up to and including the first SOS: frame, tables, restart interval, scan, and
    the offset of the entropy-coded data.  Raises Unsupported / ValueError."""
    if len(data) < 4 or data[0] != 0xFF or data[1] != 0xD8:
        raise ValueError("not a JPEG")
    q, dc, ac = {}, {}, {}
    frame, ri, jfif, adobe = None, 0, False, None
    p = 2
    while p + 4 <= len(data):
        if data[p] != 0xFF:
            raise ValueError("marker expected")
        m = data[p + 1]
        if m == 0xFF:
            p += 1
            continue
        n = data[p + 2] << 8 | data[p + 3]
        seg = data[p + 4:p + 2 + n]
        if len(seg) != n - 2:
            raise ValueError("truncated segment")
        if m in (0xC0, 0xC1):
            if seg[0] != 8:
                raise Unsupported("sample precision")
            H, W, nc = seg[1] << 8 | seg[2], seg[3] << 8 | seg[4], seg[5]
            comps = [dict(id=seg[6 + 3 * i], h=seg[7 + 3 * i] >> 4, v=seg[7 + 3 * i] & 15, tq=seg[8 + 3 * i])
                     for i in range(nc)]
            frame = dict(H=H, W=W, comps=comps)
        elif m in (0xC2, 0xC3, 0xC5, 0xC6, 0xC7, 0xC9, 0xCA, 0xCB, 0xCD, 0xCE, 0xCF):
            raise Unsupported(f"SOF{m - 0xC0}")
        elif m == 0xC4:
            i = 0
            while i < len(seg):
                tc, th = seg[i] >> 4, seg[i] & 15
                counts = list(seg[i + 1:i + 17])
                syms = list(seg[i + 17:i + 17 + sum(counts)])
                (dc if tc == 0 else ac)[th] = (counts, syms)
                i += 17 + sum(counts)
        elif m == 0xDB:
            i = 0
            while i < len(seg):
                pq, tq = seg[i] >> 4, seg[i] & 15
                if pq == 0:
                    vals = list(seg[i + 1:i + 65])
                    i += 65
                else:
                    vals = [seg[i + 1 + 2 * k] << 8 | seg[i + 2 + 2 * k] for k in range(64)]
                    i += 129
                t = np.zeros(64, np.int32)
                t[ZZ] = vals                     # stored in zigzag order
                q[tq] = t
        elif m == 0xDD:
            ri = seg[0] << 8 | seg[1]
        elif m == 0xE0 and seg[:5] == b"JFIF\0":
            jfif = True
        elif m == 0xEE and seg[:5] == b"Adobe" and len(seg) >= 12:
            adobe = seg[11]
        elif m == 0xDA:
            if frame is None:
                raise ValueError("SOS before SOF")
            ns = seg[0]
            scomps = [(seg[1 + 2 * i], seg[2 + 2 * i] >> 4, seg[2 + 2 * i] & 15) for i in range(ns)]
            ss, se, ahl = seg[1 + 2 * ns], seg[2 + 2 * ns], seg[3 + 2 * ns]
            if (ss, se, ahl) != (0, 63, 0):
                raise Unsupported("spectral selection")
            return dict(frame=frame, q=q, dc=dc, ac=ac, ri=ri, jfif=jfif, adobe=adobe,
                        scan=scomps, offset=p + 2 + n)
        p += 2 + n
    raise ValueError("no scan")


def layout(hdr: dict) -> dict:
    """Checks the frame is inside the GPU path and derives its geometry (T.81 A.1.1, A.2)."""
    fr = hdr["frame"]
    comps = fr["comps"]
    nc = len(comps)
    if nc not in (1, 3) or fr["H"] < 1 or fr["W"] < 1:
        raise Unsupported("components / size")
    if [c[0] for c in hdr["scan"]] != [c["id"] for c in comps]:
        raise Unsupported("multi-scan sequential")
    if nc == 3:
        # colour space as libjpeg infers it: JFIF means YCbCr; else an Adobe marker's
        # transform flag (0 = RGB); else component ids 'R', 'G', 'B' mean RGB
        ids = [c["id"] for c in comps]
        if not hdr["jfif"] and (hdr["adobe"] == 0 if hdr["adobe"] is not None else ids == [82, 71, 66]):
            raise Unsupported("RGB colour space")
    hmax = max(c["h"] for c in comps)
    vmax = max(c["v"] for c in comps)
    H, W = fr["H"], fr["W"]
    out = []
    for i, c in enumerate(comps):
        if c["tq"] not in hdr["q"]:
            raise ValueError("missing quantization table")
        fh, fv = hmax // c["h"], vmax // c["v"]
        if nc == 1:
            fh = fv = 1
        elif hmax % c["h"] or vmax % c["v"] or (fh, fv) not in ((1, 1), (2, 1), (2, 2), (1, 2)):
            raise Unsupported("sampling factors")
        if i == 0 and (fh, fv) != (1, 1):
            raise Unsupported("subsampled luma")
        cw = -(-W * c["h"] // hmax) if nc > 1 else W
        ch = -(-H * c["v"] // vmax) if nc > 1 else H
        if (fh == 2 and cw < 3) or (fv == 2 and ch < 3):
            raise Unsupported("chroma plane too small")
        out.append(dict(cw=cw, ch=ch, fh=fh, fv=fv))
    if nc == 1:
        mx, my = -(-W // 8), -(-H // 8)
        out[0].update(bw=mx, bh=my)
    else:
        mx, my = -(-W // (8 * hmax)), -(-H // (8 * vmax))
        for c, o in zip(comps, out):
            o.update(bw=mx * c["h"], bh=my * c["v"])
    return dict(H=H, W=W, nc=nc, hmax=hmax, vmax=vmax, mcux=mx, mcuy=my, comps=out)


# ------------------------------------------------------------------ entropy decoding
def _table(spec):
    """{(length, code): symbol} of a canonical Huffman table (T.81 C.2)."""
    counts, syms = spec
    t, code, k = {}, 0, 0
    for length in range(1, 17):
        for _ in range(counts[length - 1]):
            t[(length, code)] = syms[k]
            k += 1
            code += 1
        code <<= 1
    return t


class _Bits:
    """MSB-first bit reader over entropy-coded bytes with 0xFF00 stuffing; a marker (or the
    end of data) yields zero bits, as libjpeg does for truncated data."""

    def __init__(self, data: bytes, p: int):
        self.d, self.p, self.acc, self.n = data, p, 0, 0

    def bit(self) -> int:
        if self.n == 0:
            b = 0
            if self.p < len(self.d):
                b = self.d[self.p]
                if b == 0xFF:
                    nxt = self.d[self.p + 1] if self.p + 1 < len(self.d) else 0xD9
                    if nxt == 0x00:
                        self.p += 2
                    else:
                        b = 0               # a marker: do not consume, feed zeros
                else:
                    self.p += 1
            self.acc, self.n = b, 8
        self.n -= 1
        return (self.acc >> self.n) & 1

    def bits(self, s: int) -> int:
        v = 0
        for _ in range(s):
            v = v << 1 | self.bit()
        return v

    def restart(self):
        """Discards the partial byte and the RSTn marker that must follow."""
        self.n = 0
        if self.p + 1 < len(self.d) and self.d[self.p] == 0xFF and 0xD0 <= self.d[self.p + 1] <= 0xD7:
            self.p += 2

    def decode(self, t) -> int:
        code = 0
        for length in range(1, 17):
            code = code << 1 | self.bit()
            s = t.get((length, code))
            if s is not None:
                return s
        raise ValueError("bad Huffman code")


def _extend(v: int, s: int) -> int:
    return v - (1 << s) + 1 if s and v < (1 << (s - 1)) else v


def coefficients(data: bytes, hdr: dict | None = None, lay: dict | None = None) -> list[np.ndarray]:
    """Quantized coefficients per component, int32 [bh, bw, 64] in natural order."""
    hdr = hdr or parse(data)
    lay = lay or layout(hdr)
    comps = hdr["frame"]["comps"]
    scan = {cid: (td, ta) for cid, td, ta in hdr["scan"]}
    tabs = [(_table(hdr["dc"][scan[c["id"]][0]]), _table(hdr["ac"][scan[c["id"]][1]])) for c in comps]
    out = [np.zeros((o["bh"], o["bw"], 64), np.int32) for o in lay["comps"]]
    bits = _Bits(data, hdr["offset"])
    pred = [0] * len(comps)

    def block(ci, by, bx):
        dct, act = tabs[ci]
        s = bits.decode(dct)
        pred[ci] += _extend(bits.bits(s), s)
        blk = out[ci][by, bx]
        blk[0] = pred[ci]
        k = 1
        while k < 64:
            rs = bits.decode(act)
            r, s = rs >> 4, rs & 15
            if s == 0:
                if r != 15:
                    break
                k += 16
                continue
            k += r
            if k > 63:
                raise ValueError("coefficient index out of range")
            blk[ZZ[k]] = _extend(bits.bits(s), s)
            k += 1

    nc, ri = lay["nc"], hdr["ri"]
    if nc == 1:
        units = [(0, by, bx) for by in range(lay["comps"][0]["bh"]) for bx in range(lay["comps"][0]["bw"])]
        mcus = [[u] for u in units]
    else:
        mcus = []
        for my in range(lay["mcuy"]):
            for mx in range(lay["mcux"]):
                mcus.append([(ci, my * c["v"] + y, mx * c["h"] + x) for ci, c in enumerate(comps)
                             for y in range(c["v"]) for x in range(c["h"])])
    for m, units in enumerate(mcus):
        if ri and m and m % ri == 0:
            bits.restart()
            pred = [0] * len(comps)
        for u in units:
            block(*u)
    return out


# ------------------------------------------------------------------ IDCT
# 13-bit fixed-point IDCT multipliers, FIX(x) = round(x * 2^13), named by their real values
# (sqrt(2) times sums of the cosines c_k = cos(k pi / 16) in the LLM flowgraph)
FIX = {name: int(float(name.replace("_", ".")) * 8192 + 0.5) for name in (
    "0_298631336", "0_390180644", "0_541196100", "0_765366865", "0_899976223", "1_175875602",
    "1_501321110", "1_847759065", "1_961570560", "2_053119869", "2_562915447", "3_072711026")}
CONST_BITS, PASS1_BITS = 13, 2


def _idct_1d(x0, x1, x2, x3, x4, x5, x6, x7, shift):
    """One 8-point islow pass over int64 arrays; outputs are rounded right shifts by `shift`
    of the 13-bit fixed-point results (inputs x_k are the k-th frequency terms)."""
    z1 = (x2 + x6) * FIX["0_541196100"]
    t2 = z1 - x6 * FIX["1_847759065"]
    t3 = z1 + x2 * FIX["0_765366865"]
    t0 = (x0 + x4) << CONST_BITS
    t1 = (x0 - x4) << CONST_BITS
    e10, e13, e11, e12 = t0 + t3, t0 - t3, t1 + t2, t1 - t2
    a0, a1, a2, a3 = x7, x5, x3, x1
    z1, z2, z3, z4 = a0 + a3, a1 + a2, a0 + a2, a1 + a3
    z5 = (z3 + z4) * FIX["1_175875602"]
    a0 = a0 * FIX["0_298631336"]
    a1 = a1 * FIX["2_053119869"]
    a2 = a2 * FIX["3_072711026"]
    a3 = a3 * FIX["1_501321110"]
    z1 = z1 * -FIX["0_899976223"]
    z2 = z2 * -FIX["2_562915447"]
    z3 = z3 * -FIX["1_961570560"] + z5
    z4 = z4 * -FIX["0_390180644"] + z5
    a0 = a0 + z1 + z3
    a1 = a1 + z2 + z4
    a2 = a2 + z2 + z3
    a3 = a3 + z1 + z4
    r = 1 << (shift - 1)
    return [(e10 + a3 + r) >> shift, (e11 + a2 + r) >> shift, (e12 + a1 + r) >> shift, (e13 + a0 + r) >> shift,
            (e13 - a0 + r) >> shift, (e12 - a1 + r) >> shift, (e11 - a2 + r) >> shift, (e10 - a3 + r) >> shift]


def range_limit(v: np.ndarray) -> np.ndarray:
    """The post-IDCT range-limit table: index v & 1023 -> sample."""
    w = v & 1023
    out = np.where(w < 128, w + 128, np.where(w < 512, 255, np.where(w < 896, 0, w - 896)))
    return out.astype(np.uint8)


def idct_plane(coef: np.ndarray, qt: np.ndarray) -> np.ndarray:
    """[bh, bw, 64] quantized coefficients -> u8 samples [bh*8, bw*8]."""
    bh, bw, _ = coef.shape
    d = (coef.astype(np.int64) * qt.astype(np.int64)).reshape(bh, bw, 8, 8)   # [.., row u, col v]
    # column pass: for each column, the 8 vertical frequencies -> 8 rows (13 - 2 bit shift)
    cols = _idct_1d(*[d[:, :, u, :] for u in range(8)], CONST_BITS - PASS1_BITS)
    ws = np.stack(cols, axis=2)                        # [bh, bw, y, v]
    rows = _idct_1d(*[ws[:, :, :, v] for v in range(8)], CONST_BITS + PASS1_BITS + 3)
    px = np.stack(rows, axis=3)                        # [bh, bw, y, x]
    return range_limit(px).transpose(0, 2, 1, 3).reshape(bh * 8, bw * 8)


# ------------------------------------------------------------------ upsampling + colour
def _h2(p: np.ndarray) -> np.ndarray:
    """h2v1 fancy: [h, w] -> [h, 2w] (first and last samples copied)."""
    h, w = p.shape
    p = p.astype(np.int32)
    out = np.empty((h, 2 * w), np.int32)
    out[:, 0] = p[:, 0]
    out[:, 1] = (3 * p[:, 0] + p[:, 1] + 2) >> 2
    out[:, 2:-2:2] = (3 * p[:, 1:-1] + p[:, :-2] + 1) >> 2
    out[:, 3:-1:2] = (3 * p[:, 1:-1] + p[:, 2:] + 2) >> 2
    out[:, -2] = (3 * p[:, -1] + p[:, -2] + 1) >> 2
    out[:, -1] = p[:, -1]
    return out


def _v2(p: np.ndarray) -> np.ndarray:
    """h1v2 fancy: [h, w] -> [2h, w]; context rows replicated at the edges."""
    p = p.astype(np.int32)
    up = np.concatenate([p[:1], p[:-1]])
    dn = np.concatenate([p[1:], p[-1:]])
    out = np.empty((2 * p.shape[0], p.shape[1]), np.int32)
    out[0::2] = (3 * p + up + 1) >> 2
    out[1::2] = (3 * p + dn + 2) >> 2
    return out


def _h2v2(p: np.ndarray) -> np.ndarray:
    """h2v2 fancy: column sums 3*this + nearer row, then the horizontal triangle with biases
    8 / 7 over 16 (edge columns: 4*sum)."""
    p = p.astype(np.int32)
    up = np.concatenate([p[:1], p[:-1]])
    dn = np.concatenate([p[1:], p[-1:]])
    out = np.empty((2 * p.shape[0], 2 * p.shape[1]), np.int32)
    for r0, nb in ((0, up), (1, dn)):
        s = 3 * p + nb
        o = out[r0::2]
        o[:, 0] = (4 * s[:, 0] + 8) >> 4
        o[:, 1] = (3 * s[:, 0] + s[:, 1] + 7) >> 4
        o[:, 2:-2:2] = (3 * s[:, 1:-1] + s[:, :-2] + 8) >> 4
        o[:, 3:-1:2] = (3 * s[:, 1:-1] + s[:, 2:] + 7) >> 4
        o[:, -2] = (3 * s[:, -1] + s[:, -2] + 8) >> 4
        o[:, -1] = (4 * s[:, -1] + 7) >> 4
    return out


def ycc_tables():
    """(Cr->R, Cb->B, Cr->G, Cb->G) fixed-point tables indexed by the sample 0..255."""
    x = np.arange(256, dtype=np.int64) - 128
    fx = lambda f: int(f * 65536 + 0.5)
    half = 1 << 15
    return ((fx(1.40200) * x + half) >> 16, (fx(1.77200) * x + half) >> 16,
            -fx(0.71414) * x, -fx(0.34414) * x + half)


def decode(data: bytes) -> np.ndarray:
    """H x W x 3 RGB u8, as PIL decodes the same bytes."""
    hdr = parse(data)
    lay = layout(hdr)
    coefs = coefficients(data, hdr, lay)
    H, W = lay["H"], lay["W"]
    planes = []
    for c, o, cf in zip(hdr["frame"]["comps"], lay["comps"], coefs):
        p = idct_plane(cf, hdr["q"][c["tq"]])[:o["ch"], :o["cw"]]
        if (o["fh"], o["fv"]) == (2, 2):
            p = _h2v2(p)
        elif o["fh"] == 2:
            p = _h2(p)
        elif o["fv"] == 2:
            p = _v2(p)
        planes.append(p[:H, :W].astype(np.int64))
    if lay["nc"] == 1:
        return np.repeat(planes[0].astype(np.uint8)[..., None], 3, axis=2)
    y, cb, cr = planes
    crr, cbb, crg, cbg = ycc_tables()
    r = np.clip(y + crr[cr], 0, 255)
    g = np.clip(y + ((cbg[cb] + crg[cr]) >> 16), 0, 255)
    b = np.clip(y + cbb[cb], 0, 255)
    return np.stack([r, g, b], axis=2).astype(np.uint8)
