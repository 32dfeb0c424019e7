"""Pins the oracle's per-op arithmetic (oracle/interp.py) against independent routines:
torch.nn.functional library ops (CPU), brute-force loops and algebraic identities.
torch is imported inside each test so a `-m gpu` run never loads it."""
import numpy as np
import pytest

import modelgen
from oracle import graphfile, interp

RNG = np.random.default_rng(1234)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a))


@pytest.mark.parametrize("B,H,W,cin,cout,k,s,g", [
    (1, 9, 11, 8, 16, 3, 1, 1), (2, 10, 10, 16, 8, 3, 2, 1), (1, 7, 5, 24, 40, 1, 1, 1),
    (2, 8, 8, 16, 16, 3, 1, 16), (1, 9, 9, 32, 32, 3, 2, 32), (1, 6, 6, 3, 16, 3, 2, 1),
    (1, 5, 5, 8, 8, 5, 1, 1)])
def test_conv_vs_torch(B, H, W, cin, cout, k, s, g):
    import torch.nn.functional as F
    p = k // 2
    x = RNG.standard_normal((B, H, W, cin), dtype=np.float32)
    w = RNG.standard_normal((cout, k, k, cin // g), dtype=np.float32)
    b = RNG.standard_normal(cout, dtype=np.float32)
    got = interp.conv2d_nhwc(x, w, b, s, p, g)
    want = F.conv2d(_t(x).permute(0, 3, 1, 2), _t(w).permute(0, 3, 1, 2), _t(b), stride=s, padding=p,
                    groups=g).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


def test_conv_bruteforce():
    """Direct sum over (ky, kx, ci) with zero padding, float64, tiny shape."""
    x = RNG.standard_normal((1, 5, 6, 8), dtype=np.float32)
    w = RNG.standard_normal((3, 3, 3, 8), dtype=np.float32)
    b = RNG.standard_normal(3, dtype=np.float32)
    got = interp.conv2d_nhwc(x, w, b, 2, 1, 1)
    Ho, Wo = 3, 3
    want = np.zeros((1, Ho, Wo, 3))
    for oy in range(Ho):
        for ox in range(Wo):
            for o in range(3):
                acc = float(b[o])
                for ky in range(3):
                    for kx in range(3):
                        iy, ix = oy * 2 - 1 + ky, ox * 2 - 1 + kx
                        if 0 <= iy < 5 and 0 <= ix < 6:
                            acc += float(np.dot(x[0, iy, ix].astype(np.float64), w[o, ky, kx].astype(np.float64)))
                want[0, oy, ox, o] = acc
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_pool_upsample_silu_vs_torch():
    import torch.nn.functional as F
    x = RNG.standard_normal((2, 7, 9, 16), dtype=np.float32)
    tx = _t(x).permute(0, 3, 1, 2)
    np.testing.assert_array_equal(interp.maxpool5(x), F.max_pool2d(tx, 5, 1, 2).permute(0, 2, 3, 1).numpy())
    np.testing.assert_array_equal(interp.upsample2(x),
                                  F.interpolate(tx, scale_factor=2, mode="nearest").permute(0, 2, 3, 1).numpy())
    np.testing.assert_allclose(interp.silu(x), F.silu(_t(x)).numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("N_hw,heads", [((20, 20), 2), ((7, 7), 3), ((4, 6), 1)])
def test_attention_vs_sdpa(N_hw, heads):
    """ultralytics Attention layout: per head [q kd | k kd | v hd] channel blocks."""
    import torch
    import torch.nn.functional as F
    H, W = N_hw
    kd, hd = 32, 64
    x = RNG.standard_normal((2, H, W, heads * (2 * kd + hd)), dtype=np.float32)
    got = interp.attention(x, heads, kd, hd)
    t = _t(x).reshape(2, H * W, heads, 2 * kd + hd).permute(0, 2, 1, 3)   # B, heads, N, per
    q, k, v = t[..., :kd], t[..., kd:2 * kd], t[..., 2 * kd:]
    o = F.scaled_dot_product_attention(q, k, v)                            # scale = kd^-1/2
    want = o.permute(0, 2, 1, 3).reshape(2, H, W, heads * hd).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    # permuting tokens permutes the outputs (no positional term)
    perm = RNG.permutation(H * W)
    xp = x.reshape(2, H * W, -1)[:, perm].reshape(x.shape)
    gp = interp.attention(xp, heads, kd, hd).reshape(2, H * W, -1)
    np.testing.assert_allclose(gp, got.reshape(2, H * W, -1)[:, perm], rtol=1e-5, atol=1e-5)
    # constant values -> output equals that value (softmax rows sum to one)
    xc = x.copy()
    xc.reshape(2, H * W, heads, -1)[..., 2 * kd:] = 0.5
    np.testing.assert_allclose(interp.attention(xc, heads, kd, hd), 0.5, atol=1e-5)


def test_convtranspose_rewrite():
    """1x1 CONV to 4C + PS2 equals ConvTranspose2d(k=2, s=2) (export/export.py:166-181)."""
    import torch.nn.functional as F
    g = modelgen.ModelGraph(5)
    x0 = g.newt(6, 5, 16)
    g.conv_transpose2(x0, 8)
    wt, bt = g.last_convt
    path = None
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        g.write(d, "detect", 80, 0)
        gf = graphfile.load(d)
        I = interp.Interp(gf, 2)
        x = RNG.standard_normal((2, 6, 5, 16), dtype=np.float32)
        I.set_input(x)
        I.run()
        got = I.view(gf.ops[-1].out)
    w16 = wt.astype(np.float16).astype(np.float32)
    want = F.conv_transpose2d(_t(x.astype(np.float16).astype(np.float32)).permute(0, 3, 1, 2), _t(w16),
                              _t(bt), stride=2).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    assert path is None


def test_fused_residual_equals_conv_then_add(tmp_path):
    """fuse_adds (engine/engine.cu:1484-1501): act(conv) + residual == CONV then ADD."""
    d = str(tmp_path / "m")
    modelgen.write_single_conv(d, 9, 9, 16, 16, 3, 1, residual=True)
    g = graphfile.load(d)
    x = RNG.standard_normal((2, 9, 9, 16), dtype=np.float32)
    a = interp.Interp(g, 2)
    a.set_input(x)
    a.run()
    fused = graphfile.fuse_adds(g.ops)
    assert len(fused) == 1 and fused[0].b == 0 and fused[0].out == g.ops[1].out
    b = interp.Interp(g, 2)
    b.set_input(x)
    b.run(fused)
    np.testing.assert_allclose(b.view(fused[0].out), a.view(g.ops[1].out), rtol=1e-6, atol=1e-6)


def test_ps2_quadrants():
    x = np.arange(2 * 3 * 4 * 8, dtype=np.float32).reshape(2, 3, 4, 8)   # 4C with C = 2
    y = interp.ps2(x)
    for di in range(2):
        for dj in range(2):
            q = 2 * di + dj
            np.testing.assert_array_equal(y[:, di::2, dj::2], x[..., 2 * q:2 * q + 2])
