"""Pins the oracle's restatement of the low-res first steps (phone/animad.cpp:392-503, moss/mossrun/mossrun.cpp:278-313)
by closed forms and invariants the reference's arithmetic fixes, not by retyping it:
- pooling constant fields gives (1 - t) d + t f n (Anima) and 2 c (MOSS); pooling is linear;
- the pooled noise of unit-variance noise keeps unit variance (why the reference multiplies the mean by f, resp. 2);
- the velocity lands sd.cpp's Euler step exactly where the reference says: x + (tn - t) v = (1 - tn) dhat + tn noise;
- bilinear upsampling with half-pixel centres reproduces constants, and linear ramps away from the clamped borders;
- animad's inline upsampling (on [C][H][W], factor 2) and mossrun's upsample2 (on token rows) are the same map;
- the scaled MOSS RoPE table equals the unscaled one at scale 1 and rotates image positions by scale x position."""
import numpy as np
import pytest

from oracle import hxo


@pytest.mark.parametrize("f", [2, 4])
def test_lowres_pool_constant_fields_and_linearity(f):
    C, H, W, t = 3, 8 * f, 4 * f, 0.75
    n = np.full((C, H, W), 0.5, np.float32)
    d = np.full((C, H, W), -1.25, np.float32)
    got = hxo.lowres_pool(n, d, f, t)
    assert got.shape == (C, H // f, W // f)
    np.testing.assert_allclose(got, (1 - t) * -1.25 + t * f * 0.5, rtol=1e-7)
    rng = np.random.default_rng(f)
    n1, n2, d1 = (rng.standard_normal((C, H, W)).astype(np.float32) for _ in range(3))
    a = hxo.lowres_pool(n1, d1, f, t) + hxo.lowres_pool(n2, np.zeros_like(d1), f, t)
    b = hxo.lowres_pool(n1 + n2, d1, f, t)
    np.testing.assert_allclose(a, b, atol=3e-6)


def test_pooled_noise_keeps_unit_variance():
    rng = np.random.default_rng(3)
    n = rng.standard_normal((16, 256, 256)).astype(np.float32)
    for f in (2, 4):
        x = hxo.lowres_pool(n, np.zeros_like(n), f, 1.0)
        assert abs(x.std() - 1.0) < 0.02 and abs(x.mean()) < 0.02
    z = rng.standard_normal((128 * 128, 64)).astype(np.float32)
    zl = hxo.moss_pool2(z, 128, 128)
    assert zl.shape == (64 * 64, 64)
    assert abs(zl.std() - 1.0) < 0.02


@pytest.mark.parametrize("f", [2, 4])
def test_lowres_velocity_lands_the_euler_step(f):
    rng = np.random.default_rng(10 + f)
    C, H, W, t, tn = 16, 8 * f, 6 * f, 0.75, 0.5
    xlow = rng.standard_normal((C, H // f, W // f)).astype(np.float32)
    vlow = rng.standard_normal((C, H // f, W // f)).astype(np.float32)
    xfull = rng.standard_normal((C, H, W)).astype(np.float32)
    nfull = rng.standard_normal((C, H, W)).astype(np.float32)
    dhat, v = hxo.lowres_velocity(xlow, vlow, xfull, nfull, f, t, tn)
    landed = xfull.astype(np.float64) + (tn - t) * v.astype(np.float64)
    target = (1 - tn) * dhat.astype(np.float64) + tn * nfull.astype(np.float64)
    np.testing.assert_allclose(landed, target, atol=2e-6)
    # the last step (dt <= 1e-6) leaves the state alone
    _, v0 = hxo.lowres_velocity(xlow, vlow, xfull, nfull, f, t, t)
    assert not v0.any()


@pytest.mark.parametrize("f", [2, 4])
def test_lowres_upsampling_constants_and_ramps(f):
    C, Hl, Wl, t = 2, 6, 5, 0.5
    H, W = Hl * f, Wl * f
    zeros = np.zeros((C, H, W), np.float32)
    # dl = xlow - t vlow: a constant clean estimate upsamples to itself
    xlow = np.full((C, Hl, Wl), 3.0, np.float32)
    vlow = np.full((C, Hl, Wl), 2.0, np.float32)  # dl = 3 - 0.5 * 2 = 2
    dhat, _ = hxo.lowres_velocity(xlow, vlow, zeros, zeros, f, t, 0.25)
    np.testing.assert_array_equal(dhat, np.full_like(dhat, 2.0))
    # a ramp along the rows: bilinear with half-pixel centres gives y_low(y) = (y + 0.5) / f - 0.5 inside the grid
    ramp = np.broadcast_to(np.arange(Hl, dtype=np.float32)[None, :, None], (C, Hl, Wl)).copy()
    dhat, _ = hxo.lowres_velocity(ramp, np.zeros_like(ramp), zeros, zeros, f, t, 0.25)
    y = np.arange(H)
    ylow = (y + 0.5) / f - 0.5
    inside = (ylow >= 0) & (ylow <= Hl - 1)
    np.testing.assert_allclose(dhat[0, inside, 0], ylow[inside], atol=1e-6)
    np.testing.assert_allclose(dhat[0, ~inside, 0], np.clip(ylow[~inside], 0, Hl - 1), atol=1e-6)


def test_anima_and_moss_upsampling_are_the_same_map():
    rng = np.random.default_rng(21)
    C4, h, w = 8, 5, 7
    rows = rng.standard_normal((h * w, C4)).astype(np.float32)
    up_rows = hxo.upsample2_rows(rows, h, w)
    chw = np.ascontiguousarray(rows.T.reshape(C4, h, w))
    zeros = np.zeros((C4, 2 * h, 2 * w), np.float32)
    dhat, _ = hxo.lowres_velocity(chw, np.zeros_like(chw), zeros, zeros, 2, 0.5, 0.25)
    np.testing.assert_array_equal(up_rows, dhat.reshape(C4, -1).T)


def test_moss_pool2_constant_and_linear():
    z = np.full((8 * 6, 4), 1.5, np.float32)
    np.testing.assert_array_equal(hxo.moss_pool2(z, 8, 6), np.full((4 * 3, 4), 3.0, np.float32))
    rng = np.random.default_rng(2)
    a, b = rng.standard_normal((2, 8 * 6, 4)).astype(np.float32)
    np.testing.assert_allclose(hxo.moss_pool2(a, 8, 6) + hxo.moss_pool2(b, 8, 6), hxo.moss_pool2(a + b, 8, 6), atol=3e-6)


def test_rope_moss_scaled():
    bands = (1.0 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
    H, W, ntxt = 4, 6, 5
    c1, s1 = hxo.rope_moss(H, W, ntxt, bands)
    c, s = hxo.rope_moss_scaled(H, W, ntxt, bands, 1.0)
    np.testing.assert_array_equal(c, c1)
    np.testing.assert_array_equal(s, s1)
    c2, s2 = hxo.rope_moss_scaled(H, W, ntxt, bands, 2.0)
    tk = 1 * W + 4  # image token (row 1, column 4)
    for d in range(32, 64):  # dims 32-47 rotate by the row position, 48-63 by the column position
        pos = ((1 - (H - 1) / 2.0) if d < 48 else (4 - (W - 1) / 2.0)) * 2.0
        assert abs(c2[tk, d] - np.cos(pos * float(bands[d % 16]))) < 1e-6
        assert abs(s2[tk, d] - np.sin(pos * float(bands[d % 16]))) < 1e-6
    np.testing.assert_array_equal(c2[H * W:], c1[H * W:])  # text rows are not scaled
