"""Pins the oracle's SPyNet pieces (CPU): each against the torch routine the reference's
kernels restate, plus closed forms.

* bicubic quarter downsample (MetalShader.swift:488-521) = torch interpolate(scale 0.25,
  bicubic, align_corners=False) within one FP16 ulp (torch sums separably); a constant
  image stays constant and a linear ramp is reproduced (the 4-tap footprint is symmetric
  about the half-pixel source position);
* pyramid (:523-570) = normalise, then repeated 2x2 avg_pool2d, within one FP16 ulp;
* border sample (:572-599) = grid_sample(border, align_corners=True); prepare (:601-639):
  upsample = interpolate(x2, bilinear, align_corners=True) * 2, warp = grid_sample of the
  support by the FP32 base flow, within one FP16 ulp;
* 7x7 conv = conv2d in float64 within one FP16 ulp; flow add = numpy FP16 add, exactly;
* the whole chain against a float32 torch SPyNet on the same weights.
"""
from __future__ import annotations

import numpy as np
import pytest

import spynet_reference as sr

torch = pytest.importorskip("torch")
F = torch.nn.functional


def ulps(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    ulp = np.maximum(np.abs(ref), 2.0 ** -14) * 2.0 ** -10
    return np.abs(got - ref) / ulp


def test_bicubic_matches_torch(oracle):
    rng = np.random.default_rng(1)
    x = sr.f16(rng.random(3 * 64 * 96))
    got = oracle.bicubic_quarter_f16(3, 64, 96, x).astype(np.float64)
    ref = F.interpolate(torch.from_numpy(x.astype(np.float32).reshape(1, 3, 64, 96)), scale_factor=0.25,
                        mode="bicubic", align_corners=False).numpy().ravel()
    assert ulps(got, sr.f16(ref)).max() <= 1.0


def test_bicubic_closed_forms(oracle):
    const = np.full(3 * 32 * 32, 0.375, np.float16)
    assert np.all(oracle.bicubic_quarter_f16(3, 32, 32, const) == np.float16(0.375))
    # ramp f(y, x) = x / 64: the output at source x = 4 ox + 1.5 is (4 ox + 1.5) / 64
    ramp = np.tile(np.arange(32, dtype=np.float32) / 64, 3 * 32).astype(np.float16)
    got = oracle.bicubic_quarter_f16(3, 32, 32, ramp).reshape(3, 8, 8).astype(np.float64)
    want = (4 * np.arange(8) + 1.5) / 64
    assert np.abs(got - want[None, None, :]).max() <= 2.0 ** -11


def test_pyramid_matches_avg_pool(oracle):
    rng = np.random.default_rng(2)
    frame = sr.smooth_frame(rng, 64, 64)
    levels = oracle.spynet_pyramid_f16(64, 64, 6, frame)
    t = torch.from_numpy(frame.astype(np.float32).reshape(1, 3, 64, 64))
    t = (t - torch.tensor(sr.MEAN).view(1, 3, 1, 1)) / torch.tensor(sr.STD).view(1, 3, 1, 1)
    for l in range(5, -1, -1):
        assert levels[l].size == 3 * (64 >> (5 - l)) ** 2
        assert ulps(levels[l], sr.f16(t.numpy().ravel())).max() <= 1.0, l
        t = F.avg_pool2d(t, 2, 2)


def test_sample_border_matches_grid_sample(oracle):
    rng = np.random.default_rng(3)
    h, w = 9, 13
    img = sr.f16(rng.standard_normal(h * w))
    ys = rng.uniform(-3, h + 2, 200).astype(np.float32)
    xs = rng.uniform(-3, w + 2, 200).astype(np.float32)
    got = np.array([oracle.load().oracle_sample_border_f16(oracle._u16(img)[1], 0, h, w, float(y), float(x))
                    for y, x in zip(ys, xs)])
    grid = torch.from_numpy(np.stack((2 * xs / (w - 1) - 1, 2 * ys / (h - 1) - 1), -1).reshape(1, 1, -1, 2))
    ref = F.grid_sample(torch.from_numpy(img.astype(np.float32).reshape(1, 1, h, w)), grid, mode="bilinear",
                        padding_mode="border", align_corners=True).numpy().ravel()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(img.astype(np.float32)).max() * 4


@pytest.mark.parametrize("first", [True, False])
def test_prepare_matches_torch(oracle, first):
    rng = np.random.default_rng(4 + first)
    h, w, sh, sw = 16, 16, 8, 8
    ref = sr.f16(rng.standard_normal(3 * h * w))
    sup = sr.f16(rng.standard_normal(3 * h * w))
    src = None if first else sr.f16(rng.uniform(-3, 3, 2 * sh * sw))
    feat, base = oracle.spynet_prepare_f16(w, h, first, ref, sup, src, sw, sh)
    if first:
        up = torch.zeros(1, 2, h, w)
    else:
        up = F.interpolate(torch.from_numpy(src.astype(np.float32).reshape(1, 2, sh, sw)), scale_factor=2,
                           mode="bilinear", align_corners=True) * 2.0
    assert ulps(base, sr.f16(up.numpy().ravel())).max() <= 1.0
    gy, gx = torch.meshgrid(torch.arange(h, dtype=torch.float32), torch.arange(w, dtype=torch.float32),
                            indexing="ij")
    grid = torch.stack((2 * (gx + up[0, 0]) / (w - 1) - 1, 2 * (gy + up[0, 1]) / (h - 1) - 1), -1)[None]
    warped = F.grid_sample(torch.from_numpy(sup.astype(np.float32).reshape(1, 3, h, w)), grid,
                           padding_mode="border", align_corners=True).numpy().ravel()
    feat = feat.reshape(8, h * w)
    assert np.array_equal(feat[:3].ravel().view(np.uint16), ref.view(np.uint16))
    assert ulps(feat[3:6].ravel(), sr.f16(warped)).max() <= 1.0
    assert np.array_equal(feat[6:].ravel().view(np.uint16), base.view(np.uint16))


def test_convk_matches_conv2d(oracle):
    rng = np.random.default_rng(6)
    ci, co, h, w = 16, 8, 11, 9
    x = sr.f16(rng.standard_normal(ci * h * w))
    wt = sr.f16(rng.normal(0, 0.05, (co, ci, 7, 7)))
    b = sr.f16(rng.normal(0, 0.1, co))
    for act in (0, 2):
        got = oracle.convk_f16(7, ci, co, h, w, x, wt, b, act)
        ref = F.conv2d(torch.from_numpy(x.astype(np.float64).reshape(1, ci, h, w)),
                       torch.from_numpy(wt.astype(np.float64)), torch.from_numpy(b.astype(np.float64)), padding=3)
        if act == 2:
            ref = F.relu(ref)
        assert ulps(got, sr.f16(ref.numpy().ravel())).max() <= 1.0
    # k = 3 is the body's conv3x3
    w3 = sr.f16(rng.normal(0, 0.05, (co, ci, 3, 3)))
    assert np.array_equal(oracle.convk_f16(3, ci, co, h, w, x, w3, b, 2).view(np.uint16),
                          oracle.conv3x3_f16(ci, co, h, w, x, w3, b, 2).view(np.uint16))


def test_add_is_fp16_add(oracle):
    rng = np.random.default_rng(7)
    a = sr.f16(rng.uniform(-40, 40, 1000))
    b = sr.f16(rng.uniform(-3, 3, 1000))
    assert np.array_equal(oracle.add_f16(a, b).view(np.uint16), (a + b).view(np.uint16))


def test_chain_matches_torch_spynet(oracle):
    rng = np.random.default_rng(8)
    weights = sr.spynet_weights(rng)
    ref = sr.smooth_frame(rng, 64, 64)
    sup = sr.smooth_frame(np.random.default_rng(9), 64, 64)
    got = sr.spynet_flow(weights, ref, sup, 64, 64).astype(np.float64)
    want = sr.torch_spynet(weights, ref, sup, 64, 64)
    scale = np.abs(want).max()
    assert 0.5 < scale < 100, scale  # a non-trivial flow field
    # FP16 rounding between 30 layers against float32 throughout.
    assert np.abs(got - want).max() <= 2e-2 * max(1.0, scale)
    assert np.abs(got - want).mean() <= 2e-3 * max(1.0, scale)
