"""Pins the CPU oracle (oracle/dcn_oracle.c) before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle (a dropped bilinear term,
a swapped dy/dx channel, a wrong offset-group index, a transposed weight, a missed
padding case) fails at least one of them:
  * the reference's own known-answer test (DeformConvCPUTests.swift:4-33);
  * closed forms: zero offsets + mask 1 == torch conv2d; integer offsets == shifted
    conv2d; mask 0 or far-away samples == bias; half-pixel offsets == 4-point means;
  * an independent DCN built from torch.nn.functional.grid_sample (align_corners=True,
    zero padding) in float64, over groups / offset groups / stride / dilation / padding;
  * brute-force float64 Python loops on tiny shapes;
  * IEEE binary16 conversion against numpy, exhaustively for binary16 -> binary32.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from jasnamacos_amd.deform_conv import DeformConvShape

RNG = np.random.default_rng(20261201)


def rand_inputs(shape: DeformConvShape, rng, offset_scale=2.5, mask_range=(0.0, 1.0)):
    c = {
        "input": rng.standard_normal(shape.batch * shape.input_channels * shape.input_height * shape.input_width),
        "offset": rng.uniform(-offset_scale, offset_scale,
                              shape.batch * 2 * shape.offset_groups * shape.kernel_area
                              * shape.output_height * shape.output_width),
        "mask": rng.uniform(*mask_range, shape.batch * shape.offset_groups * shape.kernel_area
                            * shape.output_height * shape.output_width),
        "weight": rng.uniform(-0.3, 0.3, shape.output_channels * (shape.input_channels // shape.groups)
                              * shape.kernel_area),
        "bias": rng.uniform(-0.1, 0.1, shape.output_channels),
    }
    return {k: v.astype(np.float32) for k, v in c.items()}


def grid_sample_dcn(shape: DeformConvShape, inp, off, msk, w, b) -> np.ndarray:
    """Independent float64 DCNv2 via grid_sample (bilinear, zeros, align_corners=True)."""
    s = shape
    x = torch.tensor(inp, dtype=torch.float64).reshape(s.batch, s.input_channels, s.input_height, s.input_width)
    o = torch.tensor(off, dtype=torch.float64).reshape(s.batch, s.offset_groups, s.kernel_area, 2,
                                                       s.output_height, s.output_width)
    m = torch.tensor(msk, dtype=torch.float64).reshape(s.batch, s.offset_groups, s.kernel_area,
                                                       s.output_height, s.output_width)
    wt = torch.tensor(w, dtype=torch.float64).reshape(s.output_channels, s.input_channels // s.groups, s.kernel_area)
    cg = s.input_channels // s.offset_groups
    oy = torch.arange(s.output_height, dtype=torch.float64).view(-1, 1)
    ox = torch.arange(s.output_width, dtype=torch.float64).view(1, -1)
    cols = torch.zeros(s.batch, s.input_channels, s.kernel_area, s.output_height, s.output_width, dtype=torch.float64)
    for g in range(s.offset_groups):
        xg = x[:, g * cg:(g + 1) * cg]
        for k in range(s.kernel_area):
            ky, kx = divmod(k, s.kernel_width)
            py = oy * s.stride_height - s.pad_height + ky * s.dilation_height + o[:, g, k, 0]
            px = ox * s.stride_width - s.pad_width + kx * s.dilation_width + o[:, g, k, 1]
            gx = 2.0 * px / (s.input_width - 1) - 1.0 if s.input_width > 1 else px * 0.0
            gy = 2.0 * py / (s.input_height - 1) - 1.0 if s.input_height > 1 else py * 0.0
            grid = torch.stack([gx, gy], dim=-1)
            sampled = F.grid_sample(xg, grid, mode="bilinear", padding_mode="zeros", align_corners=True)
            cols[:, g * cg:(g + 1) * cg, k] = sampled * m[:, g, k].unsqueeze(1)
    out = torch.zeros(s.batch, s.output_channels, s.output_height, s.output_width, dtype=torch.float64)
    cpg, opg = s.input_channels // s.groups, s.output_channels // s.groups
    for grp in range(s.groups):
        c = cols[:, grp * cpg:(grp + 1) * cpg]
        out[:, grp * opg:(grp + 1) * opg] = torch.einsum("bckhw,ock->bohw", c, wt[grp * opg:(grp + 1) * opg])
    out += torch.tensor(b, dtype=torch.float64).view(1, -1, 1, 1)
    return out.numpy().ravel()


def brute_force_dcn(shape: DeformConvShape, inp, off, msk, w, b) -> np.ndarray:
    """Plain float64 loops; corners outside the input contribute zero."""
    s = shape
    X = np.asarray(inp, np.float64).reshape(s.batch, s.input_channels, s.input_height, s.input_width)
    O = np.asarray(off, np.float64).reshape(s.batch, -1, s.output_height, s.output_width)
    M = np.asarray(msk, np.float64).reshape(s.batch, -1, s.output_height, s.output_width)
    W = np.asarray(w, np.float64).reshape(s.output_channels, s.input_channels // s.groups, s.kernel_height, s.kernel_width)
    out = np.zeros((s.batch, s.output_channels, s.output_height, s.output_width))
    cpg, opg = s.input_channels // s.groups, s.output_channels // s.groups
    cpog = s.input_channels // s.offset_groups

    def pix(n, c, yy, xx):
        if 0 <= yy < s.input_height and 0 <= xx < s.input_width:
            return X[n, c, yy, xx]
        return 0.0

    for n in range(s.batch):
        for oc in range(s.output_channels):
            grp = oc // opg
            for oy in range(s.output_height):
                for ox in range(s.output_width):
                    acc = float(b[oc])
                    for li in range(cpg):
                        ic = grp * cpg + li
                        og = ic // cpog
                        for ky in range(s.kernel_height):
                            for kx in range(s.kernel_width):
                                k = ky * s.kernel_width + kx
                                y = oy * s.stride_height - s.pad_height + ky * s.dilation_height + O[n, 2 * (og * s.kernel_area + k), oy, ox]
                                x = ox * s.stride_width - s.pad_width + kx * s.dilation_width + O[n, 2 * (og * s.kernel_area + k) + 1, oy, ox]
                                y0, x0 = math.floor(y), math.floor(x)
                                ly, lx = y - y0, x - x0
                                v = (pix(n, ic, y0, x0) * (1 - ly) * (1 - lx) + pix(n, ic, y0, x0 + 1) * (1 - ly) * lx
                                     + pix(n, ic, y0 + 1, x0) * ly * (1 - lx) + pix(n, ic, y0 + 1, x0 + 1) * ly * lx)
                                acc += v * M[n, og * s.kernel_area + k, oy, ox] * W[oc, li, ky, kx]
                    out[n, oc, oy, ox] = acc
    return out.ravel()


def test_reference_known_answer(oracle):
    # DeformConvCPUTests.swift:4-33: 1x1 kernel, zero offsets, mask 0.5, weight 2, bias 1.
    s = DeformConvShape(1, 1, 2, 2, 1, 2, 2, 1, 1, 0, 0, 1, 1, 1, 1, 1, 1)
    out = oracle.forward_f32(s, [1, 2, 3, 4], np.zeros(8), np.full(4, 0.5), [2], [1])
    assert out.tolist() == [2.0, 3.0, 4.0, 5.0]


def test_invalid_shape_rejected(oracle):
    s = DeformConvShape(1, 3, 4, 4, 2, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)  # 3 % 2 != 0
    with pytest.raises(ValueError):
        oracle.forward_f32(s, np.zeros(48), np.zeros(2 * 2 * 9 * 16), np.zeros(2 * 9 * 16), np.zeros(54), np.zeros(2))


@pytest.mark.parametrize("seed", [0, 1])
def test_zero_offsets_unit_mask_is_conv2d(oracle, seed):
    rng = np.random.default_rng(seed)
    s = DeformConvShape(2, 8, 9, 7, 6, 9, 7, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    d = rand_inputs(s, rng)
    d["offset"][:] = 0
    d["mask"][:] = 1
    out = oracle.forward_f32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    x = torch.tensor(d["input"], dtype=torch.float64).reshape(2, 8, 9, 7)
    w = torch.tensor(d["weight"], dtype=torch.float64).reshape(6, 8, 3, 3)
    ref = F.conv2d(x, w, torch.tensor(d["bias"], dtype=torch.float64), padding=1).numpy().ravel()
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)


def test_integer_offsets_shift_the_input(oracle):
    rng = np.random.default_rng(3)
    s = DeformConvShape(1, 4, 10, 11, 5, 10, 11, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1)
    d = rand_inputs(s, rng)
    off = d["offset"].reshape(2 * 9, 10, 11)
    off[0::2] = 2.0   # dy
    off[1::2] = -3.0  # dx
    d["mask"][:] = 1
    out = oracle.forward_f32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    x = torch.tensor(d["input"], dtype=torch.float64).reshape(1, 4, 10, 11)
    # Tap (ky, kx) of pixel (oy, ox) reads x[oy - 1 + ky + 2, ox - 1 + kx - 3] (zero outside x):
    # a valid conv over the zero-padded input cropped at (2 - 1, -3 - 1).
    P = 5
    xp = F.pad(x, (P, P, P, P))
    crop = xp[:, :, P + 2 - 1:P + 2 - 1 + 12, P - 3 - 1:P - 3 - 1 + 13]
    w = torch.tensor(d["weight"], dtype=torch.float64).reshape(5, 4, 3, 3)
    ref = F.conv2d(crop, w, torch.tensor(d["bias"], dtype=torch.float64)).numpy().ravel()
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-5)


def test_zero_mask_and_far_samples_give_bias(oracle):
    rng = np.random.default_rng(4)
    s = DeformConvShape(1, 8, 6, 6, 4, 6, 6, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    d = rand_inputs(s, rng)
    bias_plane = np.repeat(d["bias"], 36)
    m0 = d["mask"].copy()
    m0[:] = 0
    out = oracle.forward_f32(s, d["input"], d["offset"], m0, d["weight"], d["bias"])
    assert np.array_equal(out, bias_plane)
    for far in (1000.0, -1000.0, 7.0, -8.5):
        off = np.full_like(d["offset"], far)
        out = oracle.forward_f32(s, d["input"], off, d["mask"], d["weight"], d["bias"])
        assert np.array_equal(out, bias_plane), far


def test_half_pixel_offsets_average_four_neighbours(oracle):
    # 1x1 kernel, weight 1, bias 0, mask 1, offset (+0.5, +0.5): mean of the 2x2 block.
    s = DeformConvShape(1, 1, 4, 5, 1, 4, 5, 1, 1, 0, 0, 1, 1, 1, 1, 1, 1)
    x = np.arange(20, dtype=np.float32) * 0.25 - 1.0
    out = oracle.forward_f32(s, x, np.full(40, 0.5, np.float32), np.ones(20), [1.0], [0.0])
    X = np.pad(x.reshape(4, 5).astype(np.float64), ((0, 1), (0, 1)))
    ref = (X[:-1, :-1] + X[:-1, 1:] + X[1:, :-1] + X[1:, 1:]) / 4
    np.testing.assert_allclose(out, ref.ravel(), rtol=0, atol=1e-6)


SHAPES = [
    DeformConvShape(1, 8, 7, 9, 4, 7, 9, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1),
    DeformConvShape(2, 8, 6, 6, 6, 6, 6, 3, 3, 1, 1, 1, 1, 1, 1, 2, 4),   # groups 2, 4 offset groups
    DeformConvShape(1, 6, 9, 8, 3, 4, 4, 3, 3, 1, 0, 2, 2, 1, 1, 1, 3),   # stride 2, asym pad
    DeformConvShape(1, 4, 8, 8, 4, 6, 6, 3, 3, 1, 1, 1, 1, 2, 2, 2, 2),   # dilation 2
    DeformConvShape(1, 16, 5, 5, 8, 5, 5, 1, 3, 0, 1, 1, 1, 1, 1, 1, 16),  # 1x3 kernel, Cg = 1
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"b{s.batch}c{s.input_channels}g{s.groups}og{s.offset_groups}s{s.stride_height}d{s.dilation_height}k{s.kernel_height}x{s.kernel_width}")
def test_matches_grid_sample_dcn(oracle, shape):
    d = rand_inputs(shape, np.random.default_rng(shape.input_channels * 7 + shape.groups))
    out = oracle.forward_f32(shape, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    ref = grid_sample_dcn(shape, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    np.testing.assert_allclose(out, ref, rtol=0, atol=5e-5)


@pytest.mark.parametrize("shape", SHAPES[:3], ids=["plain", "groups", "stride"])
def test_matches_brute_force(oracle, shape):
    d = rand_inputs(shape, np.random.default_rng(11))
    out = oracle.forward_f32(shape, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    ref = brute_force_dcn(shape, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    np.testing.assert_allclose(out, ref, rtol=0, atol=5e-5)


def test_swapping_dy_dx_changes_result(oracle):
    # Guards the channel convention itself: channel 2k is dy, 2k+1 is dx.
    s = DeformConvShape(1, 1, 5, 5, 1, 5, 5, 1, 1, 0, 0, 1, 1, 1, 1, 1, 1)
    x = np.arange(25, dtype=np.float32)
    off = np.zeros(50, np.float32)
    off[:25] = 1.0  # dy = +1 -> value of the row below = x + 5
    out = oracle.forward_f32(s, x, off, np.ones(25), [1.0], [0.0])
    ref = np.where(np.arange(25) < 20, x + 5, 0)
    assert np.array_equal(out, ref)


@pytest.mark.parametrize("shape", [
    DeformConvShape(2, 16, 9, 11, 8, 9, 11, 3, 3, 1, 1, 1, 1, 1, 1, 1, 4),
    DeformConvShape(1, 12, 7, 8, 6, 4, 4, 3, 2, 1, 0, 2, 2, 1, 2, 3, 2),  # groups 3, stride 2, dilation
])
def test_threaded_and_oc_range_forms_equal_forward_bitwise(oracle, shape):
    """The GPU tests' checkers at the config sizes are forward_f32_threads (output channels
    spread over threads), forward_f32_oc_range (a slice of output channels) and
    forward_f32_ocs (listed channels over a thread pool): each must be forward_f32 bit for
    bit, whatever the thread count or the slicing."""
    d = rand_inputs(shape, np.random.default_rng(17))
    args = [d[k] for k in ("input", "offset", "mask", "weight", "bias")]
    want = oracle.forward_f32(shape, *args).view(np.uint32)
    for threads in (1, 3, 8):
        assert np.array_equal(oracle.forward_f32_threads(shape, *args, threads=threads).view(np.uint32), want)
    plane = shape.output_height * shape.output_width
    got = np.zeros(shape.batch * shape.output_channels * plane, np.float32)
    cuts = [0, 1, shape.output_channels // 2, shape.output_channels]
    for lo, hi in zip(cuts, cuts[1:]):
        part = oracle.forward_f32_oc_range(shape, *args, lo, hi).reshape(shape.batch, shape.output_channels, plane)
        outside = np.ones(shape.output_channels, bool)
        outside[lo:hi] = False
        assert not part[:, outside].any()  # nothing written outside the slice
        got.reshape(shape.batch, shape.output_channels, plane)[:, lo:hi] = part[:, lo:hi]
    assert np.array_equal(got.view(np.uint32), want)
    picked = [0, shape.output_channels - 1, 2]
    some = oracle.forward_f32_ocs(shape, *args, picked, threads=3).reshape(shape.batch, shape.output_channels, plane)
    full = want.view(np.float32).reshape(shape.batch, shape.output_channels, plane)
    assert np.array_equal(some[:, picked].view(np.uint32), full[:, picked].view(np.uint32))
    assert not np.delete(some, picked, axis=1).any()


def test_f16_direct_is_rounded_f32_oracle(oracle):
    s = SHAPES[1]
    d = rand_inputs(s, np.random.default_rng(5))
    h = {k: v.astype(np.float16) for k, v in d.items()}
    out16 = oracle.forward_f16_direct(s, h["input"], h["offset"], h["mask"], h["weight"], h["bias"])
    out32 = oracle.forward_f32(s, *[h[k].astype(np.float32) for k in ("input", "offset", "mask", "weight", "bias")])
    assert np.array_equal(out16.view(np.uint16), out32.astype(np.float16).view(np.uint16))


def test_im2col_times_weights_is_forward(oracle):
    s = DeformConvShape(2, 16, 7, 6, 8, 7, 6, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    d = rand_inputs(s, np.random.default_rng(6))
    h = {k: v.astype(np.float16) for k, v in d.items()}
    cols = oracle.im2col_f16(s, h["input"], h["offset"], h["mask"]).astype(np.float64)
    cols = cols.reshape(2, 42, 16 * 9)
    W = h["weight"].astype(np.float64).reshape(8, 144)
    ref = np.einsum("bpk,ok->bop", cols, W) + h["bias"].astype(np.float64)[None, :, None]
    exact = oracle.forward_f32(s, *[h[k].astype(np.float32) for k in ("input", "offset", "mask", "weight", "bias")])
    # im2col rounds each modulated sample to FP16: agreement to FP16 resolution only.
    np.testing.assert_allclose(ref.ravel(), exact, rtol=0, atol=3e-3)
    gem = oracle.gemm_f16(s, cols.astype(np.float16).ravel(), h["weight"], h["bias"]).astype(np.float64)
    np.testing.assert_allclose(gem, ref.ravel(), rtol=0, atol=2e-3)


def test_im2col_integer_offsets_copy_input(oracle):
    s = DeformConvShape(1, 8, 5, 5, 8, 5, 5, 1, 1, 0, 0, 1, 1, 1, 1, 1, 1)
    x = (np.arange(200) % 17 - 8).astype(np.float16)
    off = np.zeros(50, np.float16)
    off[:25] = -1  # dy = -1: row above
    cols = oracle.im2col_f16(s, x, off, np.ones(25, np.float16)).reshape(25, 8)
    X = x.reshape(8, 5, 5)
    for p in range(25):
        y, xx = divmod(p, 5)
        ref = X[:, y - 1, xx] if y >= 1 else np.zeros(8, np.float16)
        assert np.array_equal(cols[p], ref)


def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = oracle.f16_bits_to_f32(bits)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f32_to_f16_matches_numpy(oracle):
    rng = np.random.default_rng(8)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 4000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25,
                  2.0 ** -14, 2.0 ** -14 - 2.0 ** -30, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
        # ties: exactly halfway between two binary16 values
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -11) + np.float32(1.0)),
    ])
    got = oracle.f32_to_f16_bits(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_matches_torch(oracle):
    """The oracle's BF16 rounding (nearest, ties to even) against torch's conversion,
    over random magnitudes, ties, subnormals, overflow and infinities; the widening is
    exact (bits in the high half)."""
    rng = np.random.default_rng(18)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 4000).astype(np.float32),
        np.array([0.0, -0.0, 1e-40, -1e-40, 3.3895e38, 3.4e38, np.inf, -np.inf], np.float32),
        # ties: exactly halfway between two BF16 values (both parities)
        (np.arange(1, 600, dtype=np.float32) * np.float32(2.0 ** -8) + np.float32(1.0)),
    ])
    lib = oracle.load()
    got = np.array([lib.oracle_f32_to_bf16(float(v)) for v in vals], np.uint16)
    ref = torch.tensor(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = np.array([lib.oracle_bf16_to_f32(int(b)) for b in got[:4000]], np.float32)
    assert np.array_equal(back, torch.tensor(ref[:4000].view(np.int16)).view(torch.bfloat16).float().numpy())
    nan = lib.oracle_f32_to_bf16(float("nan"))
    assert (nan & 0x7f80) == 0x7f80 and (nan & 0x7f) != 0


def _bf16(x):
    return torch.tensor(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_im2col_bf16_integer_offsets_copy_input(oracle):
    """Integer offsets and a unit mask gather the input itself: a shifted copy, bit for bit."""
    s = DeformConvShape(1, 8, 5, 5, 8, 5, 5, 1, 1, 0, 0, 1, 1, 1, 1, 1, 1)
    x = _bf16(np.random.default_rng(19).standard_normal(200))
    off = np.zeros(50, np.float32)
    off[25:] = 1  # dx = +1: the column to the right
    cols = oracle.im2col_bf16(s, x, _bf16(off), _bf16(np.ones(25))).reshape(25, 8)
    X = x.reshape(8, 5, 5)
    for p in range(25):
        y, xx = divmod(p, 5)
        ref = X[:, y, xx + 1] if xx + 1 < 5 else np.zeros(8, np.uint16)
        assert np.array_equal(cols[p], ref)


def test_im2col_bf16_equals_f16_where_both_are_exact(oracle):
    """Inputs that are integers in [-4, 4], offsets on a quarter-pixel grid and masks that
    are multiples of 1/4: every modulated sample is a multiple of 1/64 below 4 in magnitude,
    which BF16 (8 significant bits) and FP16 hold exactly, so the BF16 gather must equal the
    (separately pinned) FP16 gather value for value, padding, coordinates and association
    included."""
    s = DeformConvShape(2, 16, 7, 6, 8, 7, 6, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    rng = np.random.default_rng(20)
    c = s.counts()
    x = rng.integers(-4, 5, c["input"]).astype(np.float32)
    off = rng.integers(-12, 13, c["offset"]).astype(np.float32) / 4
    m = rng.integers(0, 5, c["mask"]).astype(np.float32) / 4
    cb = oracle.im2col_bf16(s, _bf16(x), _bf16(off), _bf16(m))
    ch = oracle.im2col_f16(s, x.astype(np.float16), off.astype(np.float16), m.astype(np.float16))
    widened = torch.tensor(cb.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(widened, ch.astype(np.float32))
    assert np.count_nonzero(widened) > widened.size // 4


def test_nonfinite_flag(oracle):
    # MetalNonFiniteFlagTests.swift:50-52
    assert oracle.flag_nonfinite_f16(np.array([0, 1, -2, 0.5], np.float16)) == 0
    assert oracle.flag_nonfinite_f16(np.array([0, np.inf, 1], np.float16)) == 1
    assert oracle.flag_nonfinite_f16(np.array([0, np.nan, 1], np.float16)) == 1
    assert oracle.flag_nonfinite_f16(np.array([65504, -65504], np.float16)) == 0


def test_offset_transform_closed_form(oracle):
    # JasnaCLI.swift:177-211: 10*tanh(raw) + flow[y for even / x for odd], sigmoid mask, tol 5e-3.
    plane = 7
    raw = np.array([((i * 13) % 101) / 50 - 1 for i in range(432 * plane)], np.float32).astype(np.float16)
    flow1 = (np.arange(2 * plane) / 20 - 0.25).astype(np.float16)
    flow2 = (0.3 - np.arange(2 * plane) / 30).astype(np.float16)
    off, msk = oracle.offset_transform_f16(plane, raw, flow1, flow2)
    r = raw.astype(np.float64).reshape(432, plane)
    f1, f2 = flow1.astype(np.float64).reshape(2, plane), flow2.astype(np.float64).reshape(2, plane)
    exp_off = np.empty((288, plane))
    for c in range(288):
        flow = f1 if c < 144 else f2
        exp_off[c] = 10 * np.tanh(r[c]) + flow[1 if (c % 144) % 2 == 0 else 0]
    exp_msk = 1 / (1 + np.exp(-r[288:]))
    assert np.abs(off.astype(np.float64).reshape(288, plane) - exp_off).max() < 5e-3
    assert np.abs(msk.astype(np.float64).reshape(144, plane) - exp_msk).max() < 5e-3


def _warp_zero(values, y, x):
    H, W = values.shape
    y0, x0 = math.floor(y), math.floor(x)
    ly, lx = y - y0, x - x0

    def v(yy, xx):
        return values[yy, xx] if 0 <= yy < H and 0 <= xx < W else 0.0

    return (v(y0, x0) * (1 - ly) * (1 - lx) + v(y0, x0 + 1) * (1 - ly) * lx
            + v(y0 + 1, x0) * ly * (1 - lx) + v(y0 + 1, x0 + 1) * ly * lx)


def test_temporal_prepare_closed_form(oracle):
    # JasnaCLI.swift:213-311 (tolerance 4e-3), first-order flow2 exactly 0 (:300-310).
    w = h = 3
    plane = 9
    fp = np.array([((i * 11) % 71) / 50 - 0.7 for i in range(64 * plane)]).astype(np.float16)
    fc = np.array([((i * 17) % 83) / 60 - 0.6 for i in range(64 * plane)]).astype(np.float16)
    fn2 = np.array([((i * 23) % 97) / 70 - 0.65 for i in range(64 * plane)]).astype(np.float16)
    f1 = np.array([((i * 7) % 19) / 20 - 0.4 for i in range(2 * plane)]).astype(np.float16)
    pf = np.array([((i * 5) % 17) / 25 - 0.3 for i in range(2 * plane)]).astype(np.float16)
    flow2, cond, dinp = oracle.temporal_prepare_f16(w, h, True, fp, fc, fn2, f1, pf)
    F1 = f1.astype(np.float64).reshape(2, plane)
    PF = pf.astype(np.float64).reshape(2, h, w)
    exp_f2 = np.empty((2, plane))
    for c in range(2):
        for sp in range(plane):
            y, x = divmod(sp, w)
            exp_f2[c, sp] = F1[c, sp] + _warp_zero(PF[c], y + F1[1, sp], x + F1[0, sp])
    exp_f2h = exp_f2.astype(np.float16).astype(np.float64)
    FP = fp.astype(np.float64).reshape(64, h, w)
    FN = fn2.astype(np.float64).reshape(64, h, w)
    exp_cond = np.empty((196, plane))
    for c in range(196):
        for sp in range(plane):
            y, x = divmod(sp, w)
            if c < 64:
                exp_cond[c, sp] = _warp_zero(FP[c], y + F1[1, sp], x + F1[0, sp])
            elif c < 128:
                exp_cond[c, sp] = fc.astype(np.float64)[(c - 64) * plane + sp]
            elif c < 192:
                exp_cond[c, sp] = _warp_zero(FN[c - 128], y + exp_f2h[1, sp], x + exp_f2h[0, sp])
            elif c < 194:
                exp_cond[c, sp] = F1[c - 192, sp]
            else:
                exp_cond[c, sp] = exp_f2h[c - 194, sp]
    err = max(np.abs(flow2.astype(np.float64) - exp_f2.ravel()).max(),
              np.abs(cond.astype(np.float64) - exp_cond.ravel()).max())
    assert err < 4e-3
    assert np.array_equal(dinp.view(np.uint16), np.concatenate([fp, fn2]).view(np.uint16))
    flow2_first, _, _ = oracle.temporal_prepare_f16(w, h, False, fp, fc, np.zeros_like(fn2), f1, pf)
    assert np.all(flow2_first.astype(np.float32) == 0)


def test_conv3x3_matches_torch(oracle):
    rng = np.random.default_rng(9)
    cin, cout, hh, ww = 5, 4, 6, 7
    x = rng.standard_normal(cin * hh * ww).astype(np.float16)
    w = (rng.standard_normal(cout * cin * 9) * 0.2).astype(np.float16)
    b = (rng.standard_normal(cout) * 0.1).astype(np.float16)
    res = rng.standard_normal(cout * hh * ww).astype(np.float16)
    ref = F.conv2d(torch.tensor(x.astype(np.float64)).reshape(1, cin, hh, ww),
                   torch.tensor(w.astype(np.float64)).reshape(cout, cin, 3, 3),
                   torch.tensor(b.astype(np.float64)), padding=1)
    for act, fn in ((0, lambda t: t), (1, lambda t: F.leaky_relu(t, 0.1)), (2, F.relu)):
        out = oracle.conv3x3_f16(cin, cout, hh, ww, x, w, b, act, 0.1)
        np.testing.assert_allclose(out.astype(np.float64), fn(ref).numpy().ravel(), rtol=0, atol=4e-3)
    out = oracle.conv3x3_f16(cin, cout, hh, ww, x, w, b, 2, 0.1, res)
    np.testing.assert_allclose(out.astype(np.float64), F.relu(ref).numpy().ravel() + res.astype(np.float64),
                               rtol=0, atol=8e-3)


def test_conv3x3_residual_is_added_before_the_one_rounding(oracle):
    """acc = 1 + 2^-11 (bias 1, one input 1 times weight 2^-11, every other weight 0) lies
    halfway between two FP16 values; the residual 2^-11 then makes 1 + 2^-10 exactly.
    One rounding after the add gives 1 + 2^-10; rounding acc first (ties to even: 1.0) and
    then adding would give half(1 + 2^-11) = 1.0. A second residual is a separate FP16 add."""
    cin, cout, hh, ww = 2, 1, 3, 3
    x = np.zeros(cin * hh * ww, np.float16)
    x[4] = 1.0  # channel 0, centre pixel
    w = np.zeros(cout * cin * 9, np.float16)
    w[4] = np.float16(2.0 ** -11)  # ic 0, centre tap: only the centre output sees it
    b = np.ones(cout, np.float16)
    res = np.full(cout * hh * ww, np.float16(2.0 ** -11))
    out = oracle.conv3x3_f16(cin, cout, hh, ww, x, w, b, 0, 0.1, res)
    assert out[4] == np.float16(1 + 2.0 ** -10)
    assert np.float16(np.float16(1 + 2.0 ** -11) + res[4]) == np.float16(1.0)  # the other order
    # Elsewhere acc = 1 exactly: 1 + 2^-11 ties to even, 1.0.
    assert np.all(np.delete(out, 4) == np.float16(1.0))
    two = oracle.add_f16(out, res)
    assert two[4] == np.float16(np.float32(out[4]) + np.float32(res[4]))


# ---- property test over random shapes (Hypothesis) ------------------------------------

from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402


@st.composite
def dcn_cases(draw):
    groups = draw(st.sampled_from([1, 2]))
    offset_groups = draw(st.sampled_from([1, 2, 4]))
    unit = groups * offset_groups // math.gcd(groups, offset_groups)
    cin = unit * draw(st.integers(1, 2))
    cout = groups * draw(st.integers(1, 2))
    kh, kw = draw(st.integers(1, 3)), draw(st.integers(1, 3))
    sh, sw = draw(st.integers(1, 2)), draw(st.integers(1, 2))
    dh, dw = draw(st.integers(1, 2)), draw(st.integers(1, 2))
    ph, pw = draw(st.integers(0, 2)), draw(st.integers(0, 2))
    h, w = draw(st.integers(2, 6)), draw(st.integers(2, 6))
    # Output size as a standard convolution would give it (the reference takes it as given).
    ho = max(1, (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1)
    wo = max(1, (w + 2 * pw - dw * (kw - 1) - 1) // sw + 1)
    shape = DeformConvShape(draw(st.integers(1, 2)), cin, h, w, cout, ho, wo, kh, kw, ph, pw, sh, sw, dh, dw,
                            groups, offset_groups)
    seed = draw(st.integers(0, 2**31 - 1))
    scale = draw(st.sampled_from([0.5, 2.5, 8.0]))
    return shape, seed, scale


@settings(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(dcn_cases())
def test_property_random_shapes_match_brute_force(oracle, case):
    # Any valid shape: the oracle equals float64 brute force to FP32 rounding, including
    # samples far outside the map (offset scale 8 on maps of 2..6 pixels).
    shape, seed, scale = case
    d = rand_inputs(shape, np.random.default_rng(seed), offset_scale=scale)
    out = oracle.forward_f32(shape, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    ref = brute_force_dcn(shape, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    np.testing.assert_allclose(out, ref, rtol=0, atol=5e-5)
