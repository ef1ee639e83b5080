"""GPU parity of libdcn against the CPU oracle, through the C ABI.

Bars:
  * FP32 path and the FP16 direct path: bit-identical to the oracle (the reference
    asks max relative error 1e-5; identical bits meet it with margin);
  * sampler (im2col): bit-identical to the reference gather arithmetic;
  * fused FP16 path: max |err| <= 2e-2 and mean |err| <= 1e-3 against the FP32 oracle
    run on the same FP16-rounded inputs;
  * zero padding for out-of-bounds samples exactly preserved.
"""
from __future__ import annotations

import dataclasses
import os
import sys
import tempfile

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_ABS_F16 = 2e-2
MEAN_ABS_F16 = 1e-3


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def f16_inputs(d):
    return {k: np.asarray(d[k], np.float32).astype(np.float16) for k in ("input", "offset", "mask", "weight", "bias")}


def widen(h):
    return {k: v.astype(np.float32) for k, v in h.items()}


def errors(got16, ref32):
    e = np.abs(np.asarray(got16, np.float64) - np.asarray(ref32, np.float64))
    return float(e.max()), float(e.mean())


@pytest.fixture(scope="module")
def c1(dcn, oracle):
    d = dcn.generate_config_inputs(1, 1)
    ref = oracle.forward_f32_threads(d["shape"], d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    return d, ref


@pytest.fixture(scope="module")
def c2(dcn, oracle):
    d = dcn.generate_config_inputs(2, 2)
    h = f16_inputs(d)
    w = widen(h)
    ref = oracle.forward_f32_threads(d["shape"], w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    return d["shape"], h, ref


def rand_case(shape, seed, offset_scale=3.0):
    rng = np.random.default_rng(seed)
    c = shape.counts()
    d = {
        "input": rng.standard_normal(c["input"]),
        "offset": rng.uniform(-offset_scale, offset_scale, c["offset"]),
        "mask": rng.uniform(0, 1, c["mask"]),
        "weight": rng.uniform(-0.2, 0.2, c["weight"]),
        "bias": rng.uniform(-0.1, 0.1, c["bias"]),
    }
    return {k: v.astype(np.float32) for k, v in d.items()}


GENERAL_SHAPES = [
    # (batch, Cin, H, W, Cout, Ho, Wo, Kh, Kw, ph, pw, sh, sw, dh, dw, groups, offset_groups)
    (1, 2, 5, 5, 3, 5, 5, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1),      # the reference self-test shape
    (2, 8, 6, 6, 6, 6, 6, 3, 3, 1, 1, 1, 1, 1, 1, 2, 4),
    (1, 6, 9, 8, 3, 4, 4, 3, 3, 1, 0, 2, 2, 1, 1, 1, 3),
    (1, 4, 8, 8, 4, 6, 6, 3, 3, 1, 1, 1, 1, 2, 2, 2, 2),
    (3, 16, 5, 7, 8, 5, 7, 1, 3, 0, 1, 1, 1, 1, 1, 1, 16),
]


# ---- FP32 ------------------------------------------------------------------------

def test_fp32_bit_exact_c1(gpu_ctx, c1):
    d, ref = c1
    log("case: fp32 C1 1x128x64x64 -> 64, 16 dg")
    out = gpu_ctx.run_float32(d["shape"], d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_fp32_reference_self_test(gpu_ctx, dcn, oracle):
    # correctnessTest (JasnaCLI.swift:68-110): SeededGenerator(0xC0FFEE), gate max abs < 2e-5.
    s = dcn.DeformConvShape(*GENERAL_SHAPES[0])
    rng = dcn.SeededGenerator(0xC0FFEE)
    inp = rng.floats(s.input_count, -1, 1)
    off = rng.floats(s.offset_count, -0.4, 0.4)
    msk = rng.floats(s.mask_count, 0.1, 0.9)
    w = rng.floats(s.weight_count, -0.2, 0.2)
    b = rng.floats(s.output_channels, -0.1, 0.1)
    log("case: fp32 self-test 1x2x5x5 -> 3")
    out = gpu_ctx.run_float32(s, inp, off, msk, w, b)
    ref = oracle.forward_f32(s, inp, off, msk, w, b)
    assert np.abs(out - ref).max() < 2e-5
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dims", GENERAL_SHAPES[1:], ids=lambda t: "x".join(map(str, t)))
def test_fp32_general_shapes_bit_exact(gpu_ctx, dcn, oracle, dims):
    s = dcn.DeformConvShape(*dims)
    d = rand_case(s, sum(dims))
    log("case: fp32", dims)
    out = gpu_ctx.run_float32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    ref = oracle.forward_f32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


SHARED_F32_SHAPES = [
    # groups 1, Cin % 8 == 0: the shared-sample FP32 kernel (16 pixels x 64 channels)
    ((1, 8, 7, 9, 96, 7, 9, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2), 3.0),       # 63 pixels, 2 channel blocks
    ((2, 16, 10, 6, 16, 5, 3, 2, 3, 0, 1, 2, 2, 1, 1, 1, 4), 3.0),     # 2x3 taps, stride 2
    ((1, 24, 9, 9, 40, 9, 9, 1, 1, 0, 0, 1, 1, 1, 1, 1, 3), 3.0),      # 1x1, 3 offset groups
    ((1, 8, 12, 12, 8, 6, 6, 2, 2, 0, 0, 2, 2, 1, 1, 1, 1), 3.0),      # 2x2, stride 2
    ((1, 32, 8, 8, 64, 8, 8, 1, 2, 0, 0, 1, 1, 2, 2, 1, 8), 3.0),      # 1x2, dilation 2
    ((1, 16, 16, 16, 64, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2), 20.0),  # samples far outside
]


@pytest.mark.parametrize("dims,scale", SHARED_F32_SHAPES, ids=lambda t: "x".join(map(str, t)) if isinstance(t, tuple) else str(t))
def test_fp32_shared_sample_kernel_bit_exact(gpu_ctx, dcn, oracle, dims, scale):
    """The shared-sample FP32 kernel keeps the oracle's per-output summation order: bit
    for bit over tail pixels, a partial second channel block, every supported tap count,
    strides, dilation, offset groups and samples far outside the input."""
    s = dcn.DeformConvShape(*dims)
    d = rand_case(s, sum(dims), offset_scale=scale)
    log("case: fp32 shared", dims, scale)
    out = gpu_ctx.run_float32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    ref = oracle.forward_f32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


# ---- FP16 direct (reference semantics) ---------------------------------------------

def test_fp16_direct_bit_exact_c2(gpu_ctx, c2):
    s, h, ref = c2
    log("case: fp16 direct C2")
    out = gpu_ctx.run_float16(s, h["input"], h["offset"], h["mask"], h["weight"], h["bias"])
    assert np.array_equal(out.view(np.uint16), ref.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("dims", GENERAL_SHAPES[1:3], ids=lambda t: "x".join(map(str, t)))
def test_fp16_direct_general_bit_exact(gpu_ctx, dcn, oracle, dims):
    s = dcn.DeformConvShape(*dims)
    h = f16_inputs(rand_case(s, 7 + sum(dims)))
    log("case: fp16 direct", dims)
    out = gpu_ctx.run_float16(s, h["input"], h["offset"], h["mask"], h["weight"], h["bias"])
    ref = oracle.forward_f16_direct(s, h["input"], h["offset"], h["mask"], h["weight"], h["bias"])
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


# ---- sampler --------------------------------------------------------------------

def _dev(torch, a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.cuda()


def test_im2col_bit_exact(gpu_ctx, dcn, oracle, c2):
    import torch

    s, h, _ = c2
    log("case: im2col C2")
    cols_ref = oracle.im2col_f16(s, h["input"], h["offset"], h["mask"])
    x, o, m = (_dev(torch, h[k].view(np.int16)) for k in ("input", "offset", "mask"))
    cols = torch.empty(cols_ref.size, dtype=torch.int16, device="cuda")
    gpu_ctx.im2col_f16_dev(s, x, o, m, cols)
    torch.cuda.synchronize()
    assert np.array_equal(cols.cpu().numpy().view(np.uint16), cols_ref.view(np.uint16))


# ---- fused FP16 ------------------------------------------------------------------

def test_fused_exact_sampler_matches_gather_gemm(gpu_ctx, dcn, oracle, c2):
    s, h, ref32 = c2
    log("case: fused exact sampler C2")
    cols = oracle.im2col_f16(s, h["input"], h["offset"], h["mask"])
    ref_gemm = oracle.gemm_f16(s, cols, h["weight"], h["bias"]).astype(np.float64)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, dcn.SAMPLER_EXACT)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed).astype(np.float64)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1)
    # Same FP16 A and B operands; only the FP32 summation order differs (MFMA vs serial),
    # so the two agree to about one FP16 ulp of the output.
    diff = np.abs(out - ref_gemm)
    ulp = np.maximum(np.abs(ref_gemm), 2.0 ** -14) * 2.0 ** -10
    assert np.all(diff <= 2 * ulp + 1e-6), float((diff / ulp).max())
    mx, mean = errors(out, ref32)
    log(f"  exact sampler vs FP32 oracle: max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


def test_fused_fast_c2_tolerance(gpu_ctx, dcn, c2):
    s, h, ref32 = c2
    log("case: fused fast C2")
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    mx, mean = errors(out, ref32)
    log(f"  fast sampler vs FP32 oracle: max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


FUSED_CONFIGS = [(1, 1, 8), (1, 1, 4), (1, 2, 4), (1, 2, 2),   # register variant (variant, mt, ks)
                 (2, 1, 8), (2, 1, 16), (2, 2, 8),              # LDS-staged variant
                 (3, 8, 8), (3, 4, 8), (3, 4, 4), (3, 2, 4),   # LDS windows (rows, waves)
                 (4, 8, 8), (4, 4, 4),                          # LDS windows + L1 lower rows
                 (5, 1, 8), (5, 1, 12),                         # narrow 16-pixel tiles (waves)
                 (6, 8, 8),                                     # LDS windows streamed by DMA
                 (7, 16, 8), (7, 32, 8)]                        # tile windows (tile width, waves)


def test_unsupported_fused_config_is_rejected(gpu_ctx, dcn, c2):
    s, h, _ = c2
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    # 64-pixel tiles over 16 waves need 266 KB of LDS for the cross-wave reduction.
    gpu_ctx.set_fused_config(2, 16, -1, dcn.VARIANT_STAGED)
    try:
        with pytest.raises(dcn.DeformConvError) as e:
            gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
        assert e.value.status == dcn.INVALID_ARGUMENT and "unsupported fused config" in e.value.message
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)


@pytest.mark.parametrize("variant,mt,ks", FUSED_CONFIGS)
@pytest.mark.parametrize("sampler", [0, 1])
def test_fused_configs(gpu_ctx, dcn, c2, variant, mt, ks, sampler):
    s, h, ref32 = c2
    log("case: fused config", variant, mt, ks, sampler)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(mt, ks, sampler, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
        again = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1)
    assert np.array_equal(out.view(np.uint16), again.view(np.uint16))  # deterministic
    mx, mean = errors(out, ref32)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, (mx, mean)


@pytest.mark.parametrize("variant,mt,ks", FUSED_CONFIGS)
def test_exact_sampler_through_one_hot_weights(gpu_ctx, dcn, oracle, c2, variant, mt, ks):
    """Each fused kernel with the reference's sampler arithmetic and one-hot weights (output
    channel oc weighs one K element, ic * 9 + tap = 18 oc, with 1.0; no bias): every other
    product is a signed zero, so each output is one sample, exactly, and must equal the
    oracle's gather (deform_conv2d_fp16_jasna_gather) at that K element and pixel, value
    for value (zeros of either sign compare equal)."""
    s, h, _ = c2
    log("case: one-hot exact sampler", variant, mt, ks)
    w = np.zeros((64, 128, 9), np.float16)
    kk = 18 * np.arange(64)
    w[np.arange(64), kk // 9, kk % 9] = 1.0
    bias = np.zeros(64, np.float16)
    packed = gpu_ctx.prepack(s, w.reshape(-1), bias)
    gpu_ctx.set_fused_config(mt, ks, dcn.SAMPLER_EXACT, variant)
    try:
        cfg = gpu_ctx.get_fused_config(s)
        assert (cfg["variant"], cfg["sampler"]) == (variant, dcn.SAMPLER_EXACT), cfg
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    cols = oracle.im2col_f16(s, h["input"], h["offset"], h["mask"]).view(np.float16).reshape(64 * 64, 128 * 9)
    want = cols[:, kk].T.astype(np.float32)  # [oc][pixel]
    got = out.reshape(64, 64 * 64).astype(np.float32)
    bad = np.nonzero(got != want)
    assert bad[0].size == 0, (bad[0].size, got[bad][:4], want[bad][:4])


def test_automatic_config_per_workload(gpu_ctx, dcn):
    """The automatic choice: narrow 16-pixel tiles for one 64 x 64 map (C2), the tile kernel
    for batches of small maps (C3) and for one large map (C5), with either sampler."""
    want = {2: dcn.VARIANT_NARROW, 3: 7, 5: 7}
    for c, v in want.items():
        assert gpu_ctx.get_fused_config(dcn.config_shape(c))["variant"] == v, c
    gpu_ctx.set_fused_config(0, 0, dcn.SAMPLER_EXACT)
    try:
        for c, v in want.items():
            cfg = gpu_ctx.get_fused_config(dcn.config_shape(c))
            assert (cfg["variant"], cfg["sampler"]) == (v, dcn.SAMPLER_EXACT), (c, cfg)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1)


@pytest.fixture(scope="module")
def c3(dcn, oracle):
    """C3's 16 tiles with the FP32 oracle over the whole batch (computed once)."""
    d = dcn.generate_config_inputs(3, 3)
    h = f16_inputs(d)
    w = widen(h)
    ref = oracle.forward_f32_threads(d["shape"], w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    return d["shape"], h, ref


@pytest.mark.parametrize("variant", [0, 3, 5, 6, 7])
def test_fused_c3_batched_tiles(gpu_ctx, dcn, c3, variant):
    s, h, ref = c3
    log("case: fused C3 16 tiles, variant", variant)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, -1, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    n = dataclasses.replace(s, batch=1).counts()["output"]
    for b in range(s.batch):  # every tile, every output channel and pixel
        mx, mean = errors(out[b * n:(b + 1) * n], ref[b * n:(b + 1) * n])
        log(f"  tile {b}: max {mx:.3e} mean {mean:.3e}")
        assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, b


@pytest.mark.parametrize("cout", [32, 128])
@pytest.mark.parametrize("variant", [3, 4])
def test_window_one_group_per_stage(gpu_ctx, dcn, oracle, cout, variant):
    """An odd group count puts one offset group in each stage of the window kernel
    (5 K-steps per stage): the weight-fragment ring must hand every stage its own K-steps.
    Three groups, three stages, against the oracle."""
    s = dcn.DeformConvShape(1, 24, 24, 40, cout, 24, 40, 3, 3, 1, 1, 1, 1, 1, 1, 1, 3)
    rng = np.random.default_rng(cout + variant)
    c = s.counts()
    h = {"input": rng.standard_normal(c["input"]).astype(np.float16),
         "offset": rng.uniform(-3, 3, c["offset"]).astype(np.float16),
         "mask": rng.random(c["mask"]).astype(np.float16),
         "weight": (rng.standard_normal(c["weight"]) * 0.05).astype(np.float16),
         "bias": (rng.standard_normal(cout) * 0.1).astype(np.float16)}
    log("case: window, 3 groups, cout", cout, "variant", variant)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, -1, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    w = widen(h)
    ref = oracle.forward_f32_threads(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    log(f"  max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


@pytest.mark.parametrize("spread", [3.0, 40.0])
def test_window_batch_uniform_and_overflow(gpu_ctx, dcn, oracle, spread):
    """The window variant on a batch of 64 x 64 maps (the uniform LDS K-loop when every
    window of a stage fits); offsets of +-40 px overflow the windows, so the stage falls
    back to the general loop with global gathers. Both within the FP16 bars."""
    s = dcn.DeformConvShape(2, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    rng = np.random.default_rng(int(spread) + 7)
    c = s.counts()
    h = {"input": rng.standard_normal(c["input"]).astype(np.float16),
         "offset": rng.uniform(-spread, spread, c["offset"]).astype(np.float16),
         "mask": rng.random(c["mask"]).astype(np.float16),
         "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
         "bias": (rng.standard_normal(64) * 0.1).astype(np.float16)}
    log("case: window batch, offsets +-", spread)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, -1, 3)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    w = widen(h)
    ref = oracle.forward_f32_threads(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    log(f"  max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


@pytest.mark.parametrize("batch,h,w", [(5, 7, 9), (4, 16, 16), (16, 64, 64)])
def test_narrow_batch_equals_single_images(gpu_ctx, dcn, batch, h, w):
    """The narrow variant over a batch (from four images on: several images per workgroup,
    weights kept in registers) == one call per image, bit for bit."""
    s = dcn.DeformConvShape(batch, 128, h, w, 64, h, w, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    one = dataclasses.replace(s, batch=1)
    rng = np.random.default_rng(batch * 100 + h)
    c = s.counts()
    x = rng.standard_normal(c["input"]).astype(np.float16)
    off = (rng.standard_normal(c["offset"]) * 4).astype(np.float16)
    msk = rng.random(c["mask"]).astype(np.float16)
    wt = (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16)
    b = (rng.standard_normal(64) * 0.1).astype(np.float16)
    log("case: narrow batch", batch, h, w)
    gpu_ctx.set_fused_config(0, 0, -1, 5)
    try:
        packed = gpu_ctx.prepack(s, wt, b)
        out = gpu_ctx.run_float16_prepacked(s, x, off, msk, packed)
        c1 = one.counts()
        for i in range(batch):
            o1 = gpu_ctx.run_float16_prepacked(one, x[i * c1["input"]:(i + 1) * c1["input"]],
                                               off[i * c1["offset"]:(i + 1) * c1["offset"]],
                                               msk[i * c1["mask"]:(i + 1) * c1["mask"]], packed)
            assert np.array_equal(out[i * c1["output"]:(i + 1) * c1["output"]].view(np.uint16),
                                  np.asarray(o1).view(np.uint16)), i
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)


@pytest.fixture(scope="module")
def c5(dcn, oracle):
    """C5's large map with the FP32 oracle over all 64 output channels (computed once)."""
    d = dcn.generate_config_inputs(5, 5)
    h = f16_inputs(d)
    w = widen(h)
    ref = oracle.forward_f32_threads(d["shape"], w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    return d["shape"], h, ref


@pytest.mark.parametrize("variant", [0, 6, 7])
def test_fused_c5_large_map(gpu_ctx, dcn, c5, variant):
    s, h, ref = c5
    log("case: fused C5 1x128x180x320, variant", variant)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, -1, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    plane = s.output_height * s.output_width
    # Every output channel and pixel, reported in slices of 16 channels.
    for lo in range(0, s.output_channels, 16):
        sl = slice(lo * plane, (lo + 16) * plane)
        mx, mean = errors(out[sl], ref[sl])
        log(f"  C5 oc {lo}..{lo + 15}: max {mx:.3e} mean {mean:.3e}")
        assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, lo
    mx, mean = errors(out, ref)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16
    assert np.all(np.isfinite(out.astype(np.float32)))


EDGE_SHAPES = [
    (1, 128, 7, 9, 64, 7, 9, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16),    # 63 pixels: tile tail
    (2, 8, 11, 13, 32, 11, 13, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1),   # 9 K-blocks (odd), Cout 32
    (1, 64, 10, 10, 96, 10, 10, 3, 3, 1, 1, 1, 1, 1, 1, 1, 8),  # Cout 96
    (1, 32, 9, 12, 128, 9, 12, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2),   # Cout 128, 16 channels per group
    (1, 16, 17, 15, 64, 8, 7, 3, 3, 1, 1, 2, 2, 1, 1, 1, 2),    # stride 2
    (1, 16, 12, 12, 32, 10, 10, 3, 3, 1, 1, 1, 1, 2, 2, 1, 1),  # dilation 2
    (3, 24, 6, 5, 32, 6, 5, 1, 3, 0, 1, 1, 1, 1, 1, 1, 3),      # 1x3 kernel, batch 3
    (2, 16, 7, 6, 32, 7, 6, 3, 1, 1, 0, 1, 1, 1, 1, 1, 2),      # 3x1 kernel (Kw 1)
    (1, 32, 5, 9, 64, 5, 9, 1, 1, 0, 0, 1, 1, 1, 1, 1, 4),      # 1x1 kernel (Kh*Kw 1)
    (5, 128, 7, 9, 64, 7, 9, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16),    # batch 5 of 63-pixel maps
]


@pytest.mark.parametrize("dims", EDGE_SHAPES, ids=lambda t: "x".join(map(str, t)))
@pytest.mark.parametrize("sampler", [0, 1])
@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5, 6, 7])
def test_fused_edge_shapes(gpu_ctx, dcn, oracle, dims, sampler, variant):
    s = dcn.DeformConvShape(*dims)
    assert s.fused_supported
    d = rand_case(s, sum(dims), offset_scale=4.0)
    d["weight"] *= 0.5
    h = f16_inputs(d)
    w = widen(h)
    log("case: fused edge", dims, "sampler", sampler, "variant", variant)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, sampler, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1)
    ref = oracle.forward_f32(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, (mx, mean)


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5, 6, 7])
def test_large_offsets_force_global_fallback(gpu_ctx, dcn, oracle, variant):
    # Offsets up to +-40 px on a 64x64 map: a tile's sample box spans the whole plane
    # (74 KB), larger than one LDS window, so the window variant gathers from global.
    s = dcn.JASNA_SHAPE
    d = rand_case(s, 40, offset_scale=40.0)
    d["weight"] *= 0.3
    h = f16_inputs(d)
    w = widen(h)
    log("case: offsets +-40, variant", variant)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, -1, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    ref = oracle.forward_f32_threads(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, (mx, mean)


@pytest.mark.parametrize("tw", [16, 32])
def test_tile_stages_lds_and_global(gpu_ctx, dcn, oracle, tw):
    """The tile variant with offsets of +-3 px in groups 0-7 and +-40 px in groups 8-15:
    stages 0-3 gather from LDS windows, stages 4-7 (windows over the LDS budget) from global
    memory, in one call over a batch of two 64 x 64 maps; within the FP16 bars."""
    s = dcn.DeformConvShape(2, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    rng = np.random.default_rng(tw)
    c = s.counts()
    off = rng.uniform(-3, 3, c["offset"]).reshape(2, 16, 18, 64 * 64)
    off[:, 8:] = rng.uniform(-40, 40, off[:, 8:].shape)
    h = {"input": rng.standard_normal(c["input"]).astype(np.float16),
         "offset": off.reshape(-1).astype(np.float16),
         "mask": rng.random(c["mask"]).astype(np.float16),
         "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
         "bias": (rng.standard_normal(64) * 0.1).astype(np.float16)}
    log("case: tile variant, LDS and global stages, width", tw)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(tw, 8, -1, 7)
    try:
        assert gpu_ctx.get_fused_config(s)["variant"] == 7
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
        again = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    assert np.array_equal(out.view(np.uint16), again.view(np.uint16))
    w = widen(h)
    ref = oracle.forward_f32_threads(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    log(f"  max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


def tile_stage_windows(off, H, W, G, th, tw):
    """Bytes of the two CB8 windows of every (map, tile, stage) of the tile variant: each
    window is the bounding box of the clamped sample corners of the stage's group over the
    tile, plus one row and column (16 bytes per pixel)."""
    off = off.astype(np.float32).reshape(-1, G, 9, 2, H, W)
    ky = (np.arange(9) // 3)[None, :, None, None] - 1
    kx = (np.arange(9) % 3)[None, :, None, None] - 1
    sizes = []
    for b in range(off.shape[0]):
        iy = np.clip(np.floor(np.arange(H)[None, None, :, None] + ky + off[b, :, :, 0]), -2, H).astype(int)
        ix = np.clip(np.floor(np.arange(W)[None, None, None, :] + kx + off[b, :, :, 1]), -2, W).astype(int)
        for ty in range(0, H, th):
            for tx in range(0, W, tw):
                for st in range(G // 2):
                    pair = []
                    for g in (2 * st, 2 * st + 1):
                        y = iy[g, :, ty:ty + th, tx:tx + tw]
                        x = ix[g, :, ty:ty + th, tx:tx + tw]
                        pair.append((y.max() - y.min() + 2) * (x.max() - x.min() + 2) * 16)
                    sizes.append(pair)
    return np.array(sizes)


@pytest.mark.parametrize("tw", [16, 32])
def test_tile_split_stages(gpu_ctx, dcn, oracle, tw):
    """The tile variant with offsets of +-3 px in groups 0-7 and +-20 px in groups 8-15:
    stages 4-7 have windows that fit the 64 KB LDS buffer one at a time but not together,
    so each runs one pass per group (the other group's lanes masked to zero); within the
    FP16 bars of the FP32 oracle, and deterministic."""
    s = dcn.DeformConvShape(2, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    rng = np.random.default_rng(100 + tw)
    c = s.counts()
    off = rng.uniform(-3, 3, c["offset"]).reshape(2, 16, 18, 64 * 64)
    off[:, 8:] = rng.uniform(-20, 20, off[:, 8:].shape)
    off = off.reshape(-1).astype(np.float16)
    sizes = tile_stage_windows(off, 64, 64, 16, 8 * 16 // tw, tw)
    split = (sizes.sum(axis=1) > 65536) & (sizes.max(axis=1) <= 65536)
    assert split.sum() >= 8, "the case must exercise split stages"
    h = {"input": rng.standard_normal(c["input"]).astype(np.float16),
         "offset": off,
         "mask": rng.random(c["mask"]).astype(np.float16),
         "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
         "bias": (rng.standard_normal(64) * 0.1).astype(np.float16)}
    log("case: tile variant, split stages, width", tw, "split stages", int(split.sum()), "of", len(split))
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(tw, 8, -1, 7)
    try:
        assert gpu_ctx.get_fused_config(s)["variant"] == 7
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
        again = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    assert np.array_equal(out.view(np.uint16), again.view(np.uint16))
    w = widen(h)
    ref = oracle.forward_f32_threads(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    log(f"  max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


@pytest.mark.parametrize("tw", [16, 32])
def test_tile_exact_sampler_matches_gather_gemm(gpu_ctx, dcn, oracle, tw):
    """The tile variant pinned with the reference's sampler arithmetic (FP32 bilinear in the
    reference's association, half(sampled * mask)), on the split-stage case above (one
    pass per group in stages 4-7): the samples are the oracle im2col's FP16 values, so the
    output is within two FP16 ulps of the oracle's gather + FP32 GEMM (only the summation
    order differs), and deterministic."""
    s = dcn.DeformConvShape(2, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    rng = np.random.default_rng(200 + tw)
    c = s.counts()
    off = rng.uniform(-3, 3, c["offset"]).reshape(2, 16, 18, 64 * 64)
    off[:, 8:] = rng.uniform(-20, 20, off[:, 8:].shape)
    off = off.reshape(-1).astype(np.float16)
    sizes = tile_stage_windows(off, 64, 64, 16, 8 * 16 // tw, tw)
    split = (sizes.sum(axis=1) > 65536) & (sizes.max(axis=1) <= 65536)
    assert split.sum() >= 8, "the case must exercise split stages"
    h = {"input": rng.standard_normal(c["input"]).astype(np.float16),
         "offset": off,
         "mask": rng.random(c["mask"]).astype(np.float16),
         "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
         "bias": (rng.standard_normal(64) * 0.1).astype(np.float16)}
    log("case: tile variant, exact sampler, width", tw, "split stages", int(split.sum()))
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(tw, 8, dcn.SAMPLER_EXACT, 7)
    try:
        assert gpu_ctx.get_fused_config(s) == {"variant": 7, "mt": tw, "ks": 8, "sampler": dcn.SAMPLER_EXACT}
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
        again = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    assert np.array_equal(out.view(np.uint16), again.view(np.uint16))
    cols = oracle.im2col_f16(s, h["input"], h["offset"], h["mask"])
    ref = oracle.gemm_f16(s, cols, h["weight"], h["bias"]).astype(np.float64)
    diff = np.abs(out.astype(np.float64) - ref)
    ulp = np.maximum(np.abs(ref), 2.0 ** -14) * 2.0 ** -10
    assert np.all(diff <= 2 * ulp + 1e-6), float((diff / ulp).max())


@pytest.mark.parametrize("batch,h,w,tw", [(1, 180, 320, 16), (9, 64, 64, 16), (1, 120, 320, 32), (1, 150, 264, 16),
                                          (16, 64, 64, 16), (16, 64, 64, 32), (1, 250, 248, 16)])
def test_tile_placement_plan_is_bit_identical(gpu_ctx, dcn, oracle, batch, h, w, tw):
    """The tile kernel's placements (ks 8): cost-ordered where an XCD's band has 33-63 tiles
    (C5's 460, 9 maps of 64 x 64 = 288, 300 tiles of 4 x 32, 19 x 17 partial tiles with a
    short last band), heavier-of-two first where it has exactly 64 (C3's 512 tiles of 8 x 16
    and of 4 x 32; 32 x 16 tiles of a 250 x 248 map, partial at two edges). They only
    change which workgroup runs which tile: the output equals the fixed placement's (ks 1)
    bit for bit, and the FP32 oracle within the FP16 bars."""
    s = dcn.DeformConvShape(batch, 128, h, w, 64, h, w, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    th = 128 // tw
    tiles = batch * ((h + th - 1) // th) * ((w + tw - 1) // tw)
    per_xcd = (tiles + 7) // 8
    assert 32 < per_xcd <= 64, tiles
    rng = np.random.default_rng(tiles)
    c = s.counts()
    # a smooth +-24 px flow (so that some tiles' windows split) plus a +-6 px residue
    flow = np.repeat(np.repeat(rng.uniform(-24, 24, (batch, 2, 6, 6)), (h + 5) // 6, axis=2), (w + 5) // 6, axis=3)
    flow = flow[:, :, :h, :w]
    off = (flow[:, None] + rng.uniform(-6, 6, (batch, 144, 2, h, w))).reshape(-1)
    h16 = {"input": rng.standard_normal(c["input"]).astype(np.float16),
           "offset": off.astype(np.float16),
           "mask": rng.random(c["mask"]).astype(np.float16),
           "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
           "bias": (rng.standard_normal(64) * 0.1).astype(np.float16)}
    log("case: tile placement plan", batch, h, w, "width", tw, "tiles", tiles)
    packed = gpu_ctx.prepack(s, h16["weight"], h16["bias"])
    outs = {}
    try:
        for ks in (8, 1):
            gpu_ctx.set_fused_config(tw, ks, -1, 7)
            assert gpu_ctx.get_fused_config(s) == {"variant": 7, "mt": tw, "ks": ks, "sampler": 1}
            outs[ks] = gpu_ctx.run_float16_prepacked(s, h16["input"], h16["offset"], h16["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    assert np.array_equal(outs[8].view(np.uint16), outs[1].view(np.uint16))
    w32 = widen(h16)
    ref = oracle.forward_f32_threads(s, w32["input"], w32["offset"], w32["mask"], w32["weight"], w32["bias"])
    mx, mean = errors(outs[8], ref)
    log(f"  max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


@pytest.mark.parametrize("batch,h,w,cout,tw", [(2, 64, 64, 64, 16), (1, 24, 48, 64, 16), (2, 64, 64, 32, 16),
                                                (1, 40, 96, 64, 32)])
def test_tile_clock_stamps_every_tile(gpu_ctx, dcn, batch, h, w, cout, tw):
    """dcn_set_tile_clock_dev: with a clock buffer set, the tile kernel writes one record per
    workgroup that runs a tile (start <= both wave ends, every tile exactly once, the
    grid's padding workgroups write nothing), the output is bit-identical to a launch
    without stamps, and a buffer smaller than 4 stamps per workgroup is refused."""
    import torch

    s = dcn.DeformConvShape(batch, 128, h, w, cout, h, w, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    th = 128 // tw
    tiles = batch * ((h + th - 1) // th) * ((w + tw - 1) // tw)
    grid = (tiles + 7) // 8 * 8
    rng = np.random.default_rng(tiles)
    c = s.counts()
    h16 = {"input": rng.standard_normal(c["input"]).astype(np.float16),
           "offset": rng.uniform(-8, 8, c["offset"]).astype(np.float16),
           "mask": rng.random(c["mask"]).astype(np.float16),
           "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
           "bias": (rng.standard_normal(cout) * 0.1).astype(np.float16)}
    log("case: tile clock", batch, h, w, "cout", cout, "width", tw, "tiles", tiles, "grid", grid)
    dev = {k: _dev(torch, h16[k].view(np.int16)) for k in ("input", "offset", "mask", "weight", "bias")}
    out = torch.empty(c["output"], dtype=torch.int16, device="cuda")
    packed = gpu_ctx.prepack_dev(s, dev["weight"], dev["bias"])
    gpu_ctx.reserve(s)
    gpu_ctx.set_fused_config(tw, 8, -1, 7)
    try:
        assert gpu_ctx.get_fused_config(s) == {"variant": 7, "mt": tw, "ks": 8, "sampler": 1}
        gpu_ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out)
        torch.cuda.synchronize()
        ref = out.clone()
        out.zero_()
        clock = torch.zeros(4 * grid, dtype=torch.int64, device="cuda")
        gpu_ctx.set_tile_clock_dev(clock)
        gpu_ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        rec = clock.cpu().numpy().view(np.uint64).reshape(grid, 4)
        small = torch.zeros(4 * grid - 1, dtype=torch.int64, device="cuda")
        gpu_ctx.set_tile_clock_dev(small)
        with pytest.raises(dcn.DeformConvError):
            gpu_ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out)
        torch.cuda.synchronize()
    finally:
        gpu_ctx.set_tile_clock_dev(None)
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    assert not np.any(small.cpu().numpy())  # the refused launch ran nothing
    per_xcd = (tiles + 7) // 8
    has_tile = np.array([b // 8 < min(per_xcd, tiles - (b % 8) * per_xcd) for b in range(grid)])
    assert np.all(rec[has_tile, 0] > 0) and not np.any(rec[~has_tile])
    r = rec[has_tile]
    assert np.all(r[:, 1] >= r[:, 0]) and np.all(r[:, 2] >= r[:, 0])
    assert np.all(r[:, 1] - r[:, 0] < 100_000_000)  # < 1 s on the 100 MHz clock
    tile_ids = (r[:, 3] & np.uint64(0x0FFFFFFF)).astype(np.int64)
    assert np.array_equal(np.sort(tile_ids), np.arange(tiles))


def test_tile_pair_placement_runs_heavy_tiles_first(gpu_ctx, dcn):
    """Bands of exactly 64 tiles (C3's 16 maps of 64 x 64): locals c and c + 32 share a CU
    and c is dispatched first, so a heavy tile c + 32 (window-box estimate of group 0's
    centre tap above three quarters of a group's buffer share) is swapped into local c.
    Planted: a few tiles whose estimate channels (offset channels 8, 9) spread +-32 px
    (estimates 2205-3283 on the host) while every other offset stays within +-1 px (at most
    228). The clock records show each heavy second-slot
    tile run by local c and its light partner by local c + 32, a heavy tile already in a
    first slot left where it is, every other tile in its natural slot, and the output equal
    to the fixed placement's bit for bit."""
    import torch

    s = dcn.DeformConvShape(16, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    tiles, grid = 512, 512  # 8 x 16 tiles, 32 per map, bands of 64
    rng = np.random.default_rng(64)
    c = s.counts()
    off = rng.uniform(-1, 1, (16, 288, 64, 64))
    heavy = [40, 100, 300, 455]  # band-local 40, 36, 44 (second slots) and 7 (a first slot)
    for t in heavy:
        b, r = divmod(t, 32)
        ty, tx = divmod(r, 4)
        off[b, 8:10, ty * 8:(ty + 1) * 8, tx * 16:(tx + 1) * 16] = rng.uniform(-32, 32, (2, 8, 16))
    h16 = {"input": rng.standard_normal(c["input"]).astype(np.float16),
           "offset": off.reshape(-1).astype(np.float16),
           "mask": rng.random(c["mask"]).astype(np.float16),
           "weight": (rng.standard_normal(c["weight"]) * 0.03).astype(np.float16),
           "bias": (rng.standard_normal(64) * 0.1).astype(np.float16)}
    log("case: tile pair placement, heavy tiles", heavy)
    dev = {k: _dev(torch, h16[k].view(np.int16)) for k in ("input", "offset", "mask", "weight", "bias")}
    out = torch.empty(c["output"], dtype=torch.int16, device="cuda")
    packed = gpu_ctx.prepack_dev(s, dev["weight"], dev["bias"])
    gpu_ctx.reserve(s)
    clock = torch.zeros(4 * grid, dtype=torch.int64, device="cuda")
    try:
        gpu_ctx.set_fused_config(16, 1, -1, 7)
        gpu_ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out)
        torch.cuda.synchronize()
        fixed = out.clone()
        out.zero_()
        gpu_ctx.set_fused_config(16, 8, -1, 7)
        assert gpu_ctx.get_fused_config(s) == {"variant": 7, "mt": 16, "ks": 8, "sampler": 1}
        gpu_ctx.set_tile_clock_dev(clock)
        gpu_ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out)
        torch.cuda.synchronize()
    finally:
        gpu_ctx.set_tile_clock_dev(None)
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    assert torch.equal(out, fixed)
    rec = clock.cpu().numpy().view(np.uint64).reshape(grid, 4)
    ran = (rec[:, 3] & np.uint64(0x0FFFFFFF)).astype(np.int64)  # the tile workgroup b ran
    blocks = np.arange(grid)
    natural = (blocks % 8) * 64 + blocks // 8
    assert np.array_equal(np.sort(ran), np.arange(tiles))
    want = natural.copy()
    for t in heavy:
        band, cl = divmod(t, 64)
        if cl >= 32:  # swapped with the light tile band * 64 + cl - 32
            want[(cl - 32) * 8 + band] = t
            want[cl * 8 + band] = t - 32
    assert np.array_equal(ran, want), [(int(b), int(ran[b]), int(want[b])) for b in np.nonzero(ran != want)[0][:8]]


TILE_EDGE_SHAPES = [
    # (batch, Cin, H, W, Cout, Ho, Wo, Kh, Kw, ph, pw, sh, sw, dh, dw, groups, offset_groups)
    (1, 16, 13, 40, 32, 13, 40, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2),   # Wo % 16 != 0, H % 8 != 0, Cout 32 (NB 1)
    (2, 32, 17, 31, 64, 9, 16, 3, 3, 1, 1, 2, 2, 1, 1, 1, 4),    # stride 2, H != Ho
    (1, 16, 12, 24, 32, 12, 24, 3, 3, 2, 2, 1, 1, 2, 2, 1, 2),   # dilation 2, pad 2
    (1, 32, 10, 18, 64, 8, 16, 3, 3, 0, 0, 1, 1, 1, 1, 1, 4),    # pad 0
    (1, 16, 9, 14, 64, 11, 16, 3, 3, 2, 2, 1, 1, 1, 1, 1, 2),    # pad 2: output larger than input
]


@pytest.mark.parametrize("dims", TILE_EDGE_SHAPES, ids=lambda t: "x".join(map(str, t)))
@pytest.mark.parametrize("tw", [16, 32])
def test_tile_edge_shapes(gpu_ctx, dcn, oracle, dims, tw):
    """The tile kernel (variant 7, asserted) on shapes off its C3/C5 path: rows that end
    inside a tile (clamped lanes, offset chunks past the row), output rows past the map,
    Cout 32, stride and dilation 2, pad 0 and 2; within the FP16 bars of the FP32 oracle."""
    s = dcn.DeformConvShape(*dims)
    d = rand_case(s, sum(dims) + tw, offset_scale=4.0)
    d["weight"] *= 0.5
    h = f16_inputs(d)
    w = widen(h)
    log("case: tile edge", dims, "width", tw)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(tw, 8, -1, 7)
    try:
        assert gpu_ctx.get_fused_config(s) == {"variant": 7, "mt": tw, "ks": 8, "sampler": 1}
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    ref = oracle.forward_f32(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    log(f"  max {mx:.3e} mean {mean:.3e}")
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, (mx, mean)


def bf16_case(dcn, shape, seed, offset_scale=3.0):
    """A random case as BF16 bit patterns (the FP32 draws of rand_case, rounded)."""
    return {k: dcn.f32_to_bf16_bits(v) for k, v in rand_case(shape, seed, offset_scale).items()}


def bf16_reference(dcn, oracle, s, b):
    """The BF16 path's output before its final rounding: the oracle's BF16 columns times the
    widened BF16 weights plus the bias, in float64; and the same with absolute values (the
    scale of the FP32 summation-order error)."""
    f = dcn.bf16_bits_to_f32
    plane = s.output_height * s.output_width
    kdim = s.input_channels * s.kernel_height * s.kernel_width // s.groups
    cols = f(oracle.im2col_bf16(s, b["input"], b["offset"], b["mask"])).astype(np.float64)
    cols = cols.reshape(s.batch, plane, s.groups, kdim)
    W = f(b["weight"]).astype(np.float64).reshape(s.groups, s.output_channels // s.groups, kdim)
    bias = f(b["bias"]).astype(np.float64).reshape(s.groups, -1)[None, :, :, None]
    exact = np.einsum("bpgk,gok->bgop", cols, W) + bias
    scale = np.einsum("bpgk,gok->bgop", np.abs(cols), np.abs(W)) + np.abs(bias)
    return exact.ravel(), scale.ravel(), kdim


def assert_within_one_bf16_step(dcn, got_bits, exact, scale, kdim):
    """Each output lies within one BF16 step of the exact product, after allowing for the
    FP32 summation-order error bound kdim * 2^-24 * sum |terms| (the GPU sums the same BF16
    products in FP32 in another order and rounds once)."""
    got = dcn.bf16_bits_to_f32(got_bits).astype(np.float64)
    near = dcn.f32_to_bf16_bits(exact.astype(np.float32))
    up = dcn.bf16_bits_to_f32(near | 1).astype(np.float64)
    down = dcn.bf16_bits_to_f32(near & 0xFFFE).astype(np.float64)
    step = np.maximum(np.abs(up - down), 2.0 ** -133)
    bound = step + (kdim + 1) * 2.0 ** -24 * scale
    err = np.abs(got - exact)
    log(f"  BF16: max |got - exact| {float(err.max()):.3e}, {float(np.max(err / step)):.2f} BF16 steps")
    assert np.all(err <= bound), float(np.max(err / bound))


@pytest.mark.parametrize("dims", [(1, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16),
                                  (2, 16, 17, 15, 32, 9, 8, 3, 3, 1, 1, 2, 2, 1, 1, 1, 2),
                                  (1, 64, 10, 10, 96, 10, 10, 3, 3, 1, 1, 1, 1, 1, 1, 1, 8),
                                  (9, 16, 64, 64, 32, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2),
                                  (1, 16, 180, 200, 32, 180, 200, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2),
                                  (9, 32, 64, 64, 32, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)],
                         ids=lambda t: "x".join(map(str, t)))
def test_bf16_fused_matches_oracle_columns(gpu_ctx, dcn, oracle, dims):
    """The BF16 fused path against the oracle's BF16 gather times the weights: C2's shape,
    stride 2 over a batch and 96 output channels on the narrow kernel; above 1024 tiles of
    32 pixels the window kernel (a batch of 64 x 64 maps, one 180 x 200 map) or, for a shape
    it does not take (32 channels per offset group), the register variant. Also against the
    FP32 oracle on the widened inputs within bars 8x the FP16 ones (BF16 keeps 3 fewer
    significant bits)."""
    s = dcn.DeformConvShape(*dims)
    b = bf16_case(dcn, s, sum(dims))
    log("case: BF16 fused", dims)
    packed = gpu_ctx.prepack_bf16(s, b["weight"], b["bias"])
    out = gpu_ctx.run_bfloat16_prepacked(s, b["input"], b["offset"], b["mask"], packed)
    again = gpu_ctx.run_bfloat16_prepacked(s, b["input"], b["offset"], b["mask"], packed)
    assert np.array_equal(out, again)
    assert_within_one_bf16_step(dcn, out, *bf16_reference(dcn, oracle, s, b))
    f = dcn.bf16_bits_to_f32
    ref32 = oracle.forward_f32_threads(s, *[f(b[k]) for k in ("input", "offset", "mask", "weight", "bias")])
    mx, mean = errors(f(out), ref32)
    log(f"  vs FP32 oracle: max {mx:.3e} mean {mean:.3e}")
    assert mx <= 8 * MAX_ABS_F16 and mean <= 8 * MEAN_ABS_F16


def test_bf16_and_f16_packs_do_not_mix(gpu_ctx, dcn, c2):
    s, h, _ = c2
    p16 = gpu_ctx.prepack(s, h["weight"], h["bias"])
    pbf = gpu_ctx.prepack_bf16(s, h["weight"].view(np.uint16), h["bias"].view(np.uint16))
    x = h["input"].view(np.uint16)
    with pytest.raises(dcn.DeformConvError):
        gpu_ctx.run_bfloat16_prepacked(s, x, h["offset"].view(np.uint16), h["mask"].view(np.uint16), p16)
    with pytest.raises(dcn.DeformConvError):
        gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], pbf)


def test_bf16_device_entry_points(gpu_ctx, dcn, oracle):
    import torch

    s = dcn.DeformConvShape(1, 32, 12, 12, 32, 12, 12, 3, 3, 1, 1, 1, 1, 1, 1, 1, 4)
    b = bf16_case(dcn, s, 77)
    log("case: BF16 device entry points")
    host = gpu_ctx.run_bfloat16_prepacked(s, b["input"], b["offset"], b["mask"],
                                          gpu_ctx.prepack_bf16(s, b["weight"], b["bias"]))
    dev = {k: torch.tensor(v.view(np.int16)).cuda() for k, v in b.items()}
    packed = gpu_ctx.prepack_bf16_dev(s, dev["weight"], dev["bias"])
    out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
    gpu_ctx.forward_bf16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), host)
    # From the channel-block copy: the repack moves 16-bit words, whatever their format.
    cb8 = torch.empty(gpu_ctx.cb8_count(s), dtype=torch.int16, device="cuda")
    gpu_ctx.pack_input_cb8_dev(s, dev["input"], cb8)
    out.zero_()
    gpu_ctx.forward_bf16_prepacked_cb8_dev(s, cb8, dev["offset"], dev["mask"], packed, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), host)
    with pytest.raises(dcn.DeformConvError):
        gpu_ctx.forward_f16_prepacked_cb8_dev(s, cb8, dev["offset"], dev["mask"], packed, out)
    packed.free()


def test_zero_padding_exact(gpu_ctx, dcn, c2):
    s, h, _ = c2
    log("case: zero padding")
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    bias_out = np.repeat(h["bias"], s.output_height * s.output_width)
    for far in (1000.0, -1000.0, 66.0, -2.0 - 64.0):
        off = np.full_like(h["offset"], far)
        for variant in (1, 2, 3, 4, 5, 6, 7):
            gpu_ctx.set_fused_config(0, 0, -1, variant)
            try:
                out = gpu_ctx.run_float16_prepacked(s, h["input"], off, h["mask"], packed)
            finally:
                gpu_ctx.set_fused_config(0, 0, -1, 0)
            assert np.array_equal(out.view(np.uint16), bias_out.view(np.uint16)), (far, variant)
        out = gpu_ctx.run_float16(s, h["input"], off, h["mask"], h["weight"], h["bias"])
        assert np.array_equal(out.view(np.uint16), bias_out.view(np.uint16)), far
    zero_mask = np.zeros_like(h["mask"])
    out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], zero_mask, packed)
    assert np.array_equal(out.view(np.uint16), bias_out.view(np.uint16))


def test_samples_straddling_the_border(gpu_ctx, dcn, oracle):
    # Offsets that put corners exactly on -1, 0, H-1, H and just beyond, per corner.
    s = dcn.DeformConvShape(1, 16, 6, 7, 32, 6, 7, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    rng = np.random.default_rng(12)
    d = rand_case(s, 12)
    choices = np.array([-7.5, -6.0, -5.25, -1.0, -0.5, 0.0, 0.5, 1.0, 5.5, 6.0, 6.75, 7.0], np.float32)
    d["offset"] = rng.choice(choices, d["offset"].size).astype(np.float32)
    h = f16_inputs(d)
    w = widen(h)
    log("case: border straddle")
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    ref = oracle.forward_f32(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    mx, mean = errors(out, ref)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16
    direct = gpu_ctx.run_float16(s, h["input"], h["offset"], h["mask"], h["weight"], h["bias"])
    assert np.array_equal(direct.view(np.uint16), ref.astype(np.float16).view(np.uint16))


def test_zero_offsets_unit_mask_is_conv2d(gpu_ctx, dcn):
    import torch
    import torch.nn.functional as F

    s = dcn.DeformConvShape(1, 128, 20, 24, 64, 20, 24, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    d = rand_case(s, 21)
    d["weight"] *= 0.1
    d["offset"][:] = 0
    d["mask"][:] = 1
    h = f16_inputs(d)
    log("case: zero offsets == conv2d")
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    ref = F.conv2d(torch.tensor(h["input"].astype(np.float64)).reshape(1, 128, 20, 24),
                   torch.tensor(h["weight"].astype(np.float64)).reshape(64, 128, 3, 3),
                   torch.tensor(h["bias"].astype(np.float64)), padding=1).numpy().ravel()
    mx, mean = errors(out, ref)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16


def test_prepack_layouts_and_dcnfp16_file(gpu_ctx, dcn, c2):
    s, h, _ = c2
    log("case: prepack layouts + .dcnfp16")
    p1 = gpu_ctx.prepack(s, h["weight"], h["bias"], dcn.LAYOUT_OIHW)
    packed_w = dcn.pack_ic_k_oc(h["weight"], s)
    p2 = gpu_ctx.prepack(s, packed_w, h["bias"], dcn.LAYOUT_IC_K_OC)
    o1 = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], p1)
    o2 = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], p2)
    assert np.array_equal(o1.view(np.uint16), o2.view(np.uint16))
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "forward_1.dcnfp16")
        payload = packed_w.astype("<f2").tobytes() + h["bias"].astype("<f2").tobytes()
        assert len(payload) == dcn.lib().dcn_dcnfp16_bytes() == 147584
        with open(path, "wb") as f:
            f.write(payload)
        p3 = gpu_ctx.load_dcnfp16(path, "forward_1")
        o3 = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], p3)
        assert np.array_equal(o1.view(np.uint16), o3.view(np.uint16))
        bad = os.path.join(tmp, "backward_1.dcnfp16")
        with open(bad, "wb") as f:
            f.write(payload[:-2])
        with pytest.raises(dcn.DeformConvError) as e:
            gpu_ctx.load_dcnfp16(bad)
        assert e.value.status == dcn.COMMAND_FAILED
        assert "backward_1.dcnfp16 has 147582 bytes; expected 147584" in e.value.message


def test_exported_weight_sets_load_and_run(gpu_ctx, dcn, c2):
    from jasnamacos_amd import weights as W

    s, h, _ = c2
    log("case: exported weight sets")
    rng = np.random.default_rng(8)
    sets = {d: ((h["weight"].astype(np.float32) * rng.uniform(0.5, 1.5)).astype(np.float16).reshape(64, 128, 3, 3),
                h["bias"]) for d in W.DIRECTIONS}
    with tempfile.TemporaryDirectory() as tmp:
        W.export_weight_sets(tmp, sets)
        assert len(W.validate_weight_sets(tmp)) == 4
        loaded = gpu_ctx.load_weight_sets(tmp)
        for p in loaded:
            ref = gpu_ctx.prepack(s, sets[p.direction][0], sets[p.direction][1])
            a = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], p)
            b = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], ref)
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), p.direction


def test_count_mismatch_reports_name(gpu_ctx, dcn):
    s = dcn.DeformConvShape(*GENERAL_SHAPES[0])
    c = s.counts()
    with pytest.raises(dcn.DeformConvError) as e:
        gpu_ctx.run_float32(s, np.zeros(c["input"]), np.zeros(c["offset"] - 1), np.zeros(c["mask"]),
                            np.zeros(c["weight"]), np.zeros(c["bias"]))
    assert e.value.status == dcn.INVALID_ARRAY_COUNT
    assert e.value.message == f"offset has {c['offset'] - 1} elements; expected {c['offset']}"
    big = dataclasses.replace(s, groups=2, input_channels=4, output_channels=4, offset_groups=1)
    with pytest.raises(dcn.DeformConvError) as e:
        gpu_ctx.prepack(big, np.zeros(big.weight_count, np.float16), np.zeros(4, np.float16))
    assert e.value.status == dcn.INVALID_SHAPE


def test_nonfinite_flag(gpu_ctx, dcn):
    import torch

    # MetalNonFiniteFlagTests.swift:50-52
    def flagged(values):
        t = torch.tensor(np.array(values, np.float16).view(np.int16)).cuda()
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        gpu_ctx.flag_nonfinite_f16_dev(t, t.numel(), flag)
        torch.cuda.synchronize()
        return int(flag.item())

    log("case: non-finite flag")
    assert flagged([0, 1, -2, 0.5]) == 0
    assert flagged([0, np.inf, 1]) == 1
    assert flagged([0, np.nan, 1]) == 1
    big = np.zeros(1 << 20, np.float16)
    big[-1] = np.inf
    assert flagged(big) == 1
    t = torch.tensor(big.view(np.int16)).cuda()
    with pytest.raises(dcn.DeformConvError) as e:
        gpu_ctx.check_nonfinite_f16_dev(t, t.numel())
    assert e.value.status == dcn.NONFINITE_OUTPUT and e.value.is_recoverable_numerical_failure
    gpu_ctx.check_nonfinite_f16_dev(t, t.numel() - 1)  # finite prefix: no error


def test_fp16_overflow_is_flagged(gpu_ctx, dcn, c2):
    import torch

    s, h, _ = c2
    log("case: fp16 overflow")
    w = (h["weight"].astype(np.float32) * 7e4).astype(np.float16)
    packed = gpu_ctx.prepack(s, w, h["bias"])
    out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    assert not np.all(np.isfinite(out.astype(np.float32)))
    t = torch.tensor(out.view(np.int16)).cuda()
    with pytest.raises(dcn.DeformConvError) as e:
        gpu_ctx.check_nonfinite_f16_dev(t, t.numel())
    assert e.value.is_recoverable_numerical_failure


@pytest.mark.parametrize("dims", [(2, 16, 7, 24), (1, 128, 64, 64), (3, 8, 5, 13), (1, 32, 9, 8)],
                         ids=lambda t: "x".join(map(str, t)))
def test_pack_input_cb8_layout(gpu_ctx, dcn, dims):
    """The CB8 repack equals the padded channel-block transpose of the input, border
    included, bit for bit, over an output buffer that held other values (widths that are
    and are not multiples of 8, batches, odd heights)."""
    import torch

    b, c, h, w = dims
    s = dcn.DeformConvShape(b, c, h, w, 32, h, w, 3, 3, 1, 1, 1, 1, 1, 1, 1, c // 8)
    log("case: CB8 repack", dims)
    rng = np.random.default_rng(sum(dims))
    x = rng.integers(0, 1 << 16, b * c * h * w, dtype=np.uint16)
    xd = torch.tensor(x.view(np.int16)).cuda()
    cb8 = torch.full((gpu_ctx.cb8_count(s),), -1, dtype=torch.int16, device="cuda")
    gpu_ctx.pack_input_cb8_dev(s, xd, cb8)
    torch.cuda.synchronize()
    ref = np.zeros((b, c // 8, h + 4, w + 4, 8), np.uint16)
    ref[:, :, 2:h + 2, 2:w + 2] = x.reshape(b, c // 8, 8, h, w).transpose(0, 1, 3, 4, 2)
    got = cb8.cpu().numpy().view(np.uint16)
    assert got.size >= ref.size
    assert np.array_equal(got[:ref.size].reshape(ref.shape), ref)


def test_device_entry_points_and_graph_replay(gpu_ctx, dcn, c2):
    import torch

    s, h, _ = c2
    log("case: _dev entry points + hipGraph replay")
    x, o, m = (torch.tensor(h[k].view(np.int16)).cuda() for k in ("input", "offset", "mask"))
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    host = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
    gpu_ctx.reserve(s)
    gpu_ctx.forward_f16_prepacked_dev(s, x, o, m, packed, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), host.view(np.uint16))
    # CB8 repack equals the padded channel-block transpose of the input.
    cb8 = torch.empty(gpu_ctx.cb8_count(s), dtype=torch.int16, device="cuda")
    gpu_ctx.pack_input_cb8_dev(s, x, cb8)
    torch.cuda.synchronize()
    X = h["input"].view(np.uint16).reshape(1, 16, 8, 64, 64).transpose(0, 1, 3, 4, 2)
    ref = np.zeros((1, 16, 68, 68, 8), np.uint16)
    ref[:, :, 2:66, 2:66] = X
    assert np.array_equal(cb8.cpu().numpy().view(np.uint16).reshape(ref.shape), ref)
    out2 = torch.empty_like(out)
    gpu_ctx.forward_f16_prepacked_cb8_dev(s, cb8, o, m, packed, out2)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    # Graph capture of the stream-ordered call, replayed with eager work in between.
    stream = torch.cuda.Stream()
    graph_out = torch.zeros_like(out)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        gpu_ctx.forward_f16_prepacked_dev(s, x, o, m, packed, graph_out, stream=torch.cuda.current_stream())
    scratch = torch.empty_like(out)
    for i in range(3):
        graph_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out, out), i
        gpu_ctx.forward_f16_prepacked_dev(s, x, o, m, packed, scratch)  # eager work between replays
        torch.cuda.synchronize()


def test_reference_benchmark_gate(gpu_ctx, dcn):
    # benchmarkJasnaShape gates (MetalRunner.swift:345-354) on its own seeded inputs:
    # gather + GEMM vs direct FP16 <= 2e-3.
    d = dcn.reference_benchmark_inputs()
    s = d["shape"]
    log("case: reference benchmark gate")
    direct = gpu_ctx.run_float16(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"]).astype(np.float32)
    packed = gpu_ctx.prepack(s, d["weight"], d["bias"])
    for sampler in (0, 1):
        gpu_ctx.set_fused_config(0, 0, sampler)
        try:
            fused = gpu_ctx.run_float16_prepacked(s, d["input"], d["offset"], d["mask"], packed).astype(np.float32)
        finally:
            gpu_ctx.set_fused_config(0, 0, -1)
        assert np.abs(fused - direct).max() <= 2e-3, sampler
    log("  checksum (fused, reference inputs):", dcn.checksum(fused.astype(np.float16)))


def test_benchmark_jasna_shape_harness(gpu_ctx, dcn):
    # benchmarkJasnaShape (MetalRunner.swift:187-388): statistics per variant, the gate,
    # a checksum over the fused output; with a .dcnfp16 weight set the weights come from
    # the file and the result equals a run with the same weights prepacked directly.
    from jasnamacos_amd import weights as W

    log("case: benchmark harness")
    r = gpu_ctx.benchmark_jasna_shape(iterations=5)
    assert r.iterations == 5 and len(r.fused.samples) == 5
    for st in (r.baseline, r.gather, r.fused):
        assert 0 < st.minimum <= st.median <= st.maximum
    assert r.max_difference_from_baseline <= 2e-3 and np.isfinite(r.checksum)
    log(f"  baseline {r.baseline.median:.4f} ms, gather {r.gather.median:.4f} ms, fused {r.fused.median:.4f} ms, "
        f"checksum {r.checksum:.6f}")
    rng = np.random.default_rng(17)
    w = rng.uniform(-0.02, 0.02, (64, 128, 3, 3)).astype(np.float16)
    b = rng.uniform(-0.02, 0.02, 64).astype(np.float16)
    with tempfile.TemporaryDirectory() as tmp:
        W.export_weight_sets(tmp, {"backward_1": (w, b)})
        r2 = gpu_ctx.benchmark_jasna_shape(iterations=2, weight_set=os.path.join(tmp, "backward_1.dcnfp16"))
    d = dcn.reference_benchmark_inputs()
    packed = gpu_ctx.prepack(d["shape"], w, b)
    ref = gpu_ctx.run_float16_prepacked(d["shape"], d["input"], d["offset"], d["mask"], packed)
    assert r2.checksum == dcn.checksum(ref)


# ---- property tests over random shapes (Hypothesis) ---------------------------------

from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402


@st.composite
def _direct_cases(draw):
    groups = draw(st.sampled_from([1, 2]))
    og = draw(st.sampled_from([1, 2, 4]))
    unit = groups * og // np.gcd(groups, og)
    cin = int(unit * draw(st.integers(1, 3)))
    cout = groups * draw(st.integers(1, 3))
    kh, kw = draw(st.integers(1, 3)), draw(st.integers(1, 3))
    sh, sw, dh, dw = (draw(st.integers(1, 2)) for _ in range(4))
    ph, pw = draw(st.integers(0, 2)), draw(st.integers(0, 2))
    h, w = draw(st.integers(2, 9)), draw(st.integers(2, 9))
    ho = max(1, (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1)
    wo = max(1, (w + 2 * pw - dw * (kw - 1) - 1) // sw + 1)
    return (draw(st.integers(1, 2)), cin, h, w, cout, ho, wo, kh, kw, ph, pw, sh, sw, dh, dw, groups, og), \
        draw(st.integers(0, 2**31 - 1)), draw(st.sampled_from([0.5, 3.0, 12.0]))


@settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(_direct_cases())
def test_property_fp32_direct_bit_exact(gpu_ctx, dcn, oracle, case):
    dims, seed, scale = case
    s = dcn.DeformConvShape(*dims)
    d = rand_case(s, seed % 100000, offset_scale=scale)
    log("case: property fp32", dims, seed, scale)
    out = gpu_ctx.run_float32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    ref = oracle.forward_f32(s, d["input"], d["offset"], d["mask"], d["weight"], d["bias"])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@st.composite
def _fused_cases(draw):
    og = draw(st.sampled_from([1, 2, 3, 4, 8, 16]))
    cin = og * 8 * draw(st.integers(1, 2))
    cout = 32 * draw(st.integers(1, 4))
    kh, kw = draw(st.sampled_from([(3, 3), (3, 3), (1, 3), (3, 1), (1, 1)]))
    sh, sw, dh, dw = (draw(st.integers(1, 2)) for _ in range(4))
    ph, pw = kh // 2 * dh, kw // 2 * dw
    h, w = draw(st.integers(3, 20)), draw(st.integers(3, 40))
    ho = max(1, (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1)
    wo = max(1, (w + 2 * pw - dw * (kw - 1) - 1) // sw + 1)
    return (draw(st.integers(1, 3)), cin, h, w, cout, ho, wo, kh, kw, ph, pw, sh, sw, dh, dw, 1, og), \
        draw(st.integers(0, 2**31 - 1)), draw(st.sampled_from([1, 2, 3, 5, 6, 7])), draw(st.sampled_from([0, 1]))


@settings(max_examples=30, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(_fused_cases())
def test_property_fused_f16_tolerance(gpu_ctx, dcn, oracle, case):
    dims, seed, variant, sampler = case
    s = dcn.DeformConvShape(*dims)
    assert s.fused_supported
    d = rand_case(s, seed % 100000, offset_scale=4.0)
    d["weight"] *= 0.5
    h = f16_inputs(d)
    w = widen(h)
    log("case: property fused", dims, "variant", variant, "sampler", sampler)
    packed = gpu_ctx.prepack(s, h["weight"], h["bias"])
    gpu_ctx.set_fused_config(0, 0, sampler, variant)
    try:
        out = gpu_ctx.run_float16_prepacked(s, h["input"], h["offset"], h["mask"], packed)
    finally:
        gpu_ctx.set_fused_config(0, 0, -1, 0)
    ref = oracle.forward_f32_threads(s, w["input"], w["offset"], w["mask"], w["weight"], w["bias"])
    mx, mean = errors(out, ref)
    assert mx <= MAX_ABS_F16 and mean <= MEAN_ABS_F16, (mx, mean)
