"""libdcn host-side behaviour that needs no GPU: exported symbols, shape validation,
error taxonomy, the seeded generator, FP16 conversion, checksum, statistics and the
benchmark-configuration input generators."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def header_symbols() -> list[str]:
    text = (ROOT / "include" / "dcn" / "dcn.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dcn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(dcn):
    from jasnamacos_amd import _lib

    lib = dcn.lib()
    names = header_symbols()
    assert len(names) >= 40
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    assert lib.dcn_abi_version() == 1


def test_status_recoverability(dcn):
    # DeformConvCPUTests.swift:35-41: only the non-finite output is recoverable.
    assert dcn.DeformConvError(dcn.NONFINITE_OUTPUT, "overflow").is_recoverable_numerical_failure
    for st in (dcn.INVALID_SHAPE, dcn.INVALID_ARRAY_COUNT, dcn.DEVICE_UNAVAILABLE, dcn.KERNEL_MISSING,
               dcn.COMMAND_FAILED, dcn.INVALID_ARGUMENT):
        assert not dcn.DeformConvError(st).is_recoverable_numerical_failure


def test_status_strings(dcn):
    assert dcn.lib().dcn_status_string(1).decode() == "Invalid deformable-convolution shape"
    assert dcn.lib().dcn_status_string(99).decode() == "Unknown status"


@pytest.mark.parametrize("field,value", [
    ("batch", 0), ("input_channels", 0), ("output_height", 0), ("kernel_width", 0), ("groups", 0),
    ("offset_groups", 0), ("offset_groups", 3), ("groups", 3),
])
def test_shape_validation(dcn, field, value):
    import dataclasses

    good = dcn.JASNA_SHAPE
    good.validate()
    bad = dataclasses.replace(good, **{field: value})
    with pytest.raises(dcn.DeformConvError) as e:
        bad.validate()
    assert e.value.status == dcn.INVALID_SHAPE


def test_shape_counts(dcn):
    s = dcn.JASNA_SHAPE
    c = s.counts()
    # Benchmark sizes at 1x128x64x64 -> 64, 16 offset groups.
    assert c["input"] == 524288 and c["offset"] == 1179648 and c["mask"] == 589824
    assert c["weight"] == 73728 and c["output"] == 262144 and c["bias"] == 64
    assert s.flops == 603979776
    assert s.fused_supported
    import dataclasses
    assert not dataclasses.replace(s, groups=2).fused_supported
    assert not dataclasses.replace(s, offset_groups=32).fused_supported  # 4 channels per group
    assert not dataclasses.replace(s, output_channels=48).fused_supported


def test_splitmix64_published_vectors(dcn):
    # Reference outputs of splitmix64.c (Vigna), the generator SeededGenerator restates.
    g = dcn.SeededGenerator(1234567)
    assert [g.next() for _ in range(5)] == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                            4593380528125082431, 16408922859458223821]
    g = dcn.SeededGenerator(1477776061723855037)
    assert [g.next() for _ in range(3)] == [1985237415132408290, 2979275885539914483, 13511426838097143398]


def test_splitmix64_zero_seed(dcn):
    # DeformConv.swift:172: seed 0 starts from the golden-ratio constant.
    assert dcn.lib().dcn_splitmix64_seed(0) == 0x9E3779B97F4A7C15
    a, b = dcn.SeededGenerator(0), dcn.SeededGenerator(0x9E3779B97F4A7C15)
    assert [a.next() for _ in range(4)] == [b.next() for _ in range(4)]


def test_seeded_floats_range_and_uniformity(dcn):
    # Swift's Float.random(in: lo...hi): values r * 2^-24 * delta + lo with r in [0, 2^24].
    # No published Swift output exists in the reference, so only structure is pinned here.
    g = dcn.SeededGenerator(0xC0FFEE)
    v = g.floats(200000, -1.0, 1.0)
    assert v.min() >= -1.0 and v.max() <= 1.0
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1 / np.sqrt(3)) < 0.01
    u = dcn.SeededGenerator(5).floats(1000, 0.0, 1.0)
    assert np.all(np.abs(u * 2 ** 24 - np.round(u * 2 ** 24)) == 0)  # lattice of 2^-24
    # deterministic
    assert np.array_equal(dcn.SeededGenerator(7).floats(50, -3, 3), dcn.SeededGenerator(7).floats(50, -3, 3))


def test_f16_conversion_matches_numpy(dcn):
    lib = dcn.lib()
    bits = np.arange(65536, dtype=np.uint16)
    out = np.empty(65536, dtype=np.float32)
    lib.dcn_f16_to_f32_array(bits.ctypes.data_as(C.POINTER(C.c_uint16)), out.ctypes.data_as(C.POINTER(C.c_float)), 65536)
    ref = bits.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(out[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        (rng.standard_normal(100000) * 10.0 ** rng.integers(-9, 6, 100000)).astype(np.float32),
        out[fin],  # every finite binary16 value round-trips
        out[fin][:-1] + np.diff(out[fin]) / 2,  # and every midpoint ties to even
    ]).astype(np.float32)
    got = dcn.f32_to_f16(vals).view(np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))


def test_checksum_stride_257(dcn):
    # MetalRunner.swift:332-337: sum of values[0::257] in double.
    v = np.arange(1000, dtype=np.float32)
    assert dcn.checksum(v) == 0 + 257 + 514 + 771
    h = np.ones(600, dtype=np.float16)
    assert dcn.checksum(h) == 3.0


def test_statistics_known_answer(dcn):
    # BenchmarkStatisticsTests.swift:5-20
    s = dcn.BenchmarkStatistics.of([4, 1, 3, 2])
    assert s.samples == [1, 2, 3, 4]
    assert s.minimum == 1 and s.maximum == 4 and s.median == 2.5 and s.mean == 2.5
    assert abs(s.standard_deviation - np.sqrt(1.25)) < 1e-12
    assert abs(s.percentile10 - 1.3) < 1e-12 and abs(s.percentile90 - 3.7) < 1e-12
    assert dcn.BenchmarkStatistics.of([5]).median == 5
    # BenchmarkStatisticsTests.swift:17-20
    assert dcn.BenchmarkStatistics.of([]) is None
    assert dcn.BenchmarkStatistics.of([1, np.inf]) is None


@pytest.mark.parametrize("config", [1, 2, 3, 5])
def test_config_shapes(dcn, config):
    s = dcn.config_shape(config)
    assert (s.input_channels, s.output_channels, s.offset_groups, s.kernel_area) == (128, 64, 16, 9)
    assert s.batch == (16 if config == 3 else 1)
    assert (s.input_height, s.input_width) == ((180, 320) if config == 5 else (64, 64))


def _oob_fraction(shape, offset):
    s = shape
    off = offset.reshape(s.batch, s.offset_groups * s.kernel_area, 2, s.output_height, s.output_width)
    k = np.arange(s.kernel_area)
    ky, kx = (k // 3).reshape(1, -1, 1, 1), (k % 3).reshape(1, -1, 1, 1)
    oy = np.arange(s.output_height).reshape(1, 1, -1, 1)
    ox = np.arange(s.output_width).reshape(1, 1, 1, -1)
    y = (oy - 1 + np.tile(ky, (1, s.offset_groups, 1, 1)) + off[:, :, 0]).astype(np.float64)
    x = (ox - 1 + np.tile(kx, (1, s.offset_groups, 1, 1)) + off[:, :, 1]).astype(np.float64)
    inside = (y > -1) & (y < s.input_height) & (x > -1) & (x < s.input_width)
    return 1.0 - inside.mean()


def test_out_of_bounds_fraction(dcn):
    """deform_conv.out_of_bounds_fraction against this file's restatement (stride 1, pad 1)
    on C2's inputs, and against a per-sample count on a small shape with stride, dilation
    and padding 2, with points exactly on the -1 and H / W boundaries."""
    d = dcn.generate_config_inputs(2, 7)
    assert dcn.out_of_bounds_fraction(d["shape"], d["offset"]) == pytest.approx(_oob_fraction(d["shape"], d["offset"]))
    s = dcn.DeformConvShape(1, 8, 7, 9, 8, 4, 5, 3, 3, 2, 2, 2, 2, 2, 2, 1, 1)
    rng = np.random.default_rng(3)
    off = rng.uniform(-4, 4, (2 * 9, 4, 5))
    off[0, 0, 0] = -1.0 - (0 * 2 - 2 + 0)  # y exactly -1: outside
    off[1, 0, 0] = 0.0
    off[2, 0, 1] = 7.0 - (0 * 2 - 2 + 0)   # y exactly H: outside
    n_out = 0
    for k in range(9):
        for oy in range(4):
            for ox in range(5):
                y = oy * 2 - 2 + (k // 3) * 2 + off[2 * k, oy, ox]
                x = ox * 2 - 2 + (k % 3) * 2 + off[2 * k + 1, oy, ox]
                n_out += not (-1 < y < 7 and -1 < x < 9)
    assert dcn.out_of_bounds_fraction(s, off.reshape(-1)) == pytest.approx(n_out / (9 * 4 * 5))


def test_config_inputs_c2(dcn):
    d = dcn.generate_config_inputs(2, 1)
    d2 = dcn.generate_config_inputs(2, 1)
    assert all(np.array_equal(d[k], d2[k]) for k in ("input", "offset", "mask", "weight", "bias"))
    assert not np.array_equal(d["input"], dcn.generate_config_inputs(2, 2)["input"])
    x = d["input"]
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    bound = np.sqrt(6 / 1152)
    assert np.abs(d["weight"]).max() <= bound and np.abs(d["weight"]).max() > 0.99 * bound
    assert np.abs(d["bias"]).max() <= 0.1
    assert d["mask"].min() > 0 and d["mask"].max() < 1 and abs(d["mask"].mean() - 0.5) < 0.01
    off = d["offset"].reshape(288, 64, 64)
    # residue 10*tanh(N(0,1)) plus a flow of at most 6 px shared by the 144 points
    assert np.abs(off).max() < 16.0
    flow_y = off[0::2].mean(axis=0)  # flow + residue mean (std 6.3 / 12 = 0.53)
    residue = off[0::2] - flow_y
    assert 5.8 < residue.std() < 6.8  # std of 10 * tanh(N(0, 1)) is 6.28
    assert np.abs(flow_y).max() < 6.0 + 5 * 0.53
    blocks = flow_y.reshape(8, 8, 8, 8).mean(axis=(1, 3))  # 8x8-pixel means: noise 0.07
    assert np.abs(np.diff(blocks, axis=1)).max() < 12.0 * 8 / 9 / 7 * 8 + 0.5  # smooth flow
    frac = _oob_fraction(d["shape"], d["offset"])
    assert 0.02 < frac < 0.25


def test_config_inputs_c3_oob(dcn):
    d = dcn.generate_config_inputs(3, 3)
    frac = _oob_fraction(d["shape"], d["offset"])
    assert 0.03 < frac < 0.30, frac  # roughly 5-15%: the padding path is exercised


def test_config_inputs_c5_hard_masks(dcn):
    d = dcn.generate_config_inputs(5, 5)
    m16 = d["mask"].astype(np.float16)
    zeros, ones = np.mean(m16 == 0), np.mean(m16 == 1)
    assert 0.03 < zeros < 0.07 and 0.03 < ones < 0.07  # 10% of sites forced to sigmoid(+-20)
    frac = _oob_fraction(d["shape"], d["offset"])
    assert 0.08 < frac < 0.35, frac


def test_reference_benchmark_inputs_ranges(dcn):
    d = dcn.reference_benchmark_inputs()
    assert d["input"].dtype == np.float16
    assert np.abs(d["input"]).max() <= 1 and np.abs(d["offset"]).max() <= 0.25
    assert d["mask"].min() >= 0.25 and d["mask"].max() <= 0.75
    assert np.abs(d["weight"]).max() <= 0.02


def test_pack_ic_k_oc_matches_export_tool(dcn):
    # tools/export_deform_weights.py:47: transpose(weight.reshape(64,128,9), (1,2,0))
    s = dcn.JASNA_SHAPE
    w = np.arange(s.weight_count, dtype=np.float32)
    p = dcn.pack_ic_k_oc(w, s)
    assert p.shape == (128, 9, 64)
    assert p[5, 3, 7] == w[(7 * 128 + 5) * 9 + 3]


def test_create_without_device_reports_unavailable(dcn):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    with pytest.raises(dcn.DeformConvError) as e:
        dcn.HipDeformConv(0)
    assert e.value.status == dcn.DEVICE_UNAVAILABLE



def test_automatic_fused_config_per_workload(dcn):
    """The automatic kernel choice without a device: the narrow kernel (variant 5) up to
    1024 tiles of 32 pixels (C2), the tile kernel (variant 7) above that (C3, C5)."""
    assert dcn.config_shape(2).automatic_fused_config()["variant"] == 5
    assert dcn.config_shape(3).automatic_fused_config() == {"variant": 7, "mt": 16, "ks": 8, "sampler": 1}
    assert dcn.config_shape(5).automatic_fused_config()["variant"] == 7


@pytest.mark.parametrize("side", ["input_height", "input_width"])
@pytest.mark.parametrize("n,tile", [(32000, True), (32001, False), (40000, False)])
def test_tile_kernel_side_limit(dcn, side, n, tile):
    """The tile kernel carries clamped corner coordinates (-2 .. H, -2 .. W) as signed
    16-bit pairs: maps with a side above 32000 go to another kernel, those at the limit
    still take it. The strips have 16 channels (2 offset groups), more than 1024 tiles of
    32 pixels and 8-pixel output rows: otherwise the tile kernel's domain."""
    if side == "input_width":
        s = dcn.DeformConvShape(1, 16, 2, n, 32, 2, 20000, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    else:
        s = dcn.DeformConvShape(1, 16, n, 8, 32, 5000, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 2)
    cfg = s.automatic_fused_config()
    assert (cfg["variant"] == 7) == tile, cfg


def _tile_plan_rank(loc: int, n: int) -> int:
    """The rank (0 = heaviest) of the tile that band-local slot `loc` runs under the tile
    kernel's placement plan for a band of n tiles, 32 < n < 64 (tile_band_slot in
    dcn_kernels_tile.hip): locals l and l + 32 share a CU for l < n - 32, locals n - 32 ..
    31 run alone."""
    pairs = n - 32
    if loc >= 32:
        return n - 1 - (loc - 32)
    if loc >= pairs:
        return loc - pairs
    return (32 - pairs) + loc


@pytest.mark.parametrize("n", range(33, 64))
def test_tile_plan_slots_cover_every_tile_once(n):
    """Every band size the plan applies to: the slots take ranks 0 .. n-1 exactly once, the
    single-tile slots take the heaviest ranks, and each shared CU pairs the k-th heaviest of
    the rest with the k-th lightest."""
    ranks = [_tile_plan_rank(loc, n) for loc in range(n)]
    assert sorted(ranks) == list(range(n))
    pairs = n - 32
    alone = [ranks[loc] for loc in range(pairs, 32)]
    assert sorted(alone) == list(range(32 - pairs))
    for c in range(pairs):
        assert ranks[c] == 32 - pairs + c and ranks[c + 32] == n - 1 - c
