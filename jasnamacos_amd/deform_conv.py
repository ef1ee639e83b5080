"""Python mirror of the reference's deform-conv operator surface, over libdcn.

Reference surface (ken8303/jasnaMacOS, Sources/JasnaMetalPoC/):
  DeformConvShape / validate / counts     DeformConv.swift:3-42
  DeformConvError, isRecoverable...        DeformConv.swift:44-73
  SeededGenerator (SplitMix64), floats     DeformConv.swift:168-186
  MetalDeformConv.init / runFloat32        MetalRunner.swift:107-185
  benchmarkJasnaShape (inputs, packing)    MetalRunner.swift:187-388
  DeformConvWeightSet, loadDeformConvWeightSets   DeformConvWeights.swift:4-46
  BenchmarkStatistics                      BenchmarkStatistics.swift:3-44

Every compute call goes through the HIP library; nothing here computes a convolution.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from pathlib import Path
from typing import Optional

import numpy as np

from . import _lib

OK = 0
INVALID_SHAPE = 1
INVALID_ARRAY_COUNT = 2
DEVICE_UNAVAILABLE = 3
KERNEL_MISSING = 4
NONFINITE_OUTPUT = 5
COMMAND_FAILED = 6
INVALID_ARGUMENT = 7

LAYOUT_OIHW = 0
LAYOUT_IC_K_OC = 1

SAMPLER_EXACT = 0
SAMPLER_FAST = 1

VARIANT_AUTO = 0
VARIANT_REGISTER = 1
VARIANT_STAGED = 2
VARIANT_WINDOW = 3
VARIANT_WINDOW_SPLIT = 4
VARIANT_NARROW = 5
VARIANT_WINDOW_ASYNC = 6

DIRECTIONS = ("backward_1", "forward_1", "backward_2", "forward_2")


def lib() -> C.CDLL:
    return _lib.load()


class DeformConvError(Exception):
    """DeformConvError (DeformConv.swift:44-73) carried by a dcn_status."""

    def __init__(self, status: int, message: str = ""):
        self.status = int(status)
        self.message = message or lib().dcn_status_string(self.status).decode()
        super().__init__(f"[{self.status}] {self.message}")

    @property
    def is_recoverable_numerical_failure(self) -> bool:
        return bool(lib().dcn_status_is_recoverable(self.status))


@dataclasses.dataclass(frozen=True)
class DeformConvShape:
    """DeformConvShape (DeformConv.swift:3-20); output H/W are given, not derived."""

    batch: int
    input_channels: int
    input_height: int
    input_width: int
    output_channels: int
    output_height: int
    output_width: int
    kernel_height: int = 3
    kernel_width: int = 3
    pad_height: int = 1
    pad_width: int = 1
    stride_height: int = 1
    stride_width: int = 1
    dilation_height: int = 1
    dilation_width: int = 1
    groups: int = 1
    offset_groups: int = 1

    def to_c(self) -> _lib.DcnShape:
        return _lib.DcnShape(*[getattr(self, f.name) for f in dataclasses.fields(self)])

    @classmethod
    def from_c(cls, s: _lib.DcnShape) -> "DeformConvShape":
        return cls(*[getattr(s, name) for name, _ in _lib.DcnShape._fields_])

    def validate(self) -> None:
        st = lib().dcn_shape_validate(C.byref(self.to_c()))
        if st != OK:
            raise DeformConvError(st)

    def counts(self) -> dict:
        c = _lib.DcnCounts()
        st = lib().dcn_shape_counts(C.byref(self.to_c()), C.byref(c))
        if st != OK:
            raise DeformConvError(st)
        return {name: getattr(c, name) for name, _ in _lib.DcnCounts._fields_}

    @property
    def input_count(self) -> int:
        return self.counts()["input"]

    @property
    def output_count(self) -> int:
        return self.counts()["output"]

    @property
    def kernel_area(self) -> int:
        return self.kernel_height * self.kernel_width

    @property
    def offset_count(self) -> int:
        return self.counts()["offset"]

    @property
    def mask_count(self) -> int:
        return self.counts()["mask"]

    @property
    def weight_count(self) -> int:
        return self.counts()["weight"]

    @property
    def fused_supported(self) -> bool:
        return bool(lib().dcn_shape_fused_supported(C.byref(self.to_c())))

    def automatic_fused_config(self) -> dict:
        """The fused kernel an FP16 prepacked call on this shape runs when no override is
        set (dcn_get_fused_config with a null context; no device is touched)."""
        v, mt, ks, sm = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        st = lib().dcn_get_fused_config(None, C.byref(self.to_c()), C.byref(v), C.byref(mt), C.byref(ks),
                                        C.byref(sm))
        if st != OK:
            raise DeformConvError(st)
        return {"variant": v.value, "mt": mt.value, "ks": ks.value, "sampler": sm.value}

    @property
    def flops(self) -> int:
        """2 * B * Ho * Wo * Cout * (Cin/groups) * Kh * Kw (GEMM-equivalent)."""
        return (2 * self.batch * self.output_height * self.output_width * self.output_channels
                * (self.input_channels // self.groups) * self.kernel_area)


JASNA_SHAPE = DeformConvShape(1, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        return np.ascontiguousarray(a).view(np.uint16)
    if a.dtype == np.uint16:
        return np.ascontiguousarray(a)
    raise TypeError(f"expected float16 or uint16 array, got {a.dtype}")


def _bits16(a) -> np.ndarray:
    """16-bit patterns of a BF16 tensor (numpy has no BF16 type: uint16 arrays)."""
    a = np.asarray(a)
    if a.dtype != np.uint16:
        raise TypeError(f"expected BF16 bit patterns as a uint16 array, got {a.dtype}")
    return np.ascontiguousarray(a)


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round FP32 values to BF16 (nearest, ties to even) and return the bit patterns;
    NaN stays a quiet NaN."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_bits_to_f32(b) -> np.ndarray:
    """Widen BF16 bit patterns to FP32 exactly."""
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_lib.c_f32p)


def _hp(a: np.ndarray):
    return a.ctypes.data_as(_lib.c_u16p)


def _ptr(t) -> Optional[int]:
    """Device pointer of a torch tensor (or an int address)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class PackedWeights:
    """Handle of weights prepacked into the MFMA B-fragment layout (dcn_packed)."""

    def __init__(self, handle: int, shape: DeformConvShape, direction: str = ""):
        self.handle = C.c_void_p(handle)
        self.shape = shape
        self.direction = direction

    def free(self) -> None:
        if self.handle:
            lib().dcn_packed_free(self.handle)
            self.handle = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipDeformConv:
    """MetalDeformConv's role on MI355X: one libdcn context on one HIP device."""

    def __init__(self, device: int = 0):
        self._lib = lib()
        ctx = C.c_void_p()
        st = self._lib.dcn_create(C.byref(ctx), int(device))
        if st != OK:
            raise DeformConvError(st)
        self.ctx = ctx
        self.device = device

    def close(self) -> None:
        if self.ctx:
            self._lib.dcn_destroy(self.ctx)
            self.ctx = C.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, st: int) -> None:
        if st != OK:
            raise DeformConvError(st, self._lib.dcn_last_error(self.ctx).decode())

    @property
    def last_error(self) -> str:
        return self._lib.dcn_last_error(self.ctx).decode()

    # ---- host-pointer entry points -------------------------------------------------
    def run_float32(self, shape: DeformConvShape, input, offset, mask, weight, bias) -> np.ndarray:
        """runFloat32 (MetalRunner.swift:159-185): bit-identical to DeformConvCPU.run."""
        arrs = [_f32(a).ravel() for a in (input, offset, mask, weight, bias)]
        out = np.empty(shape.output_count, dtype=np.float32)
        args = []
        for a in arrs:
            args += [_fp(a), a.size]
        self._check(self._lib.dcn_forward_f32(self.ctx, C.byref(shape.to_c()), *args, _fp(out), out.size))
        return out

    def run_float16(self, shape: DeformConvShape, input, offset, mask, weight, bias) -> np.ndarray:
        """deform_conv2d_fp16 semantics (MetalShader.swift:126-174); float16 in/out."""
        arrs = [_u16(a).ravel() for a in (input, offset, mask, weight, bias)]
        out = np.empty(shape.output_count, dtype=np.uint16)
        args = []
        for a in arrs:
            args += [_hp(a), a.size]
        self._check(self._lib.dcn_forward_f16(self.ctx, C.byref(shape.to_c()), *args, _hp(out), out.size))
        return out.view(np.float16)

    def prepack(self, shape: DeformConvShape, weight, bias, layout: int = LAYOUT_OIHW) -> PackedWeights:
        w = _u16(weight).ravel()
        b = _u16(bias).ravel()
        handle = C.c_void_p()
        self._check(self._lib.dcn_prepack_f16(self.ctx, C.byref(shape.to_c()), _hp(w), w.size, int(layout),
                                              _hp(b), b.size, C.byref(handle)))
        return PackedWeights(handle.value, shape)

    def load_dcnfp16(self, path, direction: str = "") -> PackedWeights:
        """DeformConvWeightSet(direction:url:) + makeBuffers (DeformConvWeights.swift:11-36)."""
        handle = C.c_void_p()
        self._check(self._lib.dcn_load_dcnfp16(self.ctx, str(path).encode(), C.byref(handle)))
        return PackedWeights(handle.value, JASNA_SHAPE, direction)

    def load_weight_sets(self, directory) -> list[PackedWeights]:
        """loadDeformConvWeightSets (DeformConvWeights.swift:39-46)."""
        d = Path(directory)
        return [self.load_dcnfp16(d / f"{name}.dcnfp16", name) for name in DIRECTIONS]

    def run_float16_prepacked(self, shape: DeformConvShape, input, offset, mask,
                              packed: PackedWeights) -> np.ndarray:
        """Fused sampler + MFMA GEMM (replaces executeJasnaSIMDGroupGEMM)."""
        arrs = [_u16(a).ravel() for a in (input, offset, mask)]
        out = np.empty(shape.output_count, dtype=np.uint16)
        args = []
        for a in arrs:
            args += [_hp(a), a.size]
        self._check(self._lib.dcn_forward_f16_prepacked(self.ctx, C.byref(shape.to_c()), *args,
                                                        packed.handle, _hp(out), out.size))
        return out.view(np.float16)

    # ---- BF16 storage (no counterpart in the reference) ----------------------------
    def prepack_bf16(self, shape: DeformConvShape, weight, bias, layout: int = LAYOUT_OIHW) -> PackedWeights:
        """Weights and bias as BF16 bit patterns (uint16 arrays); packed for
        run_bfloat16_prepacked only."""
        w = _bits16(weight).ravel()
        b = _bits16(bias).ravel()
        handle = C.c_void_p()
        self._check(self._lib.dcn_prepack_bf16(self.ctx, C.byref(shape.to_c()), _hp(w), w.size, int(layout),
                                               _hp(b), b.size, C.byref(handle)))
        return PackedWeights(handle.value, shape)

    def run_bfloat16_prepacked(self, shape: DeformConvShape, input, offset, mask,
                               packed: PackedWeights) -> np.ndarray:
        """The fused sampler + MFMA GEMM over BF16 tensors (uint16 bit patterns in and
        out): FP32 bilinear in the reference's association, each sample rounded once to
        BF16, BF16 MFMA with FP32 accumulation, bf16(acc + bias)."""
        arrs = [_bits16(a).ravel() for a in (input, offset, mask)]
        out = np.empty(shape.output_count, dtype=np.uint16)
        args = []
        for a in arrs:
            args += [_hp(a), a.size]
        self._check(self._lib.dcn_forward_bf16_prepacked(self.ctx, C.byref(shape.to_c()), *args,
                                                         packed.handle, _hp(out), out.size))
        return out

    def prepack_bf16_dev(self, shape, w, b, layout: int = LAYOUT_OIHW, stream=None) -> PackedWeights:
        handle = C.c_void_p()
        self._check(self._lib.dcn_prepack_bf16_dev(self.ctx, C.byref(shape.to_c()), _ptr(w), int(layout), _ptr(b),
                                                   _stream(stream), C.byref(handle)))
        return PackedWeights(handle.value, shape)

    def forward_bf16_prepacked_dev(self, shape, x, off, msk, packed: PackedWeights, out, stream=None) -> None:
        self._check(self._lib.dcn_forward_bf16_prepacked_dev(self.ctx, C.byref(shape.to_c()), _ptr(x), _ptr(off),
                                                             _ptr(msk), packed.handle, _ptr(out), _stream(stream)))

    def forward_bf16_prepacked_cb8_dev(self, shape, cb8, off, msk, packed: PackedWeights, out, stream=None) -> None:
        self._check(self._lib.dcn_forward_bf16_prepacked_cb8_dev(self.ctx, C.byref(shape.to_c()), _ptr(cb8),
                                                                 _ptr(off), _ptr(msk), packed.handle, _ptr(out),
                                                                 _stream(stream)))

    # ---- device-pointer entry points (torch tensors as plumbing) ------------------
    def forward_f32_dev(self, shape, x, off, msk, w, b, out, stream=None) -> None:
        self._check(self._lib.dcn_forward_f32_dev(self.ctx, C.byref(shape.to_c()), _ptr(x), _ptr(off), _ptr(msk),
                                                  _ptr(w), _ptr(b), _ptr(out), _stream(stream)))

    def forward_f16_dev(self, shape, x, off, msk, w, b, out, stream=None) -> None:
        self._check(self._lib.dcn_forward_f16_dev(self.ctx, C.byref(shape.to_c()), _ptr(x), _ptr(off), _ptr(msk),
                                                  _ptr(w), _ptr(b), _ptr(out), _stream(stream)))

    def prepack_dev(self, shape, w, b, layout: int = LAYOUT_OIHW, stream=None) -> PackedWeights:
        handle = C.c_void_p()
        self._check(self._lib.dcn_prepack_f16_dev(self.ctx, C.byref(shape.to_c()), _ptr(w), int(layout), _ptr(b),
                                                  _stream(stream), C.byref(handle)))
        return PackedWeights(handle.value, shape)

    def forward_f16_prepacked_dev(self, shape, x, off, msk, packed: PackedWeights, out, stream=None) -> None:
        self._check(self._lib.dcn_forward_f16_prepacked_dev(self.ctx, C.byref(shape.to_c()), _ptr(x), _ptr(off),
                                                            _ptr(msk), packed.handle, _ptr(out), _stream(stream)))

    def cb8_count(self, shape) -> int:
        return int(self._lib.dcn_cb8_count(C.byref(shape.to_c())))

    def pack_input_cb8_dev(self, shape, x, cb8, stream=None) -> None:
        self._check(self._lib.dcn_pack_input_cb8_dev(self.ctx, C.byref(shape.to_c()), _ptr(x), _ptr(cb8),
                                                     _stream(stream)))

    def forward_f16_prepacked_cb8_dev(self, shape, cb8, off, msk, packed: PackedWeights, out, stream=None) -> None:
        self._check(self._lib.dcn_forward_f16_prepacked_cb8_dev(self.ctx, C.byref(shape.to_c()), _ptr(cb8),
                                                                _ptr(off), _ptr(msk), packed.handle, _ptr(out),
                                                                _stream(stream)))

    def forward_f16_prepacked_noalloc_dev(self, shape, x, off, msk, packed: PackedWeights, out, stream=None) -> None:
        """forward_f16_prepacked_dev without any device allocation: the input's padded
        channel-block copy goes to the library's per-device scratch array (at most
        DCN_NOALLOC_SCRATCH_BYTES), shared by every call on the device."""
        self._check(self._lib.dcn_forward_f16_prepacked_noalloc_dev(self.ctx, C.byref(shape.to_c()), _ptr(x),
                                                                    _ptr(off), _ptr(msk), packed.handle, _ptr(out),
                                                                    _stream(stream)))

    def launch_floor_dev(self, workgroups: int, threads: int, lds_bytes: int = 0, stream=None) -> None:
        """An empty kernel of this launch shape (dcn_launch_floor_dev): the dispatch floor."""
        self._check(self._lib.dcn_launch_floor_dev(self.ctx, int(workgroups), int(threads), int(lds_bytes),
                                                   _stream(stream)))

    def set_tile_clock_dev(self, clock, count: int | None = None) -> None:
        """Per-workgroup clock stamps of the tile kernel (dcn_set_tile_clock_dev): `clock`
        is a device buffer of uint64 (an int64 tensor; count defaults to its numel), or
        None to turn the stamps off."""
        if clock is None:
            self._check(self._lib.dcn_set_tile_clock_dev(self.ctx, None, 0))
            return
        n = int(clock.numel()) if count is None else int(count)
        self._check(self._lib.dcn_set_tile_clock_dev(self.ctx, _ptr(clock), n))

    def im2col_f16_dev(self, shape, x, off, msk, columns, stream=None) -> None:
        self._check(self._lib.dcn_im2col_f16_dev(self.ctx, C.byref(shape.to_c()), _ptr(x), _ptr(off), _ptr(msk),
                                                 _ptr(columns), _stream(stream)))

    def flag_nonfinite_f16_dev(self, values, count: int, flag, stream=None) -> None:
        self._check(self._lib.dcn_flag_nonfinite_f16_dev(self.ctx, _ptr(values), int(count), _ptr(flag),
                                                         _stream(stream)))

    def check_nonfinite_f16_dev(self, values, count: int, stream=None) -> None:
        """Raises DeformConvError(NONFINITE_OUTPUT) (recoverable) if any value is NaN/Inf."""
        self._check(self._lib.dcn_check_nonfinite_f16_dev(self.ctx, _ptr(values), int(count), _stream(stream)))

    def reserve(self, shape) -> None:
        self._check(self._lib.dcn_reserve(self.ctx, C.byref(shape.to_c())))

    def set_fused_config(self, mt: int = 0, ks: int = 0, sampler: int = -1, variant: int = 0) -> None:
        """Pin the fused kernel's configuration (0 / -1 = automatic)."""
        self._check(self._lib.dcn_set_fused_config(self.ctx, int(variant), int(mt), int(ks), int(sampler)))

    def get_fused_config(self, shape) -> dict:
        v, mt, ks, sm = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        self._check(self._lib.dcn_get_fused_config(self.ctx, C.byref(shape.to_c()), C.byref(v), C.byref(mt),
                                                   C.byref(ks), C.byref(sm)))
        return {"variant": v.value, "mt": mt.value, "ks": ks.value, "sampler": sm.value}

    # ---- benchmark harness --------------------------------------------------------------

    def benchmark_jasna_shape(self, iterations: int = 20, weight_set=None, stream=None) -> "BenchmarkResult":
        """benchmarkJasnaShape (MetalRunner.swift:187-388) on this device.

        Seeded inputs of the reference (SeededGenerator(0x4A41534E41): input, offset, mask,
        then weight and bias unless `weight_set`, a .dcnfp16 path, supplies them), FP16
        device buffers, 2 warm-up calls then `iterations` timed calls per variant, each timed
        with HIP events around one call: the direct FP16 kernel (the baseline), the
        reference-arithmetic gather (im2col) alone, and the fused prepacked path. Checksum
        over the fused output (stride 257) and the reference's gate: the fused result within
        2e-3 of the baseline, else DeformConvError(COMMAND_FAILED)."""
        import torch

        from . import weights as _weights

        d = reference_benchmark_inputs()
        shape = d["shape"]
        w16, b16 = d["weight"], d["bias"]
        if weight_set is not None:
            packed_w, bias = _weights.unpack_weight_set(_weights.read_weight_set(weight_set))
            w16 = np.ascontiguousarray(np.transpose(packed_w, (2, 0, 1))).reshape(-1).astype(np.float16)
            b16 = np.asarray(bias, np.float16)
        dev = lambda a: torch.from_numpy(np.array(a, np.float16).view(np.int16)).cuda()  # noqa: E731 (a writable copy)
        x, off, msk, w, b = (dev(a) for a in (d["input"], d["offset"], d["mask"], w16, b16))
        base_out = torch.empty(shape.output_count, dtype=torch.int16, device="cuda")
        fused_out = torch.empty_like(base_out)
        cols = torch.empty(shape.output_height * shape.output_width * shape.input_channels * shape.kernel_area,
                           dtype=torch.int16, device="cuda")
        packed = self.prepack_dev(shape, w, b)
        self.reserve(shape)
        st = stream or torch.cuda.current_stream()
        variants = {
            "baseline": lambda: self.forward_f16_dev(shape, x, off, msk, w, b, base_out, stream=st),
            "gather": lambda: self.im2col_f16_dev(shape, x, off, msk, cols, stream=st),
            "fused": lambda: self.forward_f16_prepacked_dev(shape, x, off, msk, packed, fused_out, stream=st),
        }
        stats = {}
        for name, call in variants.items():
            for _ in range(2):
                call()
            samples = []
            for _ in range(max(iterations, 1)):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(st)
                call()
                e1.record(st)
                e1.synchronize()
                samples.append(e0.elapsed_time(e1))
            stats[name] = BenchmarkStatistics.of(samples)
            if stats[name] is None:
                raise DeformConvError(COMMAND_FAILED, "invalid DCNv2 benchmark samples")
        torch.cuda.synchronize()
        packed.free()
        base = base_out.cpu().numpy().view(np.float16).astype(np.float32)
        fused = fused_out.cpu().numpy().view(np.float16)
        max_diff = float(np.abs(fused.astype(np.float32) - base).max())
        if max_diff > 0.002:
            raise DeformConvError(COMMAND_FAILED, f"fused FP16 result differs from baseline by {max_diff}")
        return BenchmarkResult(baseline=stats["baseline"], gather=stats["gather"], fused=stats["fused"],
                               checksum=checksum(fused), max_difference_from_baseline=max_diff,
                               iterations=max(iterations, 1))

    # ---- propagation body ------------------------------------------------------------

    def offset_transform_f16(self, plane: int, raw, flow1, flow2):
        """runDCNOffsetTransform (MetalRunner.swift:469-508): FP16 arrays in, (offset, mask) out."""
        raw, flow1, flow2 = _u16(raw), _u16(flow1), _u16(flow2)
        off = np.empty(288 * plane, np.uint16)
        msk = np.empty(144 * plane, np.uint16)
        self._check(self._lib.dcn_offset_transform_f16(self.ctx, int(plane), _hp(raw), raw.size, _hp(flow1),
                                                       flow1.size, _hp(flow2), flow2.size, _hp(off), off.size,
                                                       _hp(msk), msk.size))
        return off.view(np.float16), msk.view(np.float16)

    def offset_transform_f16_dev(self, plane: int, raw, flow1, flow2, offset, mask, stream=None) -> None:
        self._check(self._lib.dcn_offset_transform_f16_dev(self.ctx, int(plane), _ptr(raw), _ptr(flow1),
                                                           _ptr(flow2), _ptr(offset), _ptr(mask), _stream(stream)))

    def temporal_prepare_f16(self, width: int, height: int, feat_prop, feat_current, feat_n2, flow1,
                             prev_flow, has_second_order: bool) -> dict:
        """runTemporalPreparation (MetalRunner.swift:510-582): conditions, deform_input, flow2."""
        a = [_u16(x) for x in (feat_prop, feat_current, feat_n2, flow1, prev_flow)]
        plane = width * height
        cond = np.empty(196 * plane, np.uint16)
        dinp = np.empty(128 * plane, np.uint16)
        flow2 = np.empty(2 * plane, np.uint16)
        args = []
        for x in a:
            args += [_hp(x), x.size]
        self._check(self._lib.dcn_temporal_prepare_f16(self.ctx, int(width), int(height), *args,
                                                       int(bool(has_second_order)), _hp(cond), cond.size,
                                                       _hp(dinp), dinp.size, _hp(flow2), flow2.size))
        return {"conditions": cond.view(np.float16), "deform_input": dinp.view(np.float16),
                "flow2": flow2.view(np.float16)}

    def temporal_prepare_f16_dev(self, width, height, feat_prop, feat_current, feat_n2, flow1, prev_flow,
                                 has_second_order, flow2, conditions, conditions_layout, deform_input,
                                 deform_input_layout, stream=None) -> None:
        self._check(self._lib.dcn_temporal_prepare_f16_dev(
            self.ctx, int(width), int(height), _ptr(feat_prop), _ptr(feat_current), _ptr(feat_n2), _ptr(flow1),
            _ptr(prev_flow), int(bool(has_second_order)), _ptr(flow2), _ptr(conditions), int(conditions_layout),
            _ptr(deform_input), int(deform_input_layout), _stream(stream)))

    def assemble_backbone_f16_dev(self, width, height, sources, out, layout=0, stream=None) -> None:
        arr = (C.c_void_p * len(sources))(*[_ptr(x) for x in sources])
        self._check(self._lib.dcn_assemble_backbone_f16_dev(self.ctx, int(width), int(height), arr, len(sources),
                                                            _ptr(out), int(layout), _stream(stream)))

    def add_residual_f16_dev(self, count, aligned, backbone, out, stream=None) -> None:
        self._check(self._lib.dcn_add_residual_f16_dev(self.ctx, int(count), _ptr(aligned), _ptr(backbone),
                                                       _ptr(out), _stream(stream)))

    def cb8_to_nchw_f16_dev(self, channels, height, width, cb8, out, stream=None) -> None:
        self._check(self._lib.dcn_cb8_to_nchw_f16_dev(self.ctx, int(channels), int(height), int(width), _ptr(cb8),
                                                      _ptr(out), _stream(stream)))

    def conv3x3(self, cin, cout, height, width, weight, bias, stream=None) -> "Conv3x3":
        handle = C.c_void_p()
        self._check(self._lib.dcn_conv3x3_create_dev(self.ctx, int(cin), int(cout), int(height), int(width),
                                                     _ptr(weight), _ptr(bias), _stream(stream), C.byref(handle)))
        return Conv3x3(self, handle.value, cin, cout, height, width)

    def body(self, height, width, weights: dict, branch: int = 0, blocks: int = 5, stream=None,
             tiles: int = 1) -> "PropagationBody":
        """weights: device tensors "offset_w{0..3}", "offset_b{0..3}", "dcn_w", "dcn_b",
        "backbone_w{0..2*blocks}", "backbone_b{0..2*blocks}" (OIHW FP16). tiles > 1: every
        step tensor holds that many independent tiles, [tiles][C][H][W]."""
        w = _body_weights(weights, blocks)
        handle = C.c_void_p()
        self._check(self._lib.dcn_body_create_tiles(self.ctx, int(height), int(width), int(branch), int(blocks),
                                                    int(tiles), C.byref(w), _stream(stream), C.byref(handle)))
        return PropagationBody(self, handle.value, height, width, branch, blocks)

    def bicubic_quarter_f16_dev(self, channels, height, width, src, out, stream=None) -> None:
        """jasna_bicubic_downsample_quarter_fp16: [c][h][w] -> [c][h/4][w/4] (h, w multiples of 4)."""
        self._check(self._lib.dcn_bicubic_quarter_f16_dev(self.ctx, int(channels), int(height), int(width),
                                                          _ptr(src), _ptr(out), _stream(stream)))

    def spynet_pyramid_f16_dev(self, height, width, frame, out, stream=None) -> None:
        """The six normalised SPyNet levels of one RGB frame, coarsest first, concatenated."""
        self._check(self._lib.dcn_spynet_pyramid_f16_dev(self.ctx, int(height), int(width), _ptr(frame), _ptr(out),
                                                         _stream(stream)))

    def spynet(self, height, width, weights, max_frames: int = 2, stream=None) -> "SpyNet":
        """weights: device tensors "w{level}_{layer}" and "b{level}_{layer}" (OIHW FP16),
        level 0..5 coarsest first, layer 0..4 (8->32->64->32->16->2, 7x7); max_frames sizes
        clip_flows_dev (2: pairs only)."""
        w = _lib.DcnSpynetWeights()
        for level in range(_lib.SPYNET_LEVELS):
            for layer in range(_lib.SPYNET_LAYERS):
                w.weight[level][layer] = _ptr(weights[f"w{level}_{layer}"])
                w.bias[level][layer] = _ptr(weights[f"b{level}_{layer}"])
        handle = C.c_void_p()
        self._check(self._lib.dcn_spynet_create(self.ctx, int(height), int(width), int(max_frames), C.byref(w),
                                                _stream(stream), C.byref(handle)))
        return SpyNet(self, handle.value, height, width, max_frames)

    def clip(self, height, width, frames, weights, blocks: int = 5, stream=None, tiles: int = 1) -> "PropagationClip":
        """The four propagation branches over `frames` frames; weights: four body weight dicts
        (backward_1, forward_1, backward_2, forward_2), as for body(). tiles > 1: spatial
        [T][tiles][64][H][W], flows [T-1][tiles][2][H][W], propagated [4][T][tiles][64][H][W]."""
        if len(weights) != 4:
            raise DeformConvError(INVALID_ARGUMENT, "a clip needs four branch weight sets")
        ws = (_lib.DcnBodyWeights * 4)(*[_body_weights(w, blocks) for w in weights])
        handle = C.c_void_p()
        self._check(self._lib.dcn_clip_create_tiles(self.ctx, int(height), int(width), int(frames), int(blocks),
                                                    int(tiles), ws, _stream(stream), C.byref(handle)))
        return PropagationClip(self, handle.value, height, width, frames, blocks)


TENSOR_NCHW = 0
TENSOR_CB8 = 1


def cb8_tensor_count(channels: int, height: int, width: int) -> int:
    return int(lib().dcn_cb8_tensor_count(int(channels), int(height), int(width)))


class Conv3x3:
    """A 3x3 body convolution with its weights packed into MFMA fragments (dcn_conv)."""

    def __init__(self, ctx: HipDeformConv, handle: int, cin, cout, height, width):
        self.ctx, self.handle = ctx, C.c_void_p(handle)
        self.cin, self.cout, self.height, self.width = cin, cout, height, width

    def run_dev(self, x_cb8, out, out_layout=TENSOR_NCHW, activation=0, slope=0.1, res1=None,
                res1_layout=TENSOR_NCHW, res2=None, res2_layout=TENSOR_NCHW, stream=None) -> None:
        self.ctx._check(self.ctx._lib.dcn_conv3x3_f16_dev(self.ctx.ctx, self.handle, _ptr(x_cb8), int(activation),
                                                          float(slope), _ptr(res1), int(res1_layout), _ptr(res2),
                                                          int(res2_layout), _ptr(out), int(out_layout),
                                                          _stream(stream)))

    def run_offsets_dev(self, x_cb8, flow1, flow2, offset, mask, stream=None) -> None:
        """The 432-channel conv_offset layer with the DCN offset transform in its epilogue:
        offset = half(10 tanh(half(conv + b)) + flow), mask = half(sigmoid(half(conv + b)))."""
        self.ctx._check(self.ctx._lib.dcn_conv3x3_offsets_f16_dev(
            self.ctx.ctx, self.handle, _ptr(x_cb8), _ptr(flow1), _ptr(flow2), _ptr(offset), _ptr(mask),
            _stream(stream)))

    def run_pair_dev(self, second: "Conv3x3", x_cb8, out, out_layout=TENSOR_NCHW, activation1=2,
                     activation2=0, slope=0.1, res1=None, res1_layout=TENSOR_NCHW, res2=None,
                     res2_layout=TENSOR_NCHW, stream=None) -> None:
        """This conv then `second` in one launch (both 64 -> 64): the intermediate
        half(act1(conv(x) + b)) stays on chip; equal to two run_dev calls bit for bit."""
        self.ctx._check(self.ctx._lib.dcn_conv3x3_pair_f16_dev(
            self.ctx.ctx, self.handle, second.handle, _ptr(x_cb8), int(activation1), int(activation2),
            float(slope), _ptr(res1), int(res1_layout), _ptr(res2), int(res2_layout), _ptr(out),
            int(out_layout), _stream(stream)))

    def free(self) -> None:
        if self.handle:
            self.ctx._lib.dcn_conv3x3_free(self.handle)
            self.handle = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class BodyGraph:
    """An executable hipGraph of one body step (dcn_graph)."""

    def __init__(self, ctx: HipDeformConv, handle: int):
        self.ctx, self.handle = ctx, C.c_void_p(handle)

    def launch(self, stream=None) -> None:
        self.ctx._check(self.ctx._lib.dcn_graph_launch(self.handle, _stream(stream)))

    def free(self) -> None:
        if self.handle:
            self.ctx._lib.dcn_graph_destroy(self.handle)
            self.handle = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PropagationBody:
    """One BasicVSR++ propagation step for one branch (dcn_body)."""

    def __init__(self, ctx: HipDeformConv, handle: int, height, width, branch, blocks):
        self.ctx, self.handle = ctx, C.c_void_p(handle)
        self.height, self.width, self.branch, self.blocks = height, width, branch, blocks

    def _args(self, feat_current, flow1, prev_flow, feat_prop, feat_n2, prefix, has_second_order, flow2_out,
              feat_prop_out):
        pre = None
        if prefix:
            pre = (C.c_void_p * len(prefix))(*[_ptr(x) for x in prefix])
        return (_ptr(feat_current), _ptr(flow1), _ptr(prev_flow), _ptr(feat_prop), _ptr(feat_n2), pre,
                int(bool(has_second_order)), _ptr(flow2_out), _ptr(feat_prop_out))

    def step_dev(self, feat_current, flow1, prev_flow, feat_prop, feat_n2, flow2_out, feat_prop_out,
                 has_second_order=True, prefix=None, stream=None) -> None:
        self.ctx._check(self.ctx._lib.dcn_body_step_dev(
            self.handle, *self._args(feat_current, flow1, prev_flow, feat_prop, feat_n2, prefix, has_second_order,
                                     flow2_out, feat_prop_out), _stream(stream)))

    def initial_step_dev(self, feat_current, feat_prop_out, prefix=None, stream=None) -> None:
        """A branch's first step: backbone on [feat_current, prefix..., 0], no alignment."""
        pre = None
        if prefix:
            pre = (C.c_void_p * len(prefix))(*[_ptr(x) for x in prefix])
        self.ctx._check(self.ctx._lib.dcn_body_initial_step_dev(self.handle, _ptr(feat_current), pre,
                                                                _ptr(feat_prop_out), _stream(stream)))

    def step_cb8_dev(self, feat_current, flow1, prev_flow, feat_prop_cb8, feat_n2_cb8, flow2_out, feat_prop_out,
                     feat_prop_out_cb8, has_second_order=True, prefix=None, stream=None) -> None:
        """dcn_body_step_cb8_dev: feat_prop / feat_n2 as 64-channel CB8 tensors, the output
        in NCHW and in CB8 (single-tile bodies)."""
        self.ctx._check(self.ctx._lib.dcn_body_step_cb8_dev(
            self.handle, *self._args(feat_current, flow1, prev_flow, feat_prop_cb8, feat_n2_cb8, prefix,
                                     has_second_order, flow2_out, feat_prop_out), _ptr(feat_prop_out_cb8),
            _stream(stream)))

    def initial_step_cb8_dev(self, feat_current, feat_prop_out, feat_prop_out_cb8, prefix=None, stream=None) -> None:
        pre = None
        if prefix:
            pre = (C.c_void_p * len(prefix))(*[_ptr(x) for x in prefix])
        self.ctx._check(self.ctx._lib.dcn_body_initial_step_cb8_dev(
            self.handle, _ptr(feat_current), pre, _ptr(feat_prop_out), _ptr(feat_prop_out_cb8), _stream(stream)))

    def capture_cb8(self, feat_current, flow1, prev_flow, feat_prop_cb8, feat_n2_cb8, flow2_out, feat_prop_out,
                    feat_prop_out_cb8, has_second_order=True, prefix=None) -> BodyGraph:
        handle = C.c_void_p()
        self.ctx._check(self.ctx._lib.dcn_body_capture_cb8(
            self.handle, *self._args(feat_current, flow1, prev_flow, feat_prop_cb8, feat_n2_cb8, prefix,
                                     has_second_order, flow2_out, feat_prop_out), _ptr(feat_prop_out_cb8),
            C.byref(handle)))
        return BodyGraph(self.ctx, handle.value)

    def capture(self, feat_current, flow1, prev_flow, feat_prop, feat_n2, flow2_out, feat_prop_out,
                has_second_order=True, prefix=None) -> BodyGraph:
        handle = C.c_void_p()
        self.ctx._check(self.ctx._lib.dcn_body_capture(
            self.handle, *self._args(feat_current, flow1, prev_flow, feat_prop, feat_n2, prefix, has_second_order,
                                     flow2_out, feat_prop_out), C.byref(handle)))
        return BodyGraph(self.ctx, handle.value)

    def free(self) -> None:
        if self.handle:
            self.ctx._lib.dcn_body_destroy(self.handle)
            self.handle = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _body_weights(weights: dict, blocks: int) -> "_lib.DcnBodyWeights":
    w = _lib.DcnBodyWeights()
    for i in range(4):
        w.offset_weight[i] = _ptr(weights[f"offset_w{i}"])
        w.offset_bias[i] = _ptr(weights[f"offset_b{i}"])
    w.dcn_weight = _ptr(weights["dcn_w"])
    w.dcn_bias = _ptr(weights["dcn_b"])
    for i in range(1 + 2 * blocks):
        w.backbone_weight[i] = _ptr(weights[f"backbone_w{i}"])
        w.backbone_bias[i] = _ptr(weights[f"backbone_b{i}"])
    return w


class SpyNet:
    """SPyNet flow estimation (dcn_spynet): RGB frames [3][H][W] in, flows [n][2][H][W] out."""

    def __init__(self, ctx: HipDeformConv, handle: int, height, width, max_frames=2):
        self.ctx, self.handle = ctx, C.c_void_p(handle)
        self.height, self.width, self.max_frames = height, width, max_frames

    def flow_dev(self, reference, support, flow, both_directions: bool = True, stream=None) -> None:
        """flow[0] = spynet(reference, support); flow[1] = spynet(support, reference) when
        both_directions (verifySPyNetPair's backward and forward, SPyNetPairProbe.swift)."""
        self.ctx._check(self.ctx._lib.dcn_spynet_flow_dev(self.handle, _ptr(reference), _ptr(support),
                                                          int(bool(both_directions)), _ptr(flow),
                                                          _stream(stream)))

    def clip_flows_dev(self, frames, count: int, flows, stream=None) -> None:
        """frames [count][3][H][W] -> flows [2][count-1][2][H][W]: [0][t] = spynet(t, t+1)
        (backward), [1][t] = spynet(t+1, t) (forward) (FusedSPyNetClipGraph.swift)."""
        self.ctx._check(self.ctx._lib.dcn_spynet_clip_flows_dev(self.handle, _ptr(frames), int(count), _ptr(flows),
                                                                _stream(stream)))

    def free(self) -> None:
        if self.handle:
            self.ctx._lib.dcn_spynet_destroy(self.handle)
            self.handle = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PropagationClip:
    """Four propagation branches over a clip (dcn_clip): the per-frame spatial features
    [frames][64][H][W] and both directions' flows [frames-1][2][H][W] in, every branch's
    propagated feature [4][frames][64][H][W] out (verifyFusedFourPassRecurrence,
    FusedFourPassRecurrenceProbe.swift:493-664, without the flow and reconstruction nets)."""

    def __init__(self, ctx: HipDeformConv, handle: int, height, width, frames, blocks):
        self.ctx, self.handle = ctx, C.c_void_p(handle)
        self.height, self.width, self.frames, self.blocks = height, width, frames, blocks

    def run_dev(self, spatial, backward_flows, forward_flows, propagated, max_frames_per_chunk: int = 0,
                stream=None) -> None:
        self.ctx._check(self.ctx._lib.dcn_clip_run_dev(self.handle, _ptr(spatial), _ptr(backward_flows),
                                                       _ptr(forward_flows), _ptr(propagated),
                                                       int(max_frames_per_chunk), _stream(stream)))

    def run_with_fallback_dev(self, spatial, backward_flows, forward_flows, propagated, stream=None,
                              report=None) -> int:
        """dcn_clip_run_with_fallback_dev: the whole recovery ladder (see
        propagate_with_fallback) in the library; returns 0, the chunk size,
        RECOVERED_TRIPLETS or RECOVERED_PASSTHROUGH. report(msg) receives the progress
        messages."""
        recovered = C.c_int()
        cb = _lib.ReportFn(lambda msg, _user: report(msg.decode()) if report else None)
        self.ctx._check(self.ctx._lib.dcn_clip_run_with_fallback_dev(
            self.handle, _ptr(spatial), _ptr(backward_flows), _ptr(forward_flows), _ptr(propagated),
            _stream(stream), cb, None, C.byref(recovered)))
        return recovered.value

    def capture(self, spatial, backward_flows, forward_flows, propagated, max_frames_per_chunk: int = 0) -> BodyGraph:
        handle = C.c_void_p()
        self.ctx._check(self.ctx._lib.dcn_clip_capture(self.handle, _ptr(spatial), _ptr(backward_flows),
                                                       _ptr(forward_flows), _ptr(propagated),
                                                       int(max_frames_per_chunk), C.byref(handle)))
        return BodyGraph(self.ctx, handle.value)

    def free(self) -> None:
        if self.handle:
            self.ctx._lib.dcn_clip_destroy(self.handle)
            self.handle = C.c_void_p(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


RECOVERED_TRIPLETS = -1  # DCN_CLIP_RECOVERED_TRIPLETS
RECOVERED_PASSTHROUGH = -2  # DCN_CLIP_RECOVERED_PASSTHROUGH


def propagate_with_fallback(run, frame_count: int, report=None, *, run_triplets, input_is_finite,
                            pass_through) -> int:
    """The recoverable-error ladder of restoreTileWithFallback
    (SideBySideRestoration.swift:1065-1136) over caller-supplied rungs:

    1. run(0) propagates the whole clip (returns 0);
    2. on the recoverable nonFiniteOutput, run(n) for recurrence chunks n = 10, 5, 3, those
       below frame_count (returns n);
    3. run_triplets() runs every frame alone as the zero-motion clip [f, f, f] and keeps
       the middle output (restoreTileFramesIndependently, :1140-1172; returns
       RECOVERED_TRIPLETS);
    4. if input_is_finite(), pass_through() hands the input on unchanged (returns
       RECOVERED_PASSTHROUGH); otherwise commandFailed.

    Any error other than nonFiniteOutput propagates at once. dcn_clip_run_with_fallback_dev
    is the same ladder over the four-branch clip, in the library."""
    report = report or (lambda msg: None)

    def recoverable(e: DeformConvError) -> bool:
        return e.is_recoverable_numerical_failure

    try:
        run(0)
        return 0
    except DeformConvError as e:
        if not recoverable(e):
            raise
        last = e
        report(f"full temporal window failed ({e}); retrying shorter recurrence chunks")
    for chunk in (10, 5, 3):
        if chunk >= frame_count:
            continue
        try:
            run(chunk)
            report(f"recovered with at most {chunk} frames per recurrence chunk")
            return chunk
        except DeformConvError as e:
            if not recoverable(e):
                raise
            last = e
            report(f"also failed with {chunk}-frame chunks ({e})")
    try:
        run_triplets()
        report("recovered with independent zero-motion frame triplets")
        return RECOVERED_TRIPLETS
    except DeformConvError as e:
        if not recoverable(e):
            raise
        last = e
        report(f"also failed independent frame recovery ({e})")
    if not input_is_finite():
        raise DeformConvError(COMMAND_FAILED, f"non-finite input after model failure: {last}")
    report(f"WARNING: using finite input passthrough because all recurrence recovery modes failed ({last})")
    pass_through()
    return RECOVERED_PASSTHROUGH


# ---- temporal schedule ----------------------------------------------------------------

BRANCH_NAMES = ("backward_1", "forward_1", "backward_2", "forward_2")


@dataclasses.dataclass(frozen=True)
class PropagationBranch:
    """PropagationBranch (TemporalSchedule.swift:8-17)."""

    name: str
    direction: str
    pass_: int
    branch_index: int

    @property
    def backbone_input_channels(self) -> int:
        return (2 + self.branch_index) * 64


@dataclasses.dataclass(frozen=True)
class PropagationStep:
    """PropagationStep (TemporalSchedule.swift:19-25); None for the reference's nil."""

    branch: PropagationBranch
    position: int
    frame_index: int
    flow_index: int | None
    second_order_frame_index: int | None


class TemporalSchedule:
    """TemporalSchedule (TemporalSchedule.swift:27-101) from dcn_temporal_schedule."""

    def __init__(self, frame_count: int):
        self.frame_count = int(frame_count)
        self.branches = tuple(PropagationBranch(n, "backward" if i % 2 == 0 else "forward", 1 + i // 2, i)
                              for i, n in enumerate(BRANCH_NAMES))
        n = C.c_size_t()
        cap = max(4 * self.frame_count, 0)
        raw = (_lib.DcnScheduleStep * max(cap, 1))()
        st = lib().dcn_temporal_schedule(self.frame_count, raw, cap, C.byref(n))
        if st != OK:
            raise DeformConvError(st)
        nil = lambda v: None if v < 0 else int(v)  # noqa: E731
        self.steps = tuple(PropagationStep(self.branches[r.branch], r.position, r.frame, nil(r.flow_index),
                                           nil(r.second_order_frame)) for r in raw[:n.value])

    @property
    def flow_count_per_direction(self) -> int:
        return max(self.frame_count - 1, 0)

    @property
    def persistent_tensor_bytes(self) -> int:
        return int(lib().dcn_schedule_persistent_bytes(self.frame_count))


def temporal_chunk_ranges(frame_count: int, maximum_frames_per_chunk: int) -> list[range]:
    """SideBySideRestoration.temporalChunkRanges (SideBySideRestoration.swift:1213-1230)."""
    starts = (C.c_int * max(frame_count, 1))()
    sizes = (C.c_int * max(frame_count, 1))()
    n = C.c_size_t()
    st = lib().dcn_temporal_chunk_ranges(int(frame_count), int(maximum_frames_per_chunk), starts, sizes,
                                         max(frame_count, 1), C.byref(n))
    if st != OK:
        raise DeformConvError(st)
    return [range(starts[i], starts[i] + sizes[i]) for i in range(n.value)]


# ---- deterministic inputs ----------------------------------------------------------

class SeededGenerator:
    """SeededGenerator (DeformConv.swift:168-186): SplitMix64 + Swift's Float.random(in:)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(lib().dcn_splitmix64_seed(C.c_uint64(seed)))

    def next(self) -> int:
        return int(lib().dcn_splitmix64_next(C.byref(self.state)))

    def floats(self, count: int, lo: float, hi: float) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        lib().dcn_seeded_floats(C.byref(self.state), count, lo, hi, _fp(out))
        return out


def config_shape(config: int) -> DeformConvShape:
    s = _lib.DcnShape()
    st = lib().dcn_config_shape(int(config), C.byref(s))
    if st != OK:
        raise DeformConvError(st)
    return DeformConvShape.from_c(s)


def generate_config_inputs(config: int, seed: int) -> dict:
    """FP32 inputs of benchmark config 1, 2, 3 or 5 (see dcn_generate_config_inputs)."""
    shape = config_shape(config)
    c = shape.counts()
    arrays = {k: np.empty(c[k], dtype=np.float32) for k in ("input", "offset", "mask", "weight", "bias")}
    args = []
    for k in ("input", "offset", "mask", "weight", "bias"):
        args += [_fp(arrays[k]), arrays[k].size]
    st = lib().dcn_generate_config_inputs(int(config), C.c_uint64(seed), *args)
    if st != OK:
        raise DeformConvError(st)
    arrays["shape"] = shape
    return arrays


def out_of_bounds_fraction(shape, offset) -> float:
    """Fraction of a layer's samples (output pixel x offset group x tap) whose sampling
    point lies where all four bilinear corners are outside the input (y <= -1, y >= H,
    x <= -1 or x >= W), so that the sample contributes zero: the out-of-bounds rate the
    benchmark configs are drawn for. offset: [B][2*G*Kh*Kw][Ho][Wo] (dy, dx), any float."""
    s = shape
    ka = s.kernel_height * s.kernel_width
    off = np.asarray(offset, np.float64).reshape(s.batch, s.offset_groups, ka, 2, s.output_height,
                                                 s.output_width)
    k = np.arange(ka)
    ky = (k // s.kernel_width).reshape(1, 1, -1, 1, 1)
    kx = (k % s.kernel_width).reshape(1, 1, -1, 1, 1)
    oy = np.arange(s.output_height).reshape(1, 1, 1, -1, 1)
    ox = np.arange(s.output_width).reshape(1, 1, 1, 1, -1)
    y = oy * s.stride_height - s.pad_height + ky * s.dilation_height + off[:, :, :, 0]
    x = ox * s.stride_width - s.pad_width + kx * s.dilation_width + off[:, :, :, 1]
    inside = (y > -1) & (y < s.input_height) & (x > -1) & (x < s.input_width)
    return float(1.0 - inside.mean())


def reference_benchmark_inputs(seed: int = 0x4A41534E41) -> dict:
    """benchmarkJasnaShape's seeded inputs (MetalRunner.swift:210-213, 233-234): input
    U(-1,1), offset U(-0.25,0.25), mask U(0.25,0.75), weight and bias U(-0.02,0.02),
    each drawn in that order and rounded to FP16."""
    shape = JASNA_SHAPE
    rng = SeededGenerator(seed)
    out = {
        "input": rng.floats(shape.input_count, -1.0, 1.0).astype(np.float16),
        "offset": rng.floats(shape.offset_count, -0.25, 0.25).astype(np.float16),
        "mask": rng.floats(shape.mask_count, 0.25, 0.75).astype(np.float16),
        "weight": rng.floats(shape.weight_count, -0.02, 0.02).astype(np.float16),
        "bias": rng.floats(shape.output_channels, -0.02, 0.02).astype(np.float16),
        "shape": shape,
    }
    return out


def generate_body_inputs(height: int = 64, width: int = 64, frames: int = 30, branch: int = 0, blocks: int = 5,
                         seed: int = 4, weight_std: float = 0.02, flow_px: float = 4.0) -> dict:
    """Synthetic config-C4 clip: random-init body weights ~N(0, weight_std) (OIHW FP16),
    per-frame spatial features ~N(0, 1) [frames][64*H*W] and first-order flows
    [frames][2*H*W] (x, y) from a bilinearly upsampled 8x8 grid of U(-flow_px, flow_px),
    all from numpy's PCG64 generator with the given seed."""
    rng = np.random.default_rng(seed)
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16)  # noqa: E731
    w = {}
    for i, (ci, co) in enumerate([(196, 64), (64, 64), (64, 64), (64, 432)]):
        w[f"offset_w{i}"] = f16(rng.normal(0, weight_std, (co, ci, 3, 3)))
        w[f"offset_b{i}"] = f16(rng.normal(0, weight_std, co))
    w["dcn_w"] = f16(rng.normal(0, weight_std, (64, 128, 3, 3)))
    w["dcn_b"] = f16(rng.normal(0, weight_std, 64))
    for i in range(1 + 2 * blocks):
        ci = 64 * (branch + 2) if i == 0 else 64
        w[f"backbone_w{i}"] = f16(rng.normal(0, weight_std, (64, ci, 3, 3)))
        w[f"backbone_b{i}"] = f16(rng.normal(0, weight_std, 64))
    plane = height * width
    feats = f16(rng.standard_normal((frames, 64 * plane)))
    grid_y = np.linspace(0, 7, height)
    grid_x = np.linspace(0, 7, width)
    flows = np.empty((frames, 2, height, width), np.float32)
    for t in range(frames):
        for c in range(2):
            g = rng.uniform(-flow_px, flow_px, (8, 8))
            y0 = np.minimum(np.floor(grid_y).astype(int), 6)
            x0 = np.minimum(np.floor(grid_x).astype(int), 6)
            ly = (grid_y - y0)[:, None]
            lx = (grid_x - x0)[None, :]
            flows[t, c] = (g[y0][:, x0] * (1 - ly) * (1 - lx) + g[y0][:, x0 + 1] * (1 - ly) * lx +
                           g[y0 + 1][:, x0] * ly * (1 - lx) + g[y0 + 1][:, x0 + 1] * ly * lx)
    prefix = f16(rng.standard_normal((branch, frames, 64 * plane)))
    return {"weights": w, "feats": feats, "flows": f16(flows.reshape(frames, 2 * plane)), "prefix": prefix,
            "height": height, "width": width, "frames": frames, "branch": branch, "blocks": blocks}


def body_flops(height: int, width: int, branch: int = 0, blocks: int = 5) -> int:
    """GEMM-equivalent flops of one body: conv_offset, the DCN and the backbone."""
    plane = height * width
    convs = [(196, 64), (64, 64), (64, 64), (64, 432), (64 * (branch + 2), 64)] + [(64, 64)] * (2 * blocks)
    return sum(2 * plane * 9 * ci * co for ci, co in convs) + 2 * plane * 9 * 128 * 64


def clip_flops(height: int, width: int, frames: int, blocks: int = 5) -> int:
    """GEMM-equivalent flops of a four-branch clip: per branch one first step (backbone
    only) and frames - 1 full bodies."""
    plane = height * width
    total = 0
    for b in range(4):
        backbone = sum(2 * plane * 9 * ci * co for ci, co in [(64 * (b + 2), 64)] + [(64, 64)] * (2 * blocks))
        total += backbone + (frames - 1) * body_flops(height, width, b, blocks)
    return total


SPYNET_LAYERS = [(8, 32), (32, 64), (64, 32), (32, 16), (16, 2)]


def generate_spynet_inputs(tile: int = 256, seed: int = 6, flow_std: float = 0.04) -> dict:
    """Synthetic SPyNet workload: two RGB LQ tiles [3][tile][tile] in [0, 1] (random
    sinusoids, the second shifted by (1.5, -2.0) px) and random-init basic modules
    (He-normal 7x7 weights for the ReLU layers, N(0, flow_std) for the flow layer, biases
    N(0, 0.01); OIHW FP16 "w{level}_{layer}" / "b{level}_{layer}"), numpy PCG64."""
    rng = np.random.default_rng(seed)
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16)  # noqa: E731
    w = {}
    for level in range(_lib.SPYNET_LEVELS):
        for i, (ci, co) in enumerate(SPYNET_LAYERS):
            std = flow_std if i == len(SPYNET_LAYERS) - 1 else np.sqrt(2.0 / (ci * 49))
            w[f"w{level}_{i}"] = f16(rng.normal(0, std, (co, ci, 7, 7)))
            w[f"b{level}_{i}"] = f16(rng.normal(0, 0.01, co))
    waves = [(rng.uniform(-0.08, 0.08, 2), rng.uniform(0.2, 1.0), rng.uniform(0, 2 * np.pi))
             for _ in range(12)]

    def frame(dy, dx):
        y, x = np.meshgrid(np.arange(tile) + dy, np.arange(tile) + dx, indexing="ij")
        out = np.empty((3, tile, tile))
        for c in range(3):
            acc = sum(a * np.sin(f[0] * y + f[1] * x + ph) for f, a, ph in waves[4 * c:4 * c + 4])
            out[c] = 0.5 + 0.12 * acc
        return f16(np.clip(out, 0, 1).ravel())

    return {"tile": tile, "weights": w, "reference": frame(0.0, 0.0), "support": frame(1.5, -2.0)}


def spynet_flops(height: int, width: int) -> int:
    """GEMM-equivalent flops of one SPyNet direction (the 7x7 convs of six levels)."""
    total = 0
    for level in range(_lib.SPYNET_LEVELS):
        plane = (height >> (_lib.SPYNET_LEVELS - 1 - level)) * (width >> (_lib.SPYNET_LEVELS - 1 - level))
        total += sum(2 * plane * 49 * ci * co for ci, co in SPYNET_LAYERS)
    return total


def pack_ic_k_oc(weight_oihw: np.ndarray, shape: DeformConvShape) -> np.ndarray:
    """OIHW -> [ic][k][oc] (MetalRunner.swift:235-243; tools/export_deform_weights.py:47)."""
    w = np.asarray(weight_oihw).reshape(shape.output_channels, shape.input_channels, shape.kernel_area)
    return np.ascontiguousarray(np.transpose(w, (1, 2, 0)))


def checksum(values: np.ndarray) -> float:
    """Sum in double of values[0::257] (MetalRunner.swift:332-337)."""
    v = np.asarray(values).ravel()
    if v.dtype == np.float32:
        v = np.ascontiguousarray(v)
        return float(lib().dcn_checksum_f32(_fp(v), v.size))
    v = _u16(v)
    return float(lib().dcn_checksum_f16(_hp(v), v.size))


@dataclasses.dataclass
class BenchmarkStatistics:
    """BenchmarkStatistics (BenchmarkStatistics.swift:3-44)."""

    samples: list
    minimum: float
    maximum: float
    median: float
    mean: float
    standard_deviation: float
    percentile10: float
    percentile90: float

    @classmethod
    def of(cls, values) -> Optional["BenchmarkStatistics"]:
        v = np.ascontiguousarray(values, dtype=np.float64)
        s = _lib.DcnStatistics()
        if lib().dcn_compute_statistics(v.ctypes.data_as(_lib.c_f64p), v.size, C.byref(s)) != OK:
            return None
        return cls(sorted(v.tolist()), s.minimum, s.maximum, s.median, s.mean,
                   s.standard_deviation, s.percentile10, s.percentile90)


@dataclasses.dataclass
class BenchmarkResult:
    """BenchmarkResult (MetalRunner.swift:67-90) for the variants this build has: the
    direct FP16 baseline, the gather alone and the fused path (milliseconds)."""

    baseline: BenchmarkStatistics
    gather: BenchmarkStatistics
    fused: BenchmarkStatistics
    checksum: float
    max_difference_from_baseline: float
    iterations: int


def f32_to_f16(values) -> np.ndarray:
    v = _f32(values).ravel()
    out = np.empty(v.size, dtype=np.uint16)
    lib().dcn_f32_to_f16_array(_fp(v), _hp(out), v.size)
    return out.view(np.float16).reshape(np.shape(values))
