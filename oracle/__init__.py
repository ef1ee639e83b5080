"""ctypes binding of the CPU oracle (oracle/dcn_oracle.c) — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as
the checker. The product (jasnamacos_amd, libdcn) never imports or links it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


class OracleShape(C.Structure):
    _fields_ = [
        (name, C.c_int32)
        for name in (
            "batch", "input_channels", "input_height", "input_width",
            "output_channels", "output_height", "output_width",
            "kernel_height", "kernel_width", "pad_height", "pad_width",
            "stride_height", "stride_width", "dilation_height", "dilation_width",
            "groups", "offset_groups",
        )
    ]


_f = C.POINTER(C.c_float)
_h = C.POINTER(C.c_uint16)
_S = C.POINTER(OracleShape)
_SIG = {
    "oracle_shape_validate": (C.c_int, [_S]),
    "oracle_dcn_forward_f32": (C.c_int, [_S, _f, _f, _f, _f, _f, _f]),
    "oracle_dcn_forward_f32_threads": (C.c_int, [_S, _f, _f, _f, _f, _f, _f, C.c_int]),
    "oracle_dcn_forward_f32_oc_range": (C.c_int, [_S, _f, _f, _f, _f, _f, _f, C.c_int, C.c_int]),
    "oracle_dcn_forward_f16_direct": (C.c_int, [_S, _h, _h, _h, _h, _h, _h]),
    "oracle_dcn_im2col_f16": (C.c_int, [_S, _h, _h, _h, _h]),
    "oracle_dcn_gemm_f16": (C.c_int, [_S, _h, _h, _h, _h]),
    "oracle_dcn_im2col_bf16": (C.c_int, [_S, _h, _h, _h, _h]),
    "oracle_f32_to_bf16": (C.c_uint16, [C.c_float]),
    "oracle_bf16_to_f32": (C.c_float, [C.c_uint16]),
    "oracle_f32_to_f16": (C.c_uint16, [C.c_float]),
    "oracle_f16_to_f32": (C.c_float, [C.c_uint16]),
    "oracle_flag_nonfinite_f16": (C.c_uint32, [_h, C.c_size_t]),
    "oracle_offset_transform_f16": (None, [C.c_size_t, _h, _h, _h, _h, _h]),
    "oracle_sample_zero_f16": (C.c_float, [_h, C.c_size_t, C.c_int, C.c_int, C.c_float, C.c_float]),
    "oracle_temporal_prepare_f16": (None, [C.c_int, C.c_int, C.c_int, _h, _h, _h, _h, _h, _h, _h, _h]),
    "oracle_conv3x3_f16": (None, [C.c_int, C.c_int, C.c_int, C.c_int, _h, _h, _h, C.c_int, C.c_float,
                                  _h, _h]),
    "oracle_bicubic_quarter_f16": (None, [C.c_int, C.c_int, C.c_int, _h, _h]),
    "oracle_spynet_pyramid_f16": (None, [C.c_int, C.c_int, C.c_int, _h, C.POINTER(_h)]),
    "oracle_sample_border_f16": (C.c_float, [_h, C.c_size_t, C.c_int, C.c_int, C.c_float, C.c_float]),
    "oracle_spynet_prepare_f16": (None, [C.c_int, C.c_int, C.c_int, _h, _h, _h, C.c_int, C.c_int, _h, _h]),
    "oracle_add_f16": (None, [C.c_size_t, _h, _h, _h]),
    "oracle_convk_f16": (None, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _h, _h, _h, C.c_int, C.c_float,
                                _h]),
}

_LIB = None


def load() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-C", str(HERE)], check=True, capture_output=True)
        lib = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def _shape(shape) -> OracleShape:
    return OracleShape(*[getattr(shape, name) for name, _ in OracleShape._fields_])


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    return a, a.ctypes.data_as(_f)


def _u16(a):
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    a = np.ascontiguousarray(a, dtype=np.uint16).ravel()
    return a, a.ctypes.data_as(_h)


def _bits(a):
    """BF16 bit patterns (uint16 arrays; numpy has no BF16 type)."""
    a = np.asarray(a)
    if a.dtype != np.uint16:
        raise TypeError(f"expected BF16 bit patterns as uint16, got {a.dtype}")
    a = np.ascontiguousarray(a).ravel()
    return a, a.ctypes.data_as(_h)


def _counts(shape):
    ka = shape.kernel_height * shape.kernel_width
    plane = shape.output_height * shape.output_width
    return {
        "output": shape.batch * shape.output_channels * plane,
        "columns": shape.batch * plane * shape.input_channels * ka,
    }


def forward_f32(shape, input, offset, mask, weight, bias) -> np.ndarray:
    """DeformConvCPU.run (DeformConv.swift:76-138)."""
    keep = [_f32(a) for a in (input, offset, mask, weight, bias)]
    out = np.empty(_counts(shape)["output"], dtype=np.float32)
    rc = load().oracle_dcn_forward_f32(C.byref(_shape(shape)), *[p for _, p in keep], out.ctypes.data_as(_f))
    if rc:
        raise ValueError("invalid shape")
    return out


def forward_f32_threads(shape, input, offset, mask, weight, bias, threads=None) -> np.ndarray:
    """forward_f32 spread over output channels; bit-identical results."""
    import os

    threads = threads or min(16, os.cpu_count() or 1)
    keep = [_f32(a) for a in (input, offset, mask, weight, bias)]
    out = np.empty(_counts(shape)["output"], dtype=np.float32)
    rc = load().oracle_dcn_forward_f32_threads(C.byref(_shape(shape)), *[p for _, p in keep],
                                               out.ctypes.data_as(_f), int(threads))
    if rc:
        raise ValueError("invalid shape")
    return out


def forward_f32_oc_range(shape, input, offset, mask, weight, bias, oc_begin, oc_end) -> np.ndarray:
    keep = [_f32(a) for a in (input, offset, mask, weight, bias)]
    out = np.zeros(_counts(shape)["output"], dtype=np.float32)
    rc = load().oracle_dcn_forward_f32_oc_range(C.byref(_shape(shape)), *[p for _, p in keep],
                                                out.ctypes.data_as(_f), int(oc_begin), int(oc_end))
    if rc:
        raise ValueError("invalid shape")
    return out


def forward_f32_ocs(shape, input, offset, mask, weight, bias, ocs, threads=None) -> np.ndarray:
    """forward_f32's output channels `ocs` (zeros elsewhere), one channel per task over a
    thread pool (the C call releases the GIL); each channel is the serial loop's bits."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    threads = threads or min(16, os.cpu_count() or 1)
    keep = [_f32(a) for a in (input, offset, mask, weight, bias)]
    out = np.zeros(_counts(shape)["output"], dtype=np.float32)
    fn = load().oracle_dcn_forward_f32_oc_range
    plane = shape.output_height * shape.output_width
    outs = {}

    def one(oc):
        part = np.zeros_like(out)
        rc = fn(C.byref(_shape(shape)), *[p for _, p in keep], part.ctypes.data_as(_f), int(oc), int(oc) + 1)
        if rc:
            raise ValueError("invalid shape")
        outs[oc] = part

    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(one, ocs))
    view, cout = out.reshape(shape.batch, -1, plane), shape.output_channels
    for oc, part in outs.items():
        view[:, oc] = part.reshape(shape.batch, cout, plane)[:, oc]
    return out


def forward_f16_direct(shape, input, offset, mask, weight, bias) -> np.ndarray:
    """deform_conv2d_fp16 (MetalShader.swift:126-174)."""
    keep = [_u16(a) for a in (input, offset, mask, weight, bias)]
    out = np.empty(_counts(shape)["output"], dtype=np.uint16)
    rc = load().oracle_dcn_forward_f16_direct(C.byref(_shape(shape)), *[p for _, p in keep],
                                              out.ctypes.data_as(_h))
    if rc:
        raise ValueError("invalid shape")
    return out.view(np.float16)


def im2col_bf16(shape, input, offset, mask) -> np.ndarray:
    """The gather of im2col_f16 over BF16 storage (uint16 bit patterns in and out), each
    sample rounded once to BF16: the columns of the library's BF16 fused path."""
    keep = [_bits(a) for a in (input, offset, mask)]
    out = np.empty(_counts(shape)["columns"], dtype=np.uint16)
    rc = load().oracle_dcn_im2col_bf16(C.byref(_shape(shape)), *[p for _, p in keep], out.ctypes.data_as(_h))
    if rc:
        raise ValueError("invalid shape")
    return out


def im2col_f16(shape, input, offset, mask) -> np.ndarray:
    """deform_conv2d_fp16_jasna_gather (MetalShader.swift:299-381), any offset groups."""
    keep = [_u16(a) for a in (input, offset, mask)]
    out = np.empty(_counts(shape)["columns"], dtype=np.uint16)
    rc = load().oracle_dcn_im2col_f16(C.byref(_shape(shape)), *[p for _, p in keep], out.ctypes.data_as(_h))
    if rc:
        raise ValueError("invalid shape")
    return out.view(np.float16)


def gemm_f16(shape, columns, weight, bias) -> np.ndarray:
    """deform_conv2d_fp16_jasna_simdgroup_gemm_fused (MetalShader.swift:387-452)."""
    keep = [_u16(a) for a in (columns, weight, bias)]
    out = np.empty(_counts(shape)["output"], dtype=np.uint16)
    rc = load().oracle_dcn_gemm_f16(C.byref(_shape(shape)), *[p for _, p in keep], out.ctypes.data_as(_h))
    if rc:
        raise ValueError("invalid shape")
    return out.view(np.float16)


def f32_to_f16_bits(values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    fn = load().oracle_f32_to_f16
    return np.array([fn(float(x)) for x in v], dtype=np.uint16)


def f16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    fn = load().oracle_f16_to_f32
    return np.array([fn(int(x)) for x in b], dtype=np.float32)


def flag_nonfinite_f16(values) -> int:
    v, p = _u16(values)
    return int(load().oracle_flag_nonfinite_f16(p, v.size))


def offset_transform_f16(plane, raw, flow1, flow2):
    """prepare_dcn_offsets_fp16 (MetalShader.swift:817-839)."""
    keep = [_u16(a) for a in (raw, flow1, flow2)]
    off = np.empty(288 * plane, dtype=np.uint16)
    msk = np.empty(144 * plane, dtype=np.uint16)
    load().oracle_offset_transform_f16(plane, *[p for _, p in keep], off.ctypes.data_as(_h),
                                       msk.ctypes.data_as(_h))
    return off.view(np.float16), msk.view(np.float16)


def temporal_prepare_f16(width, height, has_second_order, feat_prop, feat_current, feat_n2, flow1, prev_flow):
    """accumulate_second_order_flow_fp16 + assemble_temporal_alignment_fp16 (MetalShader.swift:739-813)."""
    plane = width * height
    keep = [_u16(a) for a in (feat_prop, feat_current, feat_n2, flow1, prev_flow)]
    flow2 = np.empty(2 * plane, dtype=np.uint16)
    cond = np.empty(196 * plane, dtype=np.uint16)
    dinp = np.empty(128 * plane, dtype=np.uint16)
    load().oracle_temporal_prepare_f16(width, height, int(bool(has_second_order)), *[p for _, p in keep],
                                       flow2.ctypes.data_as(_h), cond.ctypes.data_as(_h),
                                       dinp.ctypes.data_as(_h))
    return flow2.view(np.float16), cond.view(np.float16), dinp.view(np.float16)


def conv3x3_f16(cin, cout, height, width, input, weight, bias, activation=0, slope=0.1, residual=None):
    keep = [_u16(a) for a in (input, weight, bias)]
    res = _u16(residual) if residual is not None else (None, None)
    out = np.empty(cout * height * width, dtype=np.uint16)
    load().oracle_conv3x3_f16(cin, cout, height, width, *[p for _, p in keep], int(activation), float(slope),
                              res[1], out.ctypes.data_as(_h))
    return out.view(np.float16)


def bicubic_quarter_f16(channels, height, width, input):
    """jasna_bicubic_downsample_quarter_fp16 (MetalShader.swift:488-521)."""
    i, p = _u16(input)
    out = np.empty(channels * (height // 4) * (width // 4), dtype=np.uint16)
    load().oracle_bicubic_quarter_f16(channels, height, width, p, out.ctypes.data_as(_h))
    return out.view(np.float16)


def spynet_pyramid_f16(height, width, levels, frame):
    """spynet_build_pyramid_pair_fp16 (MetalShader.swift:523-570), one frame: a list of
    `levels` [3][h_l][w_l] arrays, coarsest first."""
    f, p = _u16(frame)
    outs = [np.empty(3 * (height >> (levels - 1 - l)) * (width >> (levels - 1 - l)), dtype=np.uint16)
            for l in range(levels)]
    ptrs = (_h * levels)(*[o.ctypes.data_as(_h) for o in outs])
    load().oracle_spynet_pyramid_f16(height, width, levels, p, ptrs)
    return [o.view(np.float16) for o in outs]


def spynet_prepare_f16(width, height, first_level, reference, support, source_flow, source_width,
                       source_height):
    """spynet_prepare_fp16 (MetalShader.swift:601-639): (features [8][h][w], base_flow [2][h][w])."""
    keep = [_u16(a) for a in (reference, support)]
    src = _u16(source_flow if source_flow is not None else np.zeros(2, np.float16))
    plane = width * height
    feat = np.empty(8 * plane, dtype=np.uint16)
    base = np.empty(2 * plane, dtype=np.uint16)
    load().oracle_spynet_prepare_f16(width, height, int(bool(first_level)), *[p for _, p in keep], src[1],
                                     source_width, source_height, feat.ctypes.data_as(_h),
                                     base.ctypes.data_as(_h))
    return feat.view(np.float16), base.view(np.float16)


def add_f16(base, residual):
    """spynet_add_flow_fp16 (MetalShader.swift:641-649)."""
    b, pb = _u16(base)
    r, pr = _u16(residual)
    out = np.empty(b.size, dtype=np.uint16)
    load().oracle_add_f16(b.size, pb, pr, out.ctypes.data_as(_h))
    return out.view(np.float16)


def convk_f16(k, cin, cout, height, width, input, weight, bias, activation=0, slope=0.1):
    keep = [_u16(a) for a in (input, weight, bias)]
    out = np.empty(cout * height * width, dtype=np.uint16)
    load().oracle_convk_f16(k, cin, cout, height, width, *[p for _, p in keep], int(activation), float(slope),
                            out.ctypes.data_as(_h))
    return out.view(np.float16)
