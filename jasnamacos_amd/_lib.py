"""ctypes binding of libdcn (include/dcn/dcn.h).

The library is built in-tree by jasnamacos_amd.build into jasnamacos_amd/lib/libdcn.so.
Loading fails loudly when it is missing: there is no CPU fallback behind this module.
"""
from __future__ import annotations

import ctypes as C
import os
import sys
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libdcn.so"

c_size = C.c_size_t
c_u16p = C.POINTER(C.c_uint16)
c_f32p = C.POINTER(C.c_float)
c_f64p = C.POINTER(C.c_double)
c_u64p = C.POINTER(C.c_uint64)
c_void = C.c_void_p
# dcn_report_fn: void (*)(const char* message, void* user)
ReportFn = C.CFUNCTYPE(None, C.c_char_p, C.c_void_p)


class DcnShape(C.Structure):
    """dcn_shape: the 17 DeformConvShape fields (DeformConv.swift:3-20)."""

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


class DcnCounts(C.Structure):
    _fields_ = [(n, c_size) for n in ("input", "output", "kernel_area", "offset", "mask", "weight", "bias")]


class DcnStatistics(C.Structure):
    _fields_ = [
        ("minimum", C.c_double), ("maximum", C.c_double), ("median", C.c_double),
        ("mean", C.c_double), ("standard_deviation", C.c_double),
        ("percentile10", C.c_double), ("percentile90", C.c_double), ("count", c_size),
    ]


BODY_MAX_BLOCKS = 8


class DcnScheduleStep(C.Structure):
    """dcn_schedule_step: one PropagationStep of TemporalSchedule (-1 for nil)."""

    _fields_ = [(n, C.c_int) for n in ("branch", "position", "frame", "flow_index", "second_order_frame")]


SPYNET_LEVELS = 6
SPYNET_LAYERS = 5


class DcnSpynetWeights(C.Structure):
    """dcn_spynet_weights: OIHW FP16 device pointers, [level][layer], level 0 coarsest."""

    _fields_ = [
        ("weight", (C.c_void_p * SPYNET_LAYERS) * SPYNET_LEVELS),
        ("bias", (C.c_void_p * SPYNET_LAYERS) * SPYNET_LEVELS),
    ]


class DcnBodyWeights(C.Structure):
    """dcn_body_weights: OIHW FP16 device pointers of one propagation body."""

    _fields_ = [
        ("offset_weight", C.c_void_p * 4),
        ("offset_bias", C.c_void_p * 4),
        ("dcn_weight", C.c_void_p),
        ("dcn_bias", C.c_void_p),
        ("backbone_weight", C.c_void_p * (1 + 2 * BODY_MAX_BLOCKS)),
        ("backbone_bias", C.c_void_p * (1 + 2 * BODY_MAX_BLOCKS)),
    ]


ShapeP = C.POINTER(DcnShape)
CtxP = c_void
PackedP = c_void

# name -> (restype, argtypes). Every symbol declared in include/dcn/dcn.h.
SIGNATURES: dict[str, tuple] = {
    "dcn_abi_version": (C.c_int, []),
    "dcn_status_is_recoverable": (C.c_int, [C.c_int]),
    "dcn_status_string": (C.c_char_p, [C.c_int]),
    "dcn_shape_validate": (C.c_int, [ShapeP]),
    "dcn_shape_counts": (C.c_int, [ShapeP, C.POINTER(DcnCounts)]),
    "dcn_shape_fused_supported": (C.c_int, [ShapeP]),
    "dcn_create": (C.c_int, [C.POINTER(CtxP), C.c_int]),
    "dcn_destroy": (None, [CtxP]),
    "dcn_last_error": (C.c_char_p, [CtxP]),
    "dcn_reserve": (C.c_int, [CtxP, ShapeP]),
    "dcn_forward_f32": (C.c_int, [CtxP, ShapeP, c_f32p, c_size, c_f32p, c_size, c_f32p, c_size,
                                  c_f32p, c_size, c_f32p, c_size, c_f32p, c_size]),
    "dcn_forward_f16": (C.c_int, [CtxP, ShapeP, c_u16p, c_size, c_u16p, c_size, c_u16p, c_size,
                                  c_u16p, c_size, c_u16p, c_size, c_u16p, c_size]),
    "dcn_prepack_f16": (C.c_int, [CtxP, ShapeP, c_u16p, c_size, C.c_int, c_u16p, c_size,
                                  C.POINTER(PackedP)]),
    "dcn_prepack_f16_dev": (C.c_int, [CtxP, ShapeP, c_void, C.c_int, c_void, c_void,
                                      C.POINTER(PackedP)]),
    "dcn_prepack_bf16": (C.c_int, [CtxP, ShapeP, c_u16p, c_size, C.c_int, c_u16p, c_size,
                                   C.POINTER(PackedP)]),
    "dcn_prepack_bf16_dev": (C.c_int, [CtxP, ShapeP, c_void, C.c_int, c_void, c_void,
                                       C.POINTER(PackedP)]),
    "dcn_forward_bf16_prepacked": (C.c_int, [CtxP, ShapeP, c_u16p, c_size, c_u16p, c_size,
                                             c_u16p, c_size, PackedP, c_u16p, c_size]),
    "dcn_forward_bf16_prepacked_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void, PackedP,
                                                 c_void, c_void]),
    "dcn_forward_bf16_prepacked_cb8_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void, PackedP,
                                                     c_void, c_void]),
    "dcn_packed_free": (None, [PackedP]),
    "dcn_load_dcnfp16": (C.c_int, [CtxP, C.c_char_p, C.POINTER(PackedP)]),
    "dcn_dcnfp16_bytes": (c_size, []),
    "dcn_forward_f16_prepacked": (C.c_int, [CtxP, ShapeP, c_u16p, c_size, c_u16p, c_size,
                                            c_u16p, c_size, PackedP, c_u16p, c_size]),
    "dcn_forward_f32_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void, c_void, c_void,
                                      c_void, c_void]),
    "dcn_forward_f16_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void, c_void, c_void,
                                      c_void, c_void]),
    "dcn_forward_f16_prepacked_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void, PackedP,
                                                c_void, c_void]),
    "dcn_cb8_count": (c_size, [ShapeP]),
    "dcn_pack_input_cb8_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void]),
    "dcn_forward_f16_prepacked_cb8_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void,
                                                    PackedP, c_void, c_void]),
    "dcn_forward_f16_prepacked_noalloc_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void,
                                                        PackedP, c_void, c_void]),
    "dcn_set_fused_config": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.c_int]),
    "dcn_get_fused_config": (C.c_int, [CtxP, ShapeP, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                       C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "dcn_im2col_f16_dev": (C.c_int, [CtxP, ShapeP, c_void, c_void, c_void, c_void, c_void]),
    "dcn_launch_floor_dev": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, c_void]),
    "dcn_set_tile_clock_dev": (C.c_int, [CtxP, c_void, C.c_size_t]),
    "dcn_flag_nonfinite_f16_dev": (C.c_int, [CtxP, c_void, c_size, c_void, c_void]),
    "dcn_check_nonfinite_f16_dev": (C.c_int, [CtxP, c_void, c_size, c_void]),
    "dcn_splitmix64_seed": (C.c_uint64, [C.c_uint64]),
    "dcn_splitmix64_next": (C.c_uint64, [c_u64p]),
    "dcn_seeded_floats": (None, [c_u64p, c_size, C.c_float, C.c_float, c_f32p]),
    "dcn_config_shape": (C.c_int, [C.c_int, ShapeP]),
    "dcn_generate_config_inputs": (C.c_int, [C.c_int, C.c_uint64, c_f32p, c_size, c_f32p, c_size,
                                             c_f32p, c_size, c_f32p, c_size, c_f32p, c_size]),
    "dcn_f32_to_f16": (C.c_uint16, [C.c_float]),
    "dcn_f16_to_f32": (C.c_float, [C.c_uint16]),
    "dcn_f32_to_f16_array": (None, [c_f32p, c_u16p, c_size]),
    "dcn_f16_to_f32_array": (None, [c_u16p, c_f32p, c_size]),
    "dcn_checksum_f32": (C.c_double, [c_f32p, c_size]),
    "dcn_checksum_f16": (C.c_double, [c_u16p, c_size]),
    "dcn_compute_statistics": (C.c_int, [c_f64p, c_size, C.POINTER(DcnStatistics)]),
    # propagation body
    "dcn_cb8_tensor_count": (c_size, [C.c_int, C.c_int, C.c_int]),
    "dcn_offset_transform_f16": (C.c_int, [CtxP, c_size, c_u16p, c_size, c_u16p, c_size, c_u16p, c_size,
                                           c_u16p, c_size, c_u16p, c_size]),
    "dcn_offset_transform_f16_dev": (C.c_int, [CtxP, c_size, c_void, c_void, c_void, c_void, c_void, c_void]),
    "dcn_temporal_prepare_f16": (C.c_int, [CtxP, C.c_int, C.c_int, c_u16p, c_size, c_u16p, c_size, c_u16p,
                                           c_size, c_u16p, c_size, c_u16p, c_size, C.c_int, c_u16p, c_size,
                                           c_u16p, c_size, c_u16p, c_size]),
    "dcn_temporal_prepare_f16_dev": (C.c_int, [CtxP, C.c_int, C.c_int, c_void, c_void, c_void, c_void, c_void,
                                               C.c_int, c_void, c_void, C.c_int, c_void, C.c_int, c_void]),
    "dcn_assemble_backbone_f16_dev": (C.c_int, [CtxP, C.c_int, C.c_int, C.POINTER(c_void), C.c_int, c_void,
                                                C.c_int, c_void]),
    "dcn_add_residual_f16_dev": (C.c_int, [CtxP, c_size, c_void, c_void, c_void, c_void]),
    "dcn_cb8_to_nchw_f16_dev": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, c_void, c_void, c_void]),
    "dcn_conv3x3_create_dev": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.c_int, c_void, c_void, c_void,
                                         C.POINTER(c_void)]),
    "dcn_conv3x3_free": (None, [c_void]),
    "dcn_conv3x3_f16_dev": (C.c_int, [CtxP, c_void, c_void, C.c_int, C.c_float, c_void, C.c_int, c_void,
                                      C.c_int, c_void, C.c_int, c_void]),
    "dcn_bicubic_quarter_f16_dev": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, c_void, c_void, c_void]),
    "dcn_spynet_create": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.POINTER(DcnSpynetWeights), c_void,
                                    C.POINTER(c_void)]),
    "dcn_spynet_clip_flows_dev": (C.c_int, [c_void, c_void, C.c_int, c_void, c_void]),
    "dcn_spynet_destroy": (None, [c_void]),
    "dcn_spynet_pyramid_f16_dev": (C.c_int, [CtxP, C.c_int, C.c_int, c_void, c_void, c_void]),
    "dcn_spynet_flow_dev": (C.c_int, [c_void, c_void, c_void, C.c_int, c_void, c_void]),
    "dcn_conv3x3_offsets_f16_dev": (C.c_int, [CtxP, c_void, c_void, c_void, c_void, c_void, c_void, c_void]),
    "dcn_conv3x3_pair_f16_dev": (C.c_int, [CtxP, c_void, c_void, c_void, C.c_int, C.c_int, C.c_float, c_void,
                                           C.c_int, c_void, C.c_int, c_void, C.c_int, c_void]),
    "dcn_body_create": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(DcnBodyWeights),
                                  c_void, C.POINTER(c_void)]),
    "dcn_body_create_tiles": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.POINTER(DcnBodyWeights), c_void, C.POINTER(c_void)]),
    "dcn_body_destroy": (None, [c_void]),
    "dcn_body_step_dev": (C.c_int, [c_void, c_void, c_void, c_void, c_void, c_void, C.POINTER(c_void),
                                    C.c_int, c_void, c_void, c_void]),
    "dcn_body_capture": (C.c_int, [c_void, c_void, c_void, c_void, c_void, c_void, C.POINTER(c_void),
                                   C.c_int, c_void, c_void, C.POINTER(c_void)]),
    "dcn_graph_launch": (C.c_int, [c_void, c_void]),
    "dcn_graph_destroy": (None, [c_void]),
    "dcn_body_initial_step_dev": (C.c_int, [c_void, c_void, C.POINTER(c_void), c_void, c_void]),
    "dcn_body_step_cb8_dev": (C.c_int, [c_void, c_void, c_void, c_void, c_void, c_void, C.POINTER(c_void),
                                        C.c_int, c_void, c_void, c_void, c_void]),
    "dcn_body_initial_step_cb8_dev": (C.c_int, [c_void, c_void, C.POINTER(c_void), c_void, c_void, c_void]),
    "dcn_body_capture_cb8": (C.c_int, [c_void, c_void, c_void, c_void, c_void, c_void, C.POINTER(c_void),
                                       C.c_int, c_void, c_void, c_void, C.POINTER(c_void)]),
    # temporal schedule and the four-branch clip
    "dcn_temporal_schedule": (C.c_int, [C.c_int, C.POINTER(DcnScheduleStep), c_size, C.POINTER(c_size)]),
    "dcn_schedule_persistent_bytes": (c_size, [C.c_int]),
    "dcn_temporal_chunk_ranges": (C.c_int, [C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int), c_size,
                                            C.POINTER(c_size)]),
    "dcn_clip_create": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(DcnBodyWeights), c_void,
                                  C.POINTER(c_void)]),
    "dcn_clip_create_tiles": (C.c_int, [CtxP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.POINTER(DcnBodyWeights), c_void, C.POINTER(c_void)]),
    "dcn_clip_destroy": (None, [c_void]),
    "dcn_clip_run_dev": (C.c_int, [c_void, c_void, c_void, c_void, c_void, C.c_int, c_void]),
    "dcn_clip_capture": (C.c_int, [c_void, c_void, c_void, c_void, c_void, C.c_int, C.POINTER(c_void)]),
    "dcn_clip_run_with_fallback_dev": (C.c_int, [c_void, c_void, c_void, c_void, c_void, c_void, ReportFn, c_void,
                                                 C.POINTER(C.c_int)]),
}

_LIB: C.CDLL | None = None


def _share_hip_runtime_with_torch() -> None:
    """Keep one HIP runtime per process.

    PyTorch-ROCm ships its own libamdhip64 and links it by the unversioned name, while
    libdcn links libamdhip64.so.7 from /opt/rocm. Loaded in the order libdcn-then-torch,
    the loader maps both copies and the second runtime to initialise sees no device.
    Importing torch first (when it is installed) lets libdcn bind to torch's already
    loaded runtime, whose soname matches; without torch there is only ROCm's."""
    if "torch" in sys.modules:
        return
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load() -> C.CDLL:
    """Load libdcn.so once; raise ImportError if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("DCN_LIBRARY", LIB_PATH))
    _share_hip_runtime_with_torch()
    if not path.exists():
        raise ImportError(
            f"libdcn.so not found at {path}; build it with `python -m jasnamacos_amd.build` "
            "(there is no CPU fallback)"
        )
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib
