"""CPU reference of one propagation body, built from the oracle's pinned pieces.

Test infrastructure: the chain below restates the per-step body of the reference
(FusedFourPassRecurrenceProbe.swift:570-664 for the order of the layers, the glue
kernels of MetalShader.swift:738-929) with the oracle's temporal preparation, offset
transform, conv3x3 and FP32 DCN, every tensor rounded to FP16 between layers.
"""
from __future__ import annotations

import dataclasses

import numpy as np

import oracle


def f16(a) -> np.ndarray:
    return np.asarray(a, np.float32).astype(np.float16)


def body_weights(rng: np.random.Generator, branch: int = 0, blocks: int = 5, std: float = 0.02) -> dict:
    """Random-init weights of one body (~N(0, std), biases ~N(0, std)), FP16 OIHW arrays."""
    w = {}
    for i, (ci, co) in enumerate([(196, 64), (64, 64), (64, 64), (64, 432)]):
        w[f"offset_w{i}"] = f16(rng.normal(0, std, (co, ci, 3, 3)))
        w[f"offset_b{i}"] = f16(rng.normal(0, std, co))
    w["dcn_w"] = f16(rng.normal(0, std, (64, 128, 3, 3)))
    w["dcn_b"] = f16(rng.normal(0, std, 64))
    for i in range(1 + 2 * blocks):
        ci = 64 * (branch + 2) if i == 0 else 64
        w[f"backbone_w{i}"] = f16(rng.normal(0, std, (64, ci, 3, 3)))
        w[f"backbone_b{i}"] = f16(rng.normal(0, std, 64))
    return w


def body_inputs(rng: np.random.Generator, height: int, width: int, branch: int = 0, flow_px: float = 3.0) -> dict:
    plane = height * width
    d = {
        "feat_current": f16(rng.standard_normal(64 * plane)),
        "feat_prop": f16(rng.standard_normal(64 * plane)),
        "feat_n2": f16(rng.standard_normal(64 * plane)),
        "flow1": f16(rng.uniform(-flow_px, flow_px, 2 * plane)),
        "prev_flow": f16(rng.uniform(-flow_px, flow_px, 2 * plane)),
    }
    d["prefix"] = [f16(rng.standard_normal(64 * plane)) for _ in range(branch)]
    return d


def body_step(weights: dict, x: dict, height: int, width: int, blocks: int, has_second_order: bool = True,
              shape_cls=None):
    """(flow2, feat_prop_out) of one body step on the CPU."""
    plane = height * width
    flow2, cond, dinp = oracle.temporal_prepare_f16(width, height, has_second_order, x["feat_prop"],
                                                    x["feat_current"], x["feat_n2"], x["flow1"], x["prev_flow"])
    h = cond
    for i, (ci, co) in enumerate([(196, 64), (64, 64), (64, 64)]):
        h = oracle.conv3x3_f16(ci, co, height, width, h, weights[f"offset_w{i}"], weights[f"offset_b{i}"], 1, 0.1)
    raw = oracle.conv3x3_f16(64, 432, height, width, h, weights["offset_w3"], weights["offset_b3"], 0, 0.1)
    off, msk = oracle.offset_transform_f16(plane, raw, x["flow1"], flow2)
    shape = oracle.OracleShape(1, 128, height, width, 64, height, width, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    aligned = f16(oracle.forward_f32_threads(shape, dinp.astype(np.float32), off.astype(np.float32),
                                             msk.astype(np.float32), weights["dcn_w"].astype(np.float32),
                                             weights["dcn_b"].astype(np.float32)))
    bb = np.concatenate([x["feat_current"], *x["prefix"], aligned])
    feat = oracle.conv3x3_f16(bb.size // plane, 64, height, width, bb, weights["backbone_w0"],
                              weights["backbone_b0"], 1, 0.1)
    for i in range(blocks):
        t = oracle.conv3x3_f16(64, 64, height, width, feat, weights[f"backbone_w{1 + 2 * i}"],
                               weights[f"backbone_b{1 + 2 * i}"], 2, 0.1)
        feat = oracle.conv3x3_f16(64, 64, height, width, t, weights[f"backbone_w{2 + 2 * i}"],
                                  weights[f"backbone_b{2 + 2 * i}"], 0, 0.1, feat)
    out = f16(aligned.astype(np.float32) + feat.astype(np.float32))
    return flow2, out, {"offset": off, "mask": msk, "aligned": aligned, "raw": raw, "conditions": cond,
                        "deform_input": dinp}


def backbone(weights: dict, bb: np.ndarray, height: int, width: int, blocks: int) -> np.ndarray:
    """Backbone of one step on the CPU: conv (LeakyReLU 0.1), then residual blocks."""
    plane = height * width
    feat = oracle.conv3x3_f16(bb.size // plane, 64, height, width, bb, weights["backbone_w0"],
                              weights["backbone_b0"], 1, 0.1)
    for i in range(blocks):
        t = oracle.conv3x3_f16(64, 64, height, width, feat, weights[f"backbone_w{1 + 2 * i}"],
                               weights[f"backbone_b{1 + 2 * i}"], 2, 0.1)
        feat = oracle.conv3x3_f16(64, 64, height, width, t, weights[f"backbone_w{2 + 2 * i}"],
                                  weights[f"backbone_b{2 + 2 * i}"], 0, 0.1, feat)
    return feat


def body_initial_step(weights: dict, feat_current, prefix, height: int, width: int, blocks: int) -> np.ndarray:
    """A branch's first step (FusedFourPassRecurrenceProbe.swift:528-566): backbone on
    [feat_current, prefix..., 0] and feat_prop = half(0 + backbone)."""
    zero = np.zeros(64 * height * width, np.float16)
    bb = np.concatenate([feat_current, *prefix, zero])
    feat = backbone(weights, bb, height, width, blocks)
    return f16(zero.astype(np.float32) + feat.astype(np.float32))


def to_cb8(x_nchw: np.ndarray, channels: int, height: int, width: int, pad: int = 2) -> np.ndarray:
    """NCHW FP16 -> CB8 [ceil(C/8)][H+2p][W+2p][8] with zero border and padding channels."""
    cb = (channels + 7) // 8
    full = np.zeros((cb * 8, height + 2 * pad, width + 2 * pad), np.float16)
    full[:channels, pad:pad + height, pad:pad + width] = np.asarray(x_nchw, np.float16).reshape(channels, height, width)
    return np.ascontiguousarray(full.reshape(cb, 8, height + 2 * pad, width + 2 * pad).transpose(0, 2, 3, 1))
