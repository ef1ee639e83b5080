"""CPU references of SPyNet flow estimation — test infrastructure.

`spynet_flow` chains the oracle's pinned pieces in the reference's order (pyramid,
per-level prepare, the basic module's 7x7 convs, flow add: MetalShader.swift:523-649,
levels coarsest first as tools/convert_basicvsrpp.py:82-100), every tensor rounded to
FP16 between layers like the reference's FP16 Metal graph. `torch_spynet` restates the
trace-friendly SPyNet forward (tools/convert_basicvsrpp.py:40-100: avg-pool pyramid,
grid_sample warp with border padding and align_corners, bilinear x2 flow upsampling) in
float32 torch on the CPU, the independent check of the chain.
"""
from __future__ import annotations

import numpy as np

import oracle

LEVELS = 6
LAYERS = [(8, 32), (32, 64), (64, 32), (32, 16), (16, 2)]
MEAN = (0.485, 0.456, 0.406)
STD = (0.229, 0.224, 0.225)


def f16(a) -> np.ndarray:
    return np.asarray(a, np.float32).astype(np.float16)


def spynet_weights(rng: np.random.Generator, last_std: float = 0.04) -> dict:
    """Random-init basic modules: He-normal 7x7 weights (std sqrt(2 / (cin * 49))) for the
    ReLU layers, N(0, last_std) for the flow layer, biases N(0, 0.01); FP16 OIHW."""
    w = {}
    for level in range(LEVELS):
        for i, (ci, co) in enumerate(LAYERS):
            std = last_std if i == len(LAYERS) - 1 else np.sqrt(2.0 / (ci * 49))
            w[f"w{level}_{i}"] = f16(rng.normal(0, std, (co, ci, 7, 7)))
            w[f"b{level}_{i}"] = f16(rng.normal(0, 0.01, co))
    return w


def smooth_frame(rng: np.random.Generator, height: int, width: int, shift=(0.0, 0.0)) -> np.ndarray:
    """An RGB frame in [0, 1] of a few random sinusoids (optionally shifted by (dy, dx) px)."""
    y, x = np.meshgrid(np.arange(height, dtype=np.float64) + shift[0],
                       np.arange(width, dtype=np.float64) + shift[1], indexing="ij")
    out = np.empty((3, height, width))
    for c in range(3):
        acc = np.zeros_like(y)
        for _ in range(4):
            fy, fx = rng.uniform(-0.3, 0.3, 2)
            acc += rng.uniform(0.2, 1.0) * np.sin(fy * y + fx * x + rng.uniform(0, 2 * np.pi))
        out[c] = 0.5 + 0.12 * acc
    return f16(np.clip(out, 0.0, 1.0).ravel())


def spynet_flow(weights: dict, reference, support, height: int, width: int):
    """flow [2][h][w] = spynet(reference, support), FP16 like the reference's graph."""
    rp = oracle.spynet_pyramid_f16(height, width, LEVELS, reference)
    sp = oracle.spynet_pyramid_f16(height, width, LEVELS, support)
    flow, fh, fw = None, 1, 1
    for level in range(LEVELS):
        h, w = height >> (LEVELS - 1 - level), width >> (LEVELS - 1 - level)
        x, base = oracle.spynet_prepare_f16(w, h, level == 0, rp[level], sp[level], flow, fw, fh)
        for i, (ci, co) in enumerate(LAYERS):
            x = oracle.convk_f16(7, ci, co, h, w, x, weights[f"w{level}_{i}"], weights[f"b{level}_{i}"],
                                 2 if i < len(LAYERS) - 1 else 0)
        flow, fh, fw = oracle.add_f16(base, x), h, w
    return flow


def torch_spynet(weights: dict, reference, support, height: int, width: int):
    """float32 torch restatement of the trace-friendly SPyNet forward."""
    import torch
    import torch.nn.functional as F

    def t(a, *shape):
        return torch.from_numpy(np.asarray(a, np.float32).reshape(shape))

    mean = torch.tensor(MEAN).view(1, 3, 1, 1)
    std = torch.tensor(STD).view(1, 3, 1, 1)
    r = [(t(reference, 1, 3, height, width) - mean) / std]
    s = [(t(support, 1, 3, height, width) - mean) / std]
    for _ in range(LEVELS - 1):
        r.insert(0, F.avg_pool2d(r[0], 2, 2))
        s.insert(0, F.avg_pool2d(s[0], 2, 2))

    def block(level, x):
        for i, (ci, co) in enumerate(LAYERS):
            x = F.conv2d(x, t(weights[f"w{level}_{i}"], co, ci, 7, 7), t(weights[f"b{level}_{i}"], co), padding=3)
            if i < len(LAYERS) - 1:
                x = F.relu(x)
        return x

    def warp(x, flow):
        n, _, h, w = x.shape
        gy, gx = torch.meshgrid(torch.arange(h, dtype=torch.float32), torch.arange(w, dtype=torch.float32),
                                indexing="ij")
        px = gx + flow[:, 0]
        py = gy + flow[:, 1]
        grid = torch.stack((2.0 * px / max(w - 1, 1) - 1.0, 2.0 * py / max(h - 1, 1) - 1.0), dim=-1)
        return F.grid_sample(x, grid, mode="bilinear", padding_mode="border", align_corners=True)

    flow = torch.zeros(1, 2, r[0].shape[2], r[0].shape[3])
    with torch.no_grad():
        for level in range(LEVELS):
            if level > 0:
                flow = F.interpolate(flow, scale_factor=2, mode="bilinear", align_corners=True) * 2.0
            flow = flow + block(level, torch.cat((r[level], warp(s[level], flow), flow), dim=1))
    return flow.numpy().ravel()
