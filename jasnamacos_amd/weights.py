"""`.dcnfp16` weight sets: export, manifest and validation.

Format (DeformConvWeights.swift:4-21, tools/export_deform_weights.py:43-50): one file
per propagation direction, 73,728 little-endian FP16 weights in [ic=128][k=9][oc=64]
order followed by 64 FP16 biases, 147,584 bytes. The exporter writes a manifest.json
beside the files (format tag, layout text, per-direction file name, byte count,
element counts and sha256; tools/export_deform_weights.py:35-62).

Validation mirrors `--validate-deform-weights` (JasnaCLI.swift:1407-1426): every
direction loads with the size check of DeformConvWeightSet.init, and its checksum is
the double sum of the file's FP16 values at indices 0, 257, 514, ... When a manifest is
present its sizes and sha256 digests must match too.

    python -m jasnamacos_amd.weights --validate-deform-weights DIR
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

DIRECTIONS = ("backward_1", "forward_1", "backward_2", "forward_2")
FORMAT = "jasna-metal-dcnv2-fp16-v1"
LAYOUT = "weight[input_channel,kernel_element,output_channel], then bias[output_channel]"
WEIGHT_ELEMENTS = 128 * 9 * 64
BIAS_ELEMENTS = 64
EXPECTED_BYTES = (WEIGHT_ELEMENTS + BIAS_ELEMENTS) * 2


class WeightSetError(Exception):
    """A weight file or manifest that does not match the format (the reference's
    DeformConvError.commandFailed)."""


def pack_payload(weight_oihw, bias) -> bytes:
    """OIHW [64][128][3][3] + bias [64] -> the .dcnfp16 byte payload."""
    w = np.asarray(weight_oihw, np.float16)
    b = np.asarray(bias, np.float16)
    if w.shape != (64, 128, 3, 3) or b.shape != (64,):
        raise WeightSetError(f"unexpected shapes: {w.shape}, {b.shape}")
    packed = np.ascontiguousarray(np.transpose(w.reshape(64, 128, 9), (1, 2, 0))).astype("<f2")
    return packed.tobytes(order="C") + b.astype("<f2").tobytes(order="C")


def export_weight_sets(directory, sets: dict) -> dict:
    """Write <direction>.dcnfp16 for each (weight_oihw, bias) in `sets` and manifest.json."""
    out = Path(directory)
    out.mkdir(parents=True, exist_ok=True)
    manifest = {"format": FORMAT, "layout": LAYOUT, "directions": {}}
    for direction in DIRECTIONS:
        if direction not in sets:
            continue
        payload = pack_payload(*sets[direction])
        path = out / f"{direction}.dcnfp16"
        path.write_bytes(payload)
        manifest["directions"][direction] = {
            "file": path.name,
            "bytes": len(payload),
            "weight_elements": WEIGHT_ELEMENTS,
            "bias_elements": BIAS_ELEMENTS,
            "sha256": hashlib.sha256(payload).hexdigest(),
        }
    (out / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def read_weight_set(path) -> bytes:
    """DeformConvWeightSet.init (DeformConvWeights.swift:11-21): the size check."""
    p = Path(path)
    data = p.read_bytes()
    if len(data) != EXPECTED_BYTES:
        raise WeightSetError(f"{p.name} has {len(data)} bytes; expected {EXPECTED_BYTES}")
    return data


def weight_set_checksum(data: bytes) -> float:
    """Double sum of FP16 values 0, 257, 514, ... of the whole file (JasnaCLI.swift:1415-1421)."""
    values = np.frombuffer(data, dtype="<f2")
    return float(np.sum(values[::257].astype(np.float64)))


def unpack_weight_set(data: bytes):
    """Payload -> (weight [ic][k][oc] FP16, bias [oc] FP16)."""
    values = np.frombuffer(data, dtype="<f2")
    return values[:WEIGHT_ELEMENTS].reshape(128, 9, 64), values[WEIGHT_ELEMENTS:]


def validate_weight_sets(directory) -> list[dict]:
    """Load and check every direction; verify manifest.json when it exists."""
    d = Path(directory)
    manifest = None
    mpath = d / "manifest.json"
    if mpath.exists():
        manifest = json.loads(mpath.read_text())
        if manifest.get("format") != FORMAT:
            raise WeightSetError(f"manifest format {manifest.get('format')!r}; expected {FORMAT!r}")
    results = []
    for direction in DIRECTIONS:
        path = d / f"{direction}.dcnfp16"
        data = read_weight_set(path)
        digest = hashlib.sha256(data).hexdigest()
        if manifest is not None:
            entry = manifest.get("directions", {}).get(direction)
            if entry is None:
                raise WeightSetError(f"manifest has no entry for {direction}")
            if entry.get("file") != path.name or entry.get("bytes") != len(data):
                raise WeightSetError(f"manifest entry for {direction} does not describe {path.name}")
            if entry.get("sha256") != digest:
                raise WeightSetError(f"{path.name}: sha256 {digest} does not match the manifest")
        results.append({"direction": direction, "bytes": len(data), "checksum": weight_set_checksum(data),
                        "sha256": digest})
    return results


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--validate-deform-weights", metavar="DIR", required=True)
    args = ap.parse_args(argv)
    try:
        results = validate_weight_sets(args.validate_deform_weights)
    except (WeightSetError, OSError) as e:
        print(f"Jasna DCNv2 checkpoint weights: FAIL ({e})", file=sys.stderr)
        return 1
    print("Jasna DCNv2 checkpoint weights: PASS")
    for r in results:
        print(f"{r['direction']}: {r['bytes']} bytes, checksum {r['checksum']:.6f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
