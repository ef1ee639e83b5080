"""`.dcnfp16` export / manifest / validation (CPU)."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from jasnamacos_amd import weights as W


def _sets(seed=3):
    rng = np.random.default_rng(seed)
    return {d: (rng.normal(0, 0.05, (64, 128, 3, 3)).astype(np.float16), rng.normal(0, 0.1, 64).astype(np.float16))
            for d in W.DIRECTIONS}


def _checksum_by_hand(data: bytes) -> float:
    # independent restatement: unpack every 257th little-endian binary16 with struct
    total = 0.0
    for i in range(0, len(data) // 2, 257):
        total += struct.unpack_from("<e", data, 2 * i)[0]
    return total


def test_export_validate_roundtrip(tmp_path, dcn):
    sets = _sets()
    manifest = W.export_weight_sets(tmp_path, sets)
    assert manifest["format"] == W.FORMAT
    results = W.validate_weight_sets(tmp_path)
    assert [r["direction"] for r in results] == list(W.DIRECTIONS)
    for r in results:
        data = (tmp_path / f"{r['direction']}.dcnfp16").read_bytes()
        assert r["bytes"] == 147584 == dcn.lib().dcn_dcnfp16_bytes()
        assert r["checksum"] == pytest.approx(_checksum_by_hand(data), abs=0, rel=1e-15)
        assert r["checksum"] == dcn.checksum(np.frombuffer(data, np.uint16))
        w, b = W.unpack_weight_set(data)
        ow, ob = sets[r["direction"]]
        assert np.array_equal(w, np.transpose(ow.reshape(64, 128, 9), (1, 2, 0)))
        assert np.array_equal(w.ravel(), dcn.pack_ic_k_oc(ow, dcn.JASNA_SHAPE).ravel())
        assert np.array_equal(b, ob)


def test_size_error_message(tmp_path):
    W.export_weight_sets(tmp_path, _sets())
    p = tmp_path / "forward_1.dcnfp16"
    p.write_bytes(p.read_bytes()[:-2])
    with pytest.raises(W.WeightSetError, match=r"forward_1.dcnfp16 has 147582 bytes; expected 147584"):
        W.validate_weight_sets(tmp_path)


def test_sha256_mismatch_is_caught(tmp_path):
    W.export_weight_sets(tmp_path, _sets())
    p = tmp_path / "backward_2.dcnfp16"
    data = bytearray(p.read_bytes())
    data[1000] ^= 0x01
    p.write_bytes(bytes(data))
    with pytest.raises(W.WeightSetError, match="sha256"):
        W.validate_weight_sets(tmp_path)


def test_manifest_format_and_entries(tmp_path):
    W.export_weight_sets(tmp_path, _sets())
    m = json.loads((tmp_path / "manifest.json").read_text())
    del m["directions"]["forward_2"]
    (tmp_path / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(W.WeightSetError, match="no entry for forward_2"):
        W.validate_weight_sets(tmp_path)
    m["format"] = "other"
    (tmp_path / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(W.WeightSetError, match="format"):
        W.validate_weight_sets(tmp_path)


def test_without_manifest_only_sizes_are_checked(tmp_path):
    W.export_weight_sets(tmp_path, _sets())
    (tmp_path / "manifest.json").unlink()
    assert len(W.validate_weight_sets(tmp_path)) == 4


def test_cli(tmp_path, capsys):
    W.export_weight_sets(tmp_path, _sets())
    assert W.main(["--validate-deform-weights", str(tmp_path)]) == 0
    out = capsys.readouterr().out.splitlines()
    assert out[0] == "Jasna DCNv2 checkpoint weights: PASS"
    assert out[1].startswith("backward_1: 147584 bytes, checksum ")
    (tmp_path / "forward_1.dcnfp16").unlink()
    assert W.main(["--validate-deform-weights", str(tmp_path)]) == 1


def test_wrong_shapes_rejected():
    with pytest.raises(W.WeightSetError):
        W.pack_payload(np.zeros((64, 64, 3, 3), np.float16), np.zeros(64, np.float16))
