"""Consistency of the SwiftPM binding (jasnamacos_amd/swift) with the C ABI.

No Swift toolchain is installed here, so the package is checked structurally: the module
map's umbrella header resolves to include/dcn/dcn.h and compiles as C, every libdcn
function the Swift sources call is declared there and exported by the library, and every
dcn_status and layout constant they name exists."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "jasnamacos_amd" / "swift"
HEADER = ROOT / "include" / "dcn" / "dcn.h"


def swift_sources() -> str:
    return "\n".join(p.read_text() for p in sorted((PKG / "Sources").rglob("*.swift")))


def test_package_layout():
    for rel in ("Package.swift", "Sources/CDCN/module.modulemap", "Sources/CDCN/shim.h",
                "Sources/HIPDeformConv/HIPDeformConv.swift", "Sources/HIPDeformConv/ReferenceInterface.swift",
                "Sources/dcn-self-test/main.swift"):
        assert (PKG / rel).is_file(), rel
    mm = (PKG / "Sources/CDCN/module.modulemap").read_text()
    assert 'header "shim.h"' in mm and 'link "dcn"' in mm
    manifest = (PKG / "Package.swift").read_text()
    for target in ('.systemLibrary(name: "CDCN"', 'name: "HIPDeformConv"', 'name: "dcn-self-test"'):
        assert target in manifest


def test_umbrella_header_resolves_and_compiles(tmp_path):
    shim = PKG / "Sources" / "CDCN" / "shim.h"
    inc = re.search(r'#include "([^"]+)"', shim.read_text()).group(1)
    assert (shim.parent / inc).resolve() == HEADER.resolve()
    src = tmp_path / "t.c"
    src.write_text(f'#include "{shim}"\nint main(void) {{ return (int)sizeof(dcn_shape); }}\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", str(src)], check=True)


def test_called_functions_are_declared_and_exported(dcn):
    header = HEADER.read_text()
    called = set(re.findall(r"\b(dcn_[a-z0-9_]+)\(", swift_sources())) - {"dcn_shape"}
    assert called, "no libdcn calls found"
    lib = dcn.lib()
    for name in sorted(called):
        assert re.search(rf"\b{name}\s*\(", header), f"{name} not declared in dcn.h"
        assert hasattr(lib, name), f"{name} not exported by libdcn"


def test_named_constants_exist():
    header = HEADER.read_text()
    names = set(re.findall(r"\b(DCN_[A-Z0-9_]+)\b", swift_sources()))
    assert {"DCN_OK", "DCN_INVALID_ARRAY_COUNT", "DCN_NONFINITE_OUTPUT"} <= names
    for name in names:
        assert re.search(rf"\b{name}\b", header), name


def test_array_count_message_parses_as_the_swift_side_expects():
    """HIPDeformConv splits dcn_last_error on spaces and reads parts 0, 2 and 5: the C side
    must keep building "<name> has <actual> elements; expected <expected>"."""
    src = (ROOT / "jasnamacos_amd" / "csrc" / "dcn_host.hpp").read_text()
    assert 'std::string(name) + " has " + std::to_string(actual) +' in src
    assert '" elements; expected " + std::to_string(expected)' in src
    parts = "offset has 3 elements; expected 4".split(" ")
    assert (parts[0], parts[2], parts[5]) == ("offset", "3", "4") and len(parts) == 6
    assert "parts.count == 6, let actual = Int(parts[2]), let expected = Int(parts[5])" in swift_sources()
