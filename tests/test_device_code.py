"""Generated device code has no loop that can never exit.

Reading an indeterminate value on a control path is undefined behaviour, and the compiler
may lower the paths that depend on it to a block that branches to itself with nothing else
in it (an infinite loop: the waves that reach it never finish and the launch hangs). This
test compiles every HIP source to gfx950 assembly with the library's own flags and fails
on any such block. CPU only (hipcc cross-compiles).
"""
from __future__ import annotations

import concurrent.futures
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from jasnamacos_amd import build as dcn_build

LABEL = re.compile(r"^(\.LBB\d+_\d+):")
# Instructions that leave a self-branching block unable to exit: nothing but the branch
# and copies of its condition.
INERT = re.compile(r"^s_mov_b64\s+vcc,\s*vcc$")


def self_loops(asm: str) -> list[str]:
    """Labels of blocks that consist of only a branch back to themselves."""
    lines = asm.splitlines()
    found = []
    for i, line in enumerate(lines):
        m = LABEL.match(line)
        if not m:
            continue
        label = m.group(1)
        body = []
        for nxt in lines[i + 1:]:
            t = nxt.split(";")[0].strip()
            if not t:
                continue
            body.append(t)
            if t.startswith(("s_branch", "s_cbranch")) or LABEL.match(t):
                break
        if body and re.match(rf"^s_c?branch\w*\s+{re.escape(label)}$", body[-1]) and all(
                INERT.match(t) for t in body[:-1]):
            found.append(label)
    return found


def test_self_loop_detector():
    looping = ".LBB0_3:\n\ts_mov_b64 vcc, vcc\n\ts_cbranch_vccz .LBB0_3\n"
    working = ".LBB0_3:\n\tv_add_u32_e32 v1, 1, v1\n\ts_cbranch_scc1 .LBB0_3\n"
    assert self_loops(looping) == [".LBB0_3"]
    assert self_loops(working) == []
    assert self_loops(".LBB1_7:\n\ts_branch .LBB1_7\n") == [".LBB1_7"]


def _device_asm(src: Path, out: Path) -> str:
    cmd = [dcn_build.HIPCC, "-x", "hip", *dcn_build.DEVICE, *dcn_build.COMMON, "--cuda-device-only",
           "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return out.read_text()


@pytest.mark.skipif(not Path(dcn_build.HIPCC).exists() and shutil.which("hipcc") is None,
                    reason="needs hipcc")
def test_no_infinite_loops_in_device_code(tmp_path):
    srcs = sorted(dcn_build.CSRC.glob("*.hip"))
    assert srcs
    with concurrent.futures.ThreadPoolExecutor(max_workers=8) as pool:
        asms = list(pool.map(lambda s: _device_asm(s, tmp_path / (s.name + ".s")), srcs))
    bad = {s.name: self_loops(a) for s, a in zip(srcs, asms) if self_loops(a)}
    assert not bad, f"blocks that branch only to themselves: {bad}"
