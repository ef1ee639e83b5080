"""bench.py's contract on a machine without a GPU: more than one GPU is refused with a
message (this build measures one GPU), before anything touches a device."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_bench_rejects_zero_steps():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--steps", "0"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2


def test_bench_seed_sweep_rejects_other_configs():
    """--seed-sweep covers the fused configs 2, 3 and 5; other configs are refused before
    any child process starts."""
    for extra in (["--config", "4"], ["--config", "1"], ["--spynet"]):
        r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--seed-sweep", "2", *extra],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 2, extra
        assert "--seed-sweep" in r.stderr
        assert r.stdout.strip() == ""
