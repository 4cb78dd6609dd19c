"""bench.py's command line without a GPU: the script compiles, documents its
flags, and refuses more than one GPU with exit status 2 and a message (the
path has no cross-GPU exchange; the measured figure is one GPU's)."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, cwd=ROOT)


def test_bench_help_lists_the_contract_flags():
    r = _run("--help")
    assert r.returncode == 0, r.stderr
    for flag in ("--gpus", "--steps", "--warmup", "--settle-ms"):
        assert flag in r.stdout


def test_bench_refuses_more_than_one_gpu():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
