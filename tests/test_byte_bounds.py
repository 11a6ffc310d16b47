"""Exhaustive CPU check that the kernels' byte arithmetic is memory-safe and
exact: builds tests/byte_bounds.cpp against ternel_amd/csrc/tq1_bytes.h (the
header the kernels include) with the host C++ compiler and runs it over all
256 byte values. Illegal bytes (codes > 242, tail > 26) reach these functions
whenever unvalidated words are multiplied; the reference guards the same case
with its SAFE clamp build (src/ternel_mlx/kernels.py:305,316,635-638)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def checker(tmp_path_factory) -> Path:
    compiler = shutil.which("g++")
    if compiler is None:
        pytest.skip("no host C++ compiler")
    target = tmp_path_factory.mktemp("byte_bounds") / "byte_bounds"
    subprocess.run([compiler, "-std=c++17", "-O1", "-Wall", "-Werror", "-Wno-unknown-pragmas",
                    "-D__host__=", "-D__device__=", f"-I{ROOT / 'ternel_amd' / 'csrc'}",
                    str(ROOT / "tests" / "byte_bounds.cpp"), "-o", str(target)],
                   check=True, capture_output=True, text=True)
    return target


def test_every_byte_value_stays_in_bounds(checker: Path) -> None:
    result = subprocess.run([str(checker)], capture_output=True, text=True, timeout=60)
    assert result.returncode == 0, result.stdout + result.stderr
    lines = result.stdout.splitlines()
    assert lines[-1] == "ok"
    # the bounds the kernels rely on, as measured over all 256 values
    assert "high <= 28, low <= 8" in lines[0]
