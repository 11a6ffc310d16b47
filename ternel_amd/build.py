"""Build the gfx950 shared library ``ternel_amd/_lib/libternel_tq1.so`` in-tree.

``python -m ternel_amd.build`` (or ``__graft_entry__.build()``) cross-compiles
on a machine without a GPU; the built library travels with the tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
SOURCE = PACKAGE_DIR / "csrc" / "tq1_engine.hip"
INCLUDE_DIR = REPO_ROOT / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libternel_tq1.so"
# measurement-only streaming probe (bench.py --stream-ceiling); not part of the C ABI
PROBE_SOURCE = PACKAGE_DIR / "csrc" / "stream_probe.hip"
PROBE_PATH = LIB_DIR / "libternel_probe.so"
# the same engine source with phase timestamps in the M=1 GEMV (bench.py --phase-profile)
PROFILE_PATH = LIB_DIR / "libternel_tq1_profile.so"
ARCH = "gfx950"

# Packed fp32 instructions are disabled for every HIP translation unit: some of
# their forms have given silently wrong results on these machines.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # Kernel arguments arrive in SGPRs at wave launch (with a load fallback in
    # the code object where the firmware does not preload): a workgroup that
    # starts while earlier ones flood HBM does not wait for its argument loads
    # behind their weight traffic (gate/up M=1 GEMV 10.35 -> 9.93 us on MI355X).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # a kernel whose host launch stub was not emitted must fail the build, not the load
    "-Wl,--no-undefined",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the TQ1 engine needs ROCm's hipcc to build")
    return found


def _command(source: Path, target: Path, extra: list[str]) -> list[str]:
    return [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE_DIR}", str(source), "-o", str(target.with_suffix(".so.tmp"))]


def build(verbose: bool = False) -> Path:
    """Compile the engine library, its phase-profile variant and the streaming
    probe, in parallel (always recompiles); return the engine library's path."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    jobs = [(SOURCE, LIB_PATH, []), (PROBE_SOURCE, PROBE_PATH, []),
            (SOURCE, PROFILE_PATH, ["-DTERNEL_TQ1_PROFILE"])]
    running = []
    for source, target, extra in jobs:
        cmd = _command(source, target, extra)
        if verbose:
            print(" ".join(cmd), flush=True)
        running.append((target, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                                                  env=dict(os.environ))))
    failures = []
    for target, proc in running:
        out, err = proc.communicate()
        if proc.returncode != 0:
            failures.append(f"{target.name}: hipcc failed ({proc.returncode}):\n{out}\n{err}")
    if failures:
        for target, _ in running:
            target.with_suffix(".so.tmp").unlink(missing_ok=True)
        raise RuntimeError("\n".join(failures))
    for target, _ in running:
        os.replace(target.with_suffix(".so.tmp"), target)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
