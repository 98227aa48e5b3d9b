"""Instruction rates of gfx950 that the edge kernels are designed around.

``python -m pymolecular_amd.benchmarks.isa_rates`` compiles ``isa_rates.hip``
with hipcc (into ``_build/`` next to this file) and runs it on the current GPU:
one JSON line per measurement, cycles per wave-instruction per SIMD for the
vector ALU (1, 2 and 4 waves per SIMD) and the bf16 MFMA (dependent chains, mixed
with fp32 adds), and bytes per cycle per CU for LDS reads and writes.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def build() -> Path:
    out = HERE / "_build" / "isa_rates"
    out.parent.mkdir(exist_ok=True)
    src = HERE / "isa_rates.hip"
    if not out.exists() or out.stat().st_mtime < src.stat().st_mtime:
        cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Wno-unused-result",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-o", str(out), str(src)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + r.stderr)
    return out


def main() -> int:
    exe = build()
    return subprocess.run([str(exe)]).returncode


if __name__ == "__main__":
    sys.exit(main())
