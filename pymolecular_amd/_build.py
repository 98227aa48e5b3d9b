"""Build recipe for the HIP library ``libpymolecular_egnn.so`` (gfx950).

Each ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` in
parallel and linked into one shared library next to this file, so that it
travels with the source tree.  ``python -m pymolecular_amd._build`` runs it.

Next to the library the build writes ``libpymolecular_egnn.so.srchash``: a
SHA-256 over the sources it was built from (``csrc/``, ``include/egnn.h``)
and the compiler flags.  ``_capi.lib()`` recomputes it and refuses a library
built from other sources, so a run always exercises the current tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
HEADER = PKG.parent / "include" / "egnn.h"
LIB = PKG / "libpymolecular_egnn.so"
STAMP = LIB.with_name(LIB.name + ".srchash")
OBJ = PKG / "_objs"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 VALU forms are kept out of all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# per-file flags: the edge-parallel MPNN backward keeps its MFMA accumulators in VGPRs (the VALU reads
# every product's result; the AGPR form would copy each one back)
FILE_FLAGS = {
    "egnn_mpnn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "egnn_eqfwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def source_files() -> list:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + [HEADER]


def source_hash() -> str:
    """SHA-256 over the flags and the (relative name, content) of every source file."""
    h = hashlib.sha256()
    h.update("\0".join(FLAGS).encode())
    for name in sorted(FILE_FLAGS):
        h.update(("\0" + name + "\0" + "\0".join(FILE_FLAGS[name])).encode())
    for p in source_files():
        h.update(b"\0" + p.name.encode() + b"\0")
        h.update(p.read_bytes())
    return h.hexdigest()


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(l for l in r.stderr.splitlines() if "not a recognized feature" not in l)
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    return obj


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    digest = source_hash()
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    if STAMP.exists():
        STAMP.unlink()
    os.replace(tmp, LIB)
    STAMP.write_text(digest + "\n")
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources (sources sha256 {digest[:16]})")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
