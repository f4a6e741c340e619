"""Build recipe of the native library: every ``csrc/*.hip`` into one gfx950 shared object.

``python -m foldforge_amd.build`` (or ``__graft_entry__.build()``) runs ``hipcc`` directly
and writes ``foldforge_amd/libfoldforge_amd.so`` in-tree. No JIT cache is used: the
built file travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
LIBRARY = PACKAGE / "libfoldforge_amd.so"
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError(f"hipcc not found (looked on PATH and in {rocm}/bin)")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def command(output: Path = LIBRARY) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-shared",
        "-fPIC",
        # packed fp32 VALU forms are kept out of every kernel
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        *map(str, sources()),
        "-o", str(output),
    ]


def build(verbose: bool = False) -> Path:
    """Compile the library (always: a stale build is never reused). Returns its path."""
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    stderr = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
