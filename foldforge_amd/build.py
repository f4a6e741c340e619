"""Build recipe of the native library: every ``csrc/*.hip`` into one gfx950 shared object.

``python -m foldforge_amd.build`` (or ``__graft_entry__.build()``) runs ``hipcc`` directly:
each source is compiled to an object in a temporary directory (in parallel, with the
per-file code-generation options below), then linked into
``foldforge_amd/libfoldforge_amd.so`` in-tree. No JIT cache is used: the built file
travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
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


# Kernels whose accumulators and operands together exceed 256 registers run one wave per
# SIMD with the 512-entry file; they keep MFMA results in VGPRs (values that are touched
# rarely go to the accumulation registers), which avoids copying accumulators between the
# two register files inside the hot loop.
PER_FILE_FLAGS = {
    "transition.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def compile_command(source: Path, obj: Path) -> list[str]:
    return [hipcc(), *COMMON, *PER_FILE_FLAGS.get(source.name, []), f"-I{INCLUDE}", f"-I{CSRC}",
            "-c", str(source), "-o", str(obj)]


def link_command(objects: list[Path], output: Path = LIBRARY) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(output)]


NOISE = "'-packed-fp32-ops' is not a recognized feature"


def _run(cmd: list[str]) -> tuple[int, str]:
    res = subprocess.run(cmd, capture_output=True, text=True)
    return res.returncode, "\n".join(l for l in res.stderr.splitlines() if NOISE not in l)


def build(verbose: bool = False) -> Path:
    """Compile the library (always: a stale build is never reused). Returns its path."""
    tmp = LIBRARY.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="ffk_build_") as work:
        srcs = sources()
        objs = [Path(work) / (src.stem + ".o") for src in srcs]
        cmds = [compile_command(src, obj) for src, obj in zip(srcs, objs)]
        if verbose:
            for cmd in cmds:
                print(" ".join(cmd), flush=True)
        with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
            results = list(pool.map(_run, cmds))
        for src, (rc, err) in zip(srcs, results):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {src.name} ({rc}):\n{err}")
            if verbose and err.strip():
                print(err, file=sys.stderr)
        rc, err = _run(link_command(objs, tmp))
        if rc != 0:
            raise RuntimeError(f"hipcc link failed ({rc}):\n{err}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
