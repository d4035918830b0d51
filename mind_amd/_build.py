"""Build the gfx950 HIP library ``mind_amd/lib/libesa_hip.so``.

Each ``csrc/*.hip`` file is compiled to an object with ``hipcc
--offload-arch=gfx950`` (in parallel), then linked into one shared library
whose only exported symbols are the ``extern "C"`` entry points declared in
``include/esa_hip.h``.  Objects go to ``mind_amd/_build/`` and stay out of
version control; the ``.so`` is built in-tree so it travels with the
repository snapshot to a GPU box.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libesa_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
# Packed fp32 VALU ops (v_pk_*_f32) are disabled for all device code: some of
# their forms have given wrong results on the target machines.  The host pass
# warns that it does not know the feature; that is harmless.
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs (no AGPR copies around the softmax).
    "-mllvm", "-amdgpu-mfma-vgpr-form=true",
    "-fvisibility=hidden",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MI355X library cannot be built")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPFLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        msg = "\n".join(line for line in proc.stderr.splitlines() if "packed-fp32-ops" not in line)
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link ``libesa_hip.so``.  Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {LIB.name} failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[mind_amd] built {LIB} from {len(sources)} HIP sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
