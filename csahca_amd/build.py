"""Build libcsahca.so (gfx950) in-tree with hipcc.

    python -m csahca_amd.build          # compile every source, link the library

Each HIP source compiles to an object under csahca_amd/_build/ and the objects
link into csahca_amd/libcsahca.so, which csahca_amd.native loads with ctypes.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libcsahca.so"
# The same library with the decode step's phase stamps (csahca_amd/timeline.py).
LIB_TIMELINE = PKG / "libcsahca_timeline.so"
TIMELINE_SOURCE = "csa_step.hip"
ARCH = os.environ.get("CSAHCA_OFFLOAD_ARCH", "gfx950")

SOURCES = ["status.cpp", "csa.hip", "csa_step.hip", "dsv4.hip", "dsv4_pack.hip", "hca.hip", "block.hip"]

COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # No packed fp32 instructions anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}", f"-I{SRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _link(cc: str, objs, out: Path, verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, "-shared", "-o", str(tmp)] + [str(o) for o in objs] + [f"--offload-arch={ARCH}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources (always) and link the shared library, and beside it
    the phase-timeline variant (the decode step built with its stamps)."""
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    procs = []
    objs = []
    units = [(name, SRC / name, BUILD / (name.rsplit(".", 1)[0] + ".o"), []) for name in SOURCES]
    tl_obj = BUILD / "csa_step_timeline.o"
    units.append((TIMELINE_SOURCE + " (timeline)", SRC / TIMELINE_SOURCE, tl_obj, ["-DCSAHCA_STEP_TIMELINE"]))
    for name, src, obj, extra in units:
        if not extra:
            objs.append(obj)
        cmd = [cc, "-x", "hip", "-c", str(src), "-o", str(obj)] + COMMON_FLAGS + extra
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for name, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append((name, out))
        elif verbose and out.strip():
            print(out)
    if failed:
        msg = "\n".join(f"--- {n} ---\n{o}" for n, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    _link(cc, objs, LIB, verbose)
    step_obj = BUILD / (TIMELINE_SOURCE.rsplit(".", 1)[0] + ".o")
    _link(cc, [tl_obj if o == step_obj else o for o in objs], LIB_TIMELINE, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
