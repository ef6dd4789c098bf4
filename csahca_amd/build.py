"""Build libcsahca.so (gfx950) in-tree with hipcc.

    python -m csahca_amd.build          # compile every source, link the library
    python -m csahca_amd.build --sanitized   # also the host-sanitized variant

Each HIP source compiles to an object under csahca_amd/_build/ and the objects
link into csahca_amd/libcsahca.so, which csahca_amd.native loads with ctypes.
Beside it: libcsahca_timeline.so (the decode step with phase stamps) and, on
request, csahca_amd/_build/asan/libcsahca_asan.so -- the same sources with
AddressSanitizer and UndefinedBehaviorSanitizer on the host side only (the
argument checks, workspace sizing and launch set-up of every entry point; the
device code is compiled as usual), for the CPU ABI tests
(tests/test_abi_sanitized.py), which load it through CSAHCA_LIBRARY with the
ASan runtime preloaded.
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
ASAN_BUILD = BUILD / "asan"
LIB_ASAN = ASAN_BUILD / "libcsahca_asan.so"
# Host-side sanitizers only: each -fsanitize= applies to the host compilation
# (-Xarch_host), the device code objects are the product's.
SANITIZE_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=undefined"]

COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # No packed fp32 instructions anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}", f"-I{SRC}",
]


# Per-source device flags.  csa_step.hip: the decode step's leading scalar
# parameters (the StepLead fields: 8 arguments, 14 dwords) are preloaded into
# SGPRs at wave launch, so its first loads need no argument load.  (Kernels
# whose first parameter is a struct are unaffected: preloading stops there.)
SOURCE_FLAGS = {
    "csa_step.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
    "dsv4.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
    "block.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
    "csa.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "hca.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _link(cc: str, objs, out: Path, verbose: bool, extra=()) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, "-shared", "-o", str(tmp)] + [str(o) for o in objs] + [f"--offload-arch={ARCH}"] + list(extra)
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def _compile(cc: str, units, verbose: bool, jobs: int) -> None:
    """Run the hipcc compile commands of `units` (name, source, object, extra
    flags), at most `jobs` at a time; raise with the output of any failure."""
    pending = list(units)
    running, failed = [], []
    while pending or running:
        while pending and len(running) < jobs:
            name, src, obj, extra = pending.pop(0)
            obj.parent.mkdir(parents=True, exist_ok=True)
            cmd = [cc, "-x", "hip", "-c", str(src), "-o", str(obj)] + COMMON_FLAGS + extra
            if verbose:
                print(" ".join(cmd), flush=True)
            running.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                                   text=True)))
        name, p = running.pop(0)
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append((name, out))
        elif verbose and out.strip():
            print(out)
    if failed:
        msg = "\n".join(f"--- {n} ---\n{o}" for n, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")


def build(verbose: bool = False, jobs: int | None = None, sanitized: bool = False) -> Path:
    """Compile all sources (always) and link the shared library, and beside it
    the phase-timeline variant (the decode step built with its stamps); with
    `sanitized`, also the host-sanitized variant (LIB_ASAN)."""
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or max(1, min(16, os.cpu_count() or 1))
    objs = []
    units = [(name, SRC / name, BUILD / (name.rsplit(".", 1)[0] + ".o"), list(SOURCE_FLAGS.get(name, [])))
             for name in SOURCES]
    objs = [u[2] for u in units]
    tl_obj = BUILD / "csa_step_timeline.o"
    units.append((TIMELINE_SOURCE + " (timeline)", SRC / TIMELINE_SOURCE, tl_obj,
                  ["-DCSAHCA_STEP_TIMELINE"] + SOURCE_FLAGS.get(TIMELINE_SOURCE, [])))
    asan_objs = [ASAN_BUILD / (name.rsplit(".", 1)[0] + ".o") for name in SOURCES]
    if sanitized:
        units += [(name + " (sanitized)", SRC / name, obj,
                   ["-Xarch_host", "-O1", "-Xarch_host", "-g"] + SANITIZE_FLAGS + SOURCE_FLAGS.get(name, []))
                  for name, obj in zip(SOURCES, asan_objs)]
    _compile(cc, units, verbose, jobs)
    _link(cc, objs, LIB, verbose)
    step_obj = BUILD / (TIMELINE_SOURCE.rsplit(".", 1)[0] + ".o")
    _link(cc, [tl_obj if o == step_obj else o for o in objs], LIB_TIMELINE, verbose)
    if sanitized:
        _link(cc, asan_objs, LIB_ASAN, verbose, SANITIZE_FLAGS)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, sanitized="--sanitized" in sys.argv))
