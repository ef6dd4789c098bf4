"""The CPU ABI tests (tests/test_abi_cpu.py) rerun against the host-sanitized
build of the library (csahca_amd/_build/asan/libcsahca_asan.so: the same
sources with AddressSanitizer and UndefinedBehaviorSanitizer on the host side,
built by `python -m csahca_amd.build --sanitized` and by __graft_entry__.build),
loaded through CSAHCA_LIBRARY with the ASan runtime preloaded: the argument
checks, workspace sizing and error paths of every entry point run with no
sanitizer report."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_abi_tests_pass_under_address_and_undefined_behavior_sanitizers():
    from csahca_amd import build

    if not build.LIB_ASAN.exists():
        pytest.skip("the sanitized library is not built (python -m csahca_amd.build --sanitized)")
    rt = subprocess.run([build.hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                        text=True).stdout.strip()
    if not rt or not Path(rt).exists():
        pytest.skip("no ASan runtime next to hipcc")
    env = dict(os.environ, LD_PRELOAD=rt, CSAHCA_LIBRARY=str(build.LIB_ASAN),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", str(ROOT / "tests" / "test_abi_cpu.py"), "-q",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    log = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, log
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, log
    assert " passed" in r.stdout, log
