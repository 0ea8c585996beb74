"""The C-ABI layer's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/test_abi.py -- argument validation, the workspace and grid size
arithmetic at ordinary and extreme sizes, the module state -- runs in a
subprocess against _build/san/libhsattn_san.so: the same library with
hs_api.hip's host code built with -fsanitize=address,undefined (UBSan set
not to recover, so any finding fails the run).  Python itself is not
instrumented, so the ASan runtime is preloaded.  No GPU is involved; device
code is not instrumented.  The sanitized copy is built by
``python hetero-serve_amd/build.py --sanitize`` and by __graft_entry__.build().
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "hetero-serve_amd"))

import build as hs_build  # noqa: E402


def test_abi_suite_under_asan_and_ubsan():
    lib = hs_build.SAN_LIB
    if not lib.exists():
        pytest.fail(f"{lib} missing: run python hetero-serve_amd/build.py --sanitize")
    undefined = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True,
                               text=True).stdout
    assert "__asan_report" in undefined and "__ubsan_handle" in undefined, \
        "the sanitized library is not instrumented"
    env = dict(os.environ)
    env.update(LD_PRELOAD=str(hs_build.asan_runtime()),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               HETEROSERVE_HIP_LIB=str(lib))
    r = subprocess.run([sys.executable, "-m", "pytest", str(ROOT / "tests" / "test_abi.py"), "-q",
                        "-p", "no:cacheprovider"], capture_output=True, text=True, env=env,
                       cwd=str(ROOT), timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert " passed" in r.stdout
