"""The boundary from C.  tests/c_abi/caller.c compiles against include/hsattn.h
as C99 (-pedantic -Werror), links libhsattn.so and runs on a machine without
a GPU (version check, workspace queries, argument errors as status codes);
decode_gpu.c, prefill_gpu.c and pack_gpu.c run decode, chunked prefill and a
block migration on the GPU from C (the gpu-marked test)."""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CALLER = ROOT / "tests" / "c_abi" / "caller.c"
HEADER = ROOT / "include" / "hsattn.h"


def _declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text))


def test_caller_takes_every_entry_point():
    listed = set(re.findall(r"\(any_fn\)(hs_[a-z0-9_]+)", CALLER.read_text()))
    assert listed == _declared_functions()


def test_c_host_compiles_links_and_runs(tmp_path):
    from heteroserve import _hip

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    lib = _hip.lib_path()
    if not lib.exists():
        pytest.fail(f"{lib} missing: run python hetero-serve_amd/build.py")
    exe = tmp_path / "caller"
    subprocess.run([gcc, "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror",
                    f"-I{ROOT / 'include'}", str(CALLER), f"-L{lib.parent}", f"-l:{lib.name}",
                    f"-Wl,-rpath,{lib.parent}", "-o", str(exe)], check=True,
                   capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().splitlines()[-1] == "OK", run.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("program", ["decode_gpu", "prefill_gpu", "pack_gpu"])
def test_c_host_runs_on_the_gpu(program, tmp_path):
    """C hosts that allocate and copy with the HIP runtime's C API and call
    the library: decode_gpu.c runs hs_decode (default decomposition with its
    workspace, and one pass) against its own double-precision decode of the
    same data, 1e-5 (fp32 cache); prefill_gpu.c runs hs_prefill_varlen on
    two ragged chunks over a bf16 cache, matrix cores within 2e-3 and the
    fp32 row kernel within 1e-5 of its own double-precision prefill;
    pack_gpu.c packs scattered blocks of a 3-layer pool and unpacks them into
    another pool, byte for byte."""
    from heteroserve import _hip

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    rocm = Path("/opt/rocm")
    lib = _hip.lib_path()
    exe = tmp_path / program
    subprocess.run([gcc, "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror",
                    "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", "-isystem",
                    str(rocm / "include"), str(ROOT / "tests" / "c_abi" / f"{program}.c"),
                    f"-L{lib.parent}", f"-l:{lib.name}", f"-L{rocm / 'lib'}", "-lamdhip64", "-lm",
                    f"-Wl,-rpath,{lib.parent}", f"-Wl,-rpath,{rocm / 'lib'}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    print("running", exe.name, flush=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(run.stdout, flush=True)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().splitlines()[-1] == "OK", run.stdout
