"""Build libhsattn.so, the gfx950 paged-attention library, with hipcc.

Every ``csrc/*.hip`` file is compiled for gfx950 only (one code path, no
CUDA-compatibility layer) and linked into ``heteroserve/libhsattn.so`` next
to the Python package that loads it.  The objects go to ``_build/``.

    python hetero-serve_amd/build.py          # build (always recompiles)
    python hetero-serve_amd/build.py --check  # also dump the resource usage
    python hetero-serve_amd/build.py --sanitize   # also the host-sanitized copy

The sanitized copy (``_build/san/libhsattn_san.so``) is the same library with
the host code of the C-ABI layer (hs_api.hip: argument validation, grid and
workspace arithmetic) built with AddressSanitizer and UndefinedBehaviorSanitizer;
device code is unchanged.  It is for CPU tests only (tests/test_sanitized_abi.py
loads it with the ASan runtime preloaded); nothing on a GPU box loads it.

Packed fp32 VALU instructions are disabled for device code
(``-target-feature -packed-fp32-ops``): some of their forms have produced
silent wrong results on the MI355X boxes this library was brought up on.
hipcc's host pass reports the feature as unknown; that warning is harmless.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_PATH = ROOT / "heteroserve" / "libhsattn.so"
ARCH = "gfx950"


def hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source flags.  The MFMA prefill kernel holds more live state than the
# 256 architectural VGPRs; LLVM's default then keeps MFMA accumulators in
# VGPRs and spills other values to AGPRs, reloading them every loop
# iteration.  Forcing the VGPR form for MFMA operands cut the loop's
# instruction count by ~45% (measured on the generated gfx950 code).
PER_FILE_FLAGS = {
    "hs_prefill_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true",
                            "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
    "hs_decode_gqa.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
    "hs_decode_splitmm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def _compile(src: Path, extra: list[str]) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMPILE_FLAGS, *PER_FILE_FLAGS.get(src.name, []), *extra, "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(msgs))
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


SAN_DIR = BUILD_DIR / "san"
SAN_LIB = SAN_DIR / "libhsattn_san.so"
# host-only instrumentation: each sanitizer flag applies to the host pass
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined",
             "-Xarch_host", "-fno-omit-frame-pointer", "-g"]


def asan_runtime() -> Path:
    """clang's shared ASan runtime (it carries the UBSan handlers too)."""
    out = subprocess.run([hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True).stdout.strip()
    return Path(out)


def build_sanitized() -> Path:
    """hs_api.hip with host ASan + UBSan, linked with the other objects of a
    plain build (build() first) into _build/san/libhsattn_san.so."""
    SAN_DIR.mkdir(parents=True, exist_ok=True)
    src = CSRC / "hs_api.hip"
    obj = SAN_DIR / "hs_api.o"
    cmd = [hipcc(), *COMPILE_FLAGS, *SAN_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("sanitized hs_api.hip failed:\n" + res.stdout + res.stderr)
    others = [BUILD_DIR / (s.stem + ".o") for s in sorted(CSRC.glob("*.hip")) if s.name != src.name]
    missing = [str(o) for o in others if not o.exists()]
    if missing:
        raise RuntimeError(f"build() first: missing {missing}")
    rt = asan_runtime()
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(SAN_LIB), str(obj),
           *map(str, others), str(rt), f"-Wl,-rpath,{rt.parent}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("sanitized link failed:\n" + res.stdout + res.stderr)
    return SAN_LIB


def build(jobs: int | None = None, extra_flags: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libhsattn.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    extra = list(extra_flags or [])
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--check", action="store_true",
                    help="print per-kernel VGPR/SGPR/LDS/spill usage")
    ap.add_argument("--sanitize", action="store_true",
                    help="also build the host-sanitized copy for the CPU tests")
    args = ap.parse_args()
    extra = ["-Rpass-analysis=kernel-resource-usage"] if args.check else []
    path = build(args.jobs, extra)
    print(f"built {path} ({path.stat().st_size} bytes)")
    if args.sanitize:
        print(f"built {build_sanitized()}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
