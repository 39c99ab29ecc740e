"""Build libhdcmamba_hip.so in-tree for gfx950 with hipcc.

Usage:  python -m hdcmamba_amd.build        (or hdcmamba_amd.build.build())

Every csrc/*.hip file is compiled to an object under hdcmamba_amd/_build/ and the
objects are linked into hdcmamba_amd/libhdcmamba_hip.so, which is what
hdcmamba_amd._lib loads.  Packed-fp32 VALU ops are disabled for device code.
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
LIB = PKG / "libhdcmamba_hip.so"
ARCH = os.environ.get("HDCM_OFFLOAD_ARCH", "gfx950")

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-function", "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libhdcmamba_hip.so)")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the device-only target feature; drop that one warning.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops' is not a recognized" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [hipcc, *CFLAGS, "-I", str(PKG.parent / "include"), "-c", str(s), "-o", str(o)])
                for s, o in zip(srcs, objs)]
        for s, f in zip(srcs, futs):
            msg = f.result()
            if verbose and msg.strip():
                print(f"[{s.name}]\n{msg}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
