"""Build libqsf_hip.so in-tree (gfx950) and the CPU parity checker.

    python -m qstream_amd.build          # or build() from __graft_entry__

* HIP translation units (csrc/*.hip) -> hipcc --offload-arch=gfx950
  (packed-fp32 VALU forms disabled, see HIP_FLAGS).
* C11 host layer (host/*.c) -> gcc -std=c11 against the HIP runtime C API.
* Linked into qstream_amd/libqsf_hip.so; nothing is installed.
* oracle/ (test infrastructure) -> `make -C oracle`.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
LIB = os.path.join(PKG, "libqsf_hip.so")
OBJ = os.path.join(PKG, "_build")
ARCH = os.environ.get("QSF_HIP_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(PKG, 'csrc')}", f"-I{os.path.join(ROOT, 'include')}",
]
C_FLAGS = [
    "-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
    "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{os.path.join(ROOT, 'include')}",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the device-only feature flag: drop that note
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build_oracle() -> None:
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])


def build_lib() -> str:
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    os.makedirs(OBJ, exist_ok=True)
    objs = []
    for src in sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip"))):
        o = os.path.join(OBJ, os.path.basename(src) + ".o")
        _run([hipcc, *HIP_FLAGS, "-c", src, "-o", o])
        objs.append(o)
    for src in sorted(glob.glob(os.path.join(PKG, "host", "*.c"))):
        o = os.path.join(OBJ, os.path.basename(src) + ".o")
        _run(["gcc", *C_FLAGS, "-c", src, "-o", o])
        objs.append(o)
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-L{ROCM}/lib", "-lamdhip64", "-lpthread", "-lm"])
    os.replace(tmp, LIB)
    return LIB


def build() -> str:
    build_oracle()
    return build_lib()


if __name__ == "__main__":
    print(build())
